"""GPU parity of the fused mixer epilogue (csrc/ews_mixer.hip) against the float64 oracle (oracle/mixer_oracle.py,
pinned in tests/test_oracle_mixer.py to the reference's GradedRMSNorm tests).

Bars: forward max relative error <= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|
(the reference's tests/test_engines.py:31-33). Cases cover every GradedRMSNorm variant, the binomial prescale,
basepoint blocks (no leading zero row), depths 1-3, the widths of BASELINE.json configs[3] (d = 32) and [4]
(d = 24), more than 64 hidden columns (two workgroup column passes), level sizes that are not multiples of 16,
row counts above 256K (two row tiles per wavefront in the forward),
all-zero levels (the zero-safe RMS) and the chain scan -> epilogue with gradients to the path.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import ews_oracle as O
from oracle import mixer_oracle as MO

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _module(d, N, hidden, variant, prescale, basepoint, seed):
    rng = np.random.default_rng(seed)
    m = E.MixerEpilogue(d, N, hidden, graded_variant=variant, graded_eps=[1e-3 * (k + 1) for k in range(N)],
                        graded_prescale="binomial" if prescale else None, basepoint=basepoint)
    D = m.D
    with torch.no_grad():
        m.c_down.weight.copy_(torch.tensor(rng.normal(0.0, 1.0 / np.sqrt(D), size=(hidden, D))))
        m.c_down.bias.copy_(torch.tensor(rng.normal(0.0, 0.1, size=hidden)))
        if variant == "dilation":
            m.graded.lam.fill_(float(rng.uniform(0.6, 1.5)))
        else:
            m.graded.gains.copy_(torch.tensor(rng.uniform(0.5, 2.0, size=N)))
    return m.to(DEV)


def _rows(B, R, d, N, seed):
    rng = np.random.default_rng(seed + 1)
    D = sum(d**k for k in range(1, N + 1))
    x = rng.normal(size=(B, R, 1 + D))
    x[..., 0] = 1.0
    s = 1
    for k in range(1, N + 1):
        x[..., s: s + d**k] *= 0.3**k  # levels on different scales, as in a signature
        s += d**k
    x[0, min(3, R - 1), 1: 1 + d] = 0.0  # an all-zero level 1
    if N >= 2:
        x[-1, R // 2, 1 + d: 1 + d + d * d] = 0.0  # an all-zero level 2
    return torch.tensor(x, dtype=torch.float32)


CASES = [
    # d, N, hidden, variant, prescale, basepoint, B, R
    (3, 2, 5, "live_rms", False, False, 2, 37),
    (4, 3, 20, "live_rms", True, False, 2, 23),
    (16, 2, 64, "static_gain", False, True, 3, 50),
    (32, 2, 32, "live_rms", False, False, 2, 40),
    (24, 2, 24, "dilation", True, False, 2, 33),
    (16, 3, 70, "live_rms", False, False, 1, 19),
    (5, 1, 3, "static_gain", False, False, 2, 9),
    (7, 2, 17, "live_rms", True, True, 1, 64),
    # 256K rows and more: two row tiles per wavefront in the forward
    (3, 2, 5, "live_rms", True, False, 2, 140000),
    (2, 2, 40, "static_gain", False, True, 1, 270000),
    # c_down wider than 128: the backward's row-tile kernel instead of the column-tile one
    (3, 2, 150, "live_rms", True, False, 2, 45),
]


@pytest.mark.parametrize("case", CASES, ids=[f"d{c[0]}-N{c[1]}-h{c[2]}-{c[3]}-{'pre' if c[4] else 'nopre'}-"
                                             f"{'bp' if c[5] else 'zr'}" for c in CASES])
def test_epilogue_forward_and_grads_match_oracle(case):
    d, N, hidden, variant, prescale, basepoint, B, R = case
    m = _module(d, N, hidden, variant, prescale, basepoint, seed=d * 100 + N)
    x = _rows(B, R, d, N, seed=d + N)
    xg = x.to(DEV).requires_grad_(True)
    out = m(xg)
    assert out.shape == (B, R + (0 if basepoint else 1), hidden)
    # float64 oracle with the same parameters
    W = m.c_down.weight.detach().cpu().double().requires_grad_(True)
    b = m.c_down.bias.detach().cpu().double().requires_grad_(True)
    if variant == "dilation":
        lam = m.graded.lam.detach().cpu().double().requires_grad_(True)
        gains = None
    else:
        gains = m.graded.gains.detach().cpu().double().requires_grad_(True)
        lam = None
    xr = x.double().requires_grad_(True)
    ref = MO.mixer_epilogue(xr, W, b, d, N, variant, m.graded.eps, gains=gains, lam=lam, basepoint=basepoint,
                            prescale=prescale)
    e = relerr(out, ref)
    assert e < 1e-5, f"forward relerr {e:.2e}"
    w = torch.tensor(np.random.default_rng(5).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    ex = relerr(xg.grad, xr.grad)
    assert ex < 1e-4, f"row grad relerr {ex:.2e}"
    assert float(xg.grad[..., 0].abs().max()) == 0.0  # the level-0 column does not enter
    eW = relerr(m.c_down.weight.grad, W.grad)
    eb = relerr(m.c_down.bias.grad, b.grad)
    assert eW < 1e-4 and eb < 1e-4, (eW, eb)
    gg, rg = (m.graded.lam.grad, lam.grad) if variant == "dilation" else (m.graded.gains.grad, gains.grad)
    eg = relerr(gg, rg)
    assert eg < 1e-4, f"gain grad relerr {eg:.2e}"


def test_scan_then_epilogue_chain():
    """EWS prefix rows (rotation planes, d = 16, depth 2) into the epilogue, gradients to the path and to the
    generator parameters, against the oracle scan followed by the oracle epilogue."""
    B, L, K, N, hidden = 2, 130, 8, 2, 24
    rng = np.random.default_rng(13)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 2 * K)) * 0.2, 1), dtype=torch.float32)
    clock = torch.tensor(np.broadcast_to(np.linspace(0.0, 1.0, L), (B, L)).copy(), dtype=torch.float32)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    layer = E.EWS(E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0), N=N,
                  leaf="plane_closed").to(DEV)
    ref_param = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0)
    m = _module(2 * K, N, hidden, "live_rms", False, False, seed=77)
    p = path.to(DEV).requires_grad_(True)
    out = m(layer(p, clock.to(DEV), readout="prefix"))
    pr = path.double().requires_grad_(True)
    rows = O.ews(pr, clock.double(), ref_param(), N, "prefix", leaf="plane_closed", reweighting_mode="displacement",
                 terminal_reduce="assoc", chen_expm="exact")
    W = m.c_down.weight.detach().cpu().double()
    b = m.c_down.bias.detach().cpu().double()
    g = m.graded.gains.detach().cpu().double()
    ref = MO.mixer_epilogue(rows, W, b, 2 * K, N, "live_rms", m.graded.eps, gains=g)
    assert relerr(out, ref) < 1e-5, relerr(out, ref)
    w = torch.tensor(np.random.default_rng(6).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    assert relerr(p.grad, pr.grad) < 1e-4, relerr(p.grad, pr.grad)
    for g_gpu, g_ref in zip([q.grad for q in layer.A_param.parameters()], [q.grad for q in ref_param.parameters()]):
        assert relerr(g_gpu, g_ref) < 1e-4, relerr(g_gpu, g_ref)


# ------------------------------------------------------------------------------------------ scan + epilogue, fused
def _fused_case(structure, K, N, hidden, variant, prescale, basepoint, B, L, seed, uniform=True, bf16=False):
    """Inputs of the fused scan -> epilogue route: a diagonal or rotation-plane scan of (path, clock) and a mixer
    module; returns the GPU tensors (leaves with requires_grad) and the float64 CPU copies."""
    rng = np.random.default_rng(seed)
    d = 2 * K if structure == "planes" else K
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.2, 1), dtype=torch.float32)
    if uniform:
        clock = torch.tensor(np.broadcast_to(np.arange(L, dtype=np.float64) / L, (B, L)).copy(), dtype=torch.float32)
    else:
        clock = torch.tensor(np.cumsum(rng.uniform(0.5, 1.5, size=(B, L)) / L, 1), dtype=torch.float32)
    params = (torch.tensor(np.stack([rng.uniform(0.1, 1.0, K), rng.uniform(-3.0, 3.0, K)], -1), dtype=torch.float32)
              if structure == "planes" else torch.tensor(rng.uniform(0.1, 2.0, K), dtype=torch.float32))
    m = _module(d, N, hidden, variant, prescale, basepoint, seed=seed + 7)
    if bf16:
        path = path.to(torch.bfloat16).to(torch.float32)  # exactly representable in bfloat16
    return d, path, clock, params, m


def _grad_leaves(path, clock, params, m, bf16):
    p = (path.to(torch.bfloat16) if bf16 else path).to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    q = params.to(DEV).requires_grad_(True)
    for t in m.parameters():
        t.grad = None
    return p, c, q


FUSED_CASES = [
    # structure, K, N, hidden, variant, prescale, basepoint, B, L, uniform, bf16
    ("planes", 12, 2, 24, "live_rms", False, False, 2, 300, True, False),   # c5's width, the table-free chunks
    ("planes", 3, 2, 40, "static_gain", True, True, 3, 150, False, False),  # exact per-step coefficients
    ("planes", 12, 1, 24, "dilation", True, False, 2, 200, True, True),     # depth 1, bfloat16 path
    ("real_diag", 8, 2, 32, "live_rms", True, False, 2, 500, True, False),  # a real diagonal off the sequential kernels
    ("real_diag", 5, 2, 17, "live_rms", False, True, 2, 77, False, False),
    ("planes", 16, 2, 64, "live_rms", False, False, 1, 140, True, False),   # d = 32: 1,024-lane workgroups
]


@pytest.mark.parametrize("case", FUSED_CASES, ids=[f"{c[0]}-K{c[1]}-N{c[2]}-h{c[3]}-{c[4]}" for c in FUSED_CASES])
def test_fused_scan_epilogue_equals_composed(case):
    """ews_diag_mixer_forward (the scan's output pass with the epilogue in it; the rows never written) against the
    scan's prefix rows followed by ews_mixer_forward, forward and every gradient (path, clock, generator, c_down,
    gains), on the same GPU."""
    structure, K, N, hidden, variant, prescale, basepoint, B, L, uniform, bf16 = case
    d, path, clock, params, m = _fused_case(structure, K, N, hidden, variant, prescale, basepoint, B, L, 3 + K,
                                            uniform, bf16)
    outs, grads = [], []
    for fused in (True, False):
        p, c, q = _grad_leaves(path, clock, params, m, bf16)
        if fused:
            out = E.ops.scan_mixer(p, c, q, m.c_down.weight, m.c_down.bias, m.graded.gain_tensor(), N, structure,
                                   variant=variant, eps=m.graded.eps, prepend=not basepoint, prescale=prescale)
            assert out is not None, "the configuration should run on the chunk kernels"
        else:
            rows = E.ops.diag_scan(p, c, q, N, structure, "per_interval", "prefix", True)
            out = m(rows)
        w = torch.tensor(np.random.default_rng(5).normal(size=tuple(out.shape)), dtype=torch.float32, device=DEV)
        (out * w).sum().backward()
        outs.append(out.detach())
        grads.append([p.grad, c.grad, q.grad] + [t.grad.clone() for t in m.parameters()])
    e = relerr(outs[0], outs[1])
    errs = [relerr(a, b) for a, b in zip(grads[0], grads[1])]
    print(f"fused {structure} K={K} N={N} h={hidden} {variant}: forward {e:.2e}, gradients "
          f"{['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


def test_fused_scan_epilogue_matches_oracle():
    """The fused route at c5's width (12 planes, depth 2, 24 hidden) against the float64 oracle scan followed by the
    oracle epilogue, forward and gradients to the path, the plane parameters and c_down."""
    B, L, K, N, hidden = 2, 140, 12, 2, 24
    d, path, clock, params, m = _fused_case("planes", K, N, hidden, "live_rms", True, False, B, L, 31)
    p, c, q = _grad_leaves(path, clock, params, m, False)
    out = E.ops.scan_mixer(p, c, q, m.c_down.weight, m.c_down.bias, m.graded.gain_tensor(), N, "planes",
                           variant="live_rms", eps=m.graded.eps, prepend=True, prescale=True)
    pr = path.double().requires_grad_(True)
    qr = params.double().requires_grad_(True)
    dw = torch.stack([qr[:, 0], qr[:, 1]], -1)
    A = torch.zeros(d, d, dtype=DT)
    ii = torch.arange(0, d, 2)
    A = A.index_put((ii, ii), dw[:, 0]).index_put((ii + 1, ii + 1), dw[:, 0])
    A = A.index_put((ii, ii + 1), dw[:, 1]).index_put((ii + 1, ii), -dw[:, 1])
    rows = O.ews(pr, clock.double(), A, N, "prefix", leaf="plane_closed", reweighting_mode="displacement",
                 terminal_reduce="assoc", chen_expm="exact")
    W = m.c_down.weight.detach().cpu().double().requires_grad_(True)
    b = m.c_down.bias.detach().cpu().double()
    g = m.graded.gains.detach().cpu().double()
    ref = MO.mixer_epilogue(rows, W, b, d, N, "live_rms", m.graded.eps, gains=g, prescale=True)
    e = relerr(out, ref)
    w = torch.tensor(np.random.default_rng(6).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = [relerr(p.grad, pr.grad), relerr(q.grad, qr.grad), relerr(m.c_down.weight.grad, W.grad)]
    print(f"fused vs oracle: forward {e:.2e}, gradients {['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


def test_fused_scan_epilogue_c5_block():
    """BASELINE.json configs[4]'s block at its full shape (B = 8, L = 49,920, 12 planes, depth 2, bfloat16 path,
    24 hidden): the fused route against the composed one on the same GPU, forward and gradients."""
    B, L, K, N, hidden = 8, 49920, 12, 2, 24
    d, path, clock, params, m = _fused_case("planes", K, N, hidden, "live_rms", False, False, B, L, 41, True, True)
    print(f"c5 fused block B={B} L={L}", flush=True)
    outs, grads = [], []
    for fused in (True, False):
        p, c, q = _grad_leaves(path, clock, params, m, True)
        if fused:
            out = E.ops.scan_mixer(p, c, q, m.c_down.weight, m.c_down.bias, m.graded.gain_tensor(), N, "planes",
                                   variant="live_rms", eps=m.graded.eps)
        else:
            out = m(E.ops.diag_scan(p, c, q, N, "planes", "per_interval", "prefix", True))
        w = torch.tensor(np.random.default_rng(8).normal(size=tuple(out.shape)), dtype=torch.float32, device=DEV)
        (out * w).sum().backward()
        torch.cuda.synchronize()
        outs.append(out.detach().cpu())
        grads.append([x.detach().cpu() for x in [p.grad, c.grad, q.grad] + [t.grad for t in m.parameters()]])
    e = relerr(outs[0], outs[1])
    errs = [relerr(a, b) for a, b in zip(grads[0], grads[1])]
    print(f"  forward {e:.2e}, gradients {['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    # the path gradient comes back in the path's bfloat16: float32 values that differ by ~1e-6 may round one
    # bfloat16 unit (2^-8 relative) apart, so its bar is that unit; the float32 gradients keep 1e-4
    assert errs[0] < 2.0**-8, errs[0]
    assert max(errs[1:]) < 1e-4, errs
