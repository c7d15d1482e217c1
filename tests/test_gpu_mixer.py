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
