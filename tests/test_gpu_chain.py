"""GPU parity of the depth-1 chain kernels (csrc/ews_chain.hip: a block-diagonal A of uniform chains, any number of
chains) against the float64 checker oracle/chain_oracle.py, itself pinned to oracle/ews_oracle.py's exact,
series and Van Loan leaves in tests/test_oracle_chain.py.

Bars: forward max relative error <= 1e-5, gradients <= 1e-4 (max|a-b| / max|b|).
  - the C-ABI op over every chain kind and size, chain counts 1 to 64 (not powers of two too), readouts prefix and
    terminal, flow and leaf step modes, the series leaf's order, large steps, zero clock steps, L = 2 and lengths
    that leave a partial chunk; gradients of path, clock and A (the chains' read entries);
  - the reference's banked depth-1 routes at their block shapes through the EWS layer:
      PPG (ppg_results/config.json: m = 64, 16 complex chains of size 4, jordan_closed, jordan_flows, a gated
      clock with closed gates; B = 8, L = 49,920), forward and the gradients of path, clock and the chain
      parameters;
      weather (weather_results/config.json: m = 64, 16 complex chains of size 4, the series leaf, exact flows,
      uniform time clock; B = 16, L = 720);
      rotation planes at m = 64 with the Van Loan leaf (M = 4, exact exponentials; the formal-language blocks,
      formal_language_results/even_pairs/config.json), every reweighting mode;
      the formal-language token block itself: build_token_cache at m = 64 (the chain kernels) and the depth-1
      cached scan (csrc/ews_token1.hip) against oracle/token_oracle.py, B = 256 sequences of 512 tokens.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from ews_mi355x import ops
from oracle import chain_oracle as CO

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _chain_A(kind, size, K, rng, damp=(0.1, 1.5), freq=3.0):
    """A float64 block-diagonal A of K uniform chains (reference sign: the flows are exp(-h A))."""
    d = size * K
    A = np.zeros((d, d))
    for j in range(K):
        f = size * j
        if kind == "real":
            lam, eps = rng.uniform(*damp), rng.normal()
            for i in range(size):
                A[f + i, f + i] = lam
                if i + 1 < size:
                    A[f + i, f + i + 1] = eps
        else:
            a, b, eps = rng.uniform(*damp), rng.uniform(-freq, freq), rng.normal()
            for i in range(size // 2):
                g = f + 2 * i
                A[g, g] = A[g + 1, g + 1] = a
                A[g, g + 1], A[g + 1, g] = -b, b
                if i + 1 < size // 2:
                    A[g, g + 2] = A[g + 1, g + 3] = eps
    return torch.tensor(A, dtype=DT)


def _run_case(kind, size, K, B, L, seed, readout="prefix", flow="per_interval", leaf="per_interval", q=0,
              step=0.05, zero_steps=False, level0=True):
    rng = np.random.default_rng(seed)
    d = size * K
    A = _chain_A(kind, size, K, rng)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1), dtype=torch.float32)
    steps = rng.uniform(0.2, 1.0, size=(B, L)) * step
    if zero_steps:
        steps[rng.uniform(size=(B, L)) < 0.3] = 0.0
    clock = torch.tensor(np.cumsum(steps, 1), dtype=torch.float32)
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    a = A.to(torch.float32).to(DEV).requires_grad_(True)
    out = ops.chain_scan(p, c, a, kind, size, flow, leaf, readout, level0, q)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ar = A.to(torch.float32).double().requires_grad_(True)
    ref = CO.chain_depth1(pr, cr, ar, kind, size, flow, leaf, readout, level0, q)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    w = torch.tensor(np.random.default_rng(seed + 1).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = dict(fwd=relerr(out, ref), dpath=relerr(p.grad, pr.grad), dclock=relerr(c.grad, cr.grad),
                dA=relerr(a.grad, ar.grad))
    print(f"chain {kind}{size} K={K} B={B} L={L} {readout} flow={flow} leaf={leaf} q={q}: "
          + ", ".join(f"{k} {v:.2e}" for k, v in errs.items()), flush=True)
    assert errs["fwd"] < 1e-5, errs
    assert max(errs["dpath"], errs["dclock"], errs["dA"]) < 1e-4, errs
    # only the chains' read entries carry a gradient
    mask = ar.grad != 0
    assert not (a.grad.detach().cpu() != 0)[~mask.cpu()].any()


SWEEP = [
    # kind, size, K, B, L
    ("real", 1, 5, 3, 100),
    ("real", 2, 3, 2, 70),
    ("real", 3, 7, 2, 130),
    ("real", 4, 16, 2, 65),
    ("complex", 2, 9, 3, 97),
    ("complex", 4, 16, 2, 200),
    ("complex", 6, 3, 2, 33),
    ("complex", 8, 8, 2, 64),
    ("real", 1, 64, 2, 40),      # 64 chains: one chunk per wavefront
    ("complex", 4, 1, 4, 300),   # one chain: 64 chunks per wavefront
]


@pytest.mark.parametrize("case", SWEEP, ids=[f"{c[0]}{c[1]}-K{c[2]}-L{c[4]}" for c in SWEEP])
def test_chain_kernels_match_checker(case):
    kind, size, K, B, L = case
    _run_case(kind, size, K, B, L, seed=K * 100 + L)


@pytest.mark.parametrize("readout", ["terminal", "prefix"])
@pytest.mark.parametrize("mode", ["cached", "cached_basepoint"])
def test_chain_step_modes(readout, mode):
    # flows and the Van Loan leaf on the shared step (van_loan.py:91-160), and flows alone on it (the other leaves)
    _run_case("complex", 4, 3, 2, 90, seed=7, readout=readout, flow=mode, leaf=mode)
    _run_case("real", 2, 4, 2, 90, seed=8, readout=readout, flow=mode, leaf="per_interval")


@pytest.mark.parametrize("q", [1, 4, 24, 48])
def test_chain_series_leaf(q):
    _run_case("complex", 4, 4, 2, 80, seed=q, q=q, step=0.5)
    _run_case("real", 3, 3, 2, 80, seed=q + 1, q=q, step=0.5)


def test_chain_large_and_zero_steps():
    # h |c| up to ~10 (the recurrence branch of phi^(r)), and closed gates (zero clock steps)
    _run_case("complex", 6, 3, 2, 120, seed=11, step=6.0)
    _run_case("real", 4, 3, 2, 120, seed=12, step=3.0, zero_steps=True)
    _run_case("complex", 4, 5, 2, 120, seed=13, zero_steps=True)


def test_chain_edge_lengths():
    _run_case("complex", 4, 2, 3, 2, seed=14)                      # one interval
    _run_case("complex", 2, 3, 2, 33, seed=15, readout="terminal")  # one full chunk and one step
    _run_case("real", 2, 2, 2, 50, seed=16, level0=False)


def _jordan_param(K, size, rng, damp_lo=0.005, damp_hi=0.5, freq=15.0):
    ps = [np.array([np.log(np.expm1(rng.uniform(damp_lo, damp_hi))), rng.uniform(-freq, freq)]) for _ in range(K)]
    gpu = E.AParamJordanRepeated([size] * K, ["complex"] * K, [torch.tensor(p, dtype=torch.float32) for p in ps])
    ref = E.AParamJordanRepeated([size] * K, ["complex"] * K, [torch.tensor(p, dtype=torch.float32).double()
                                                                 for p in ps])
    return gpu.to(DEV), ref


def _layer_check(layer_gpu, param_gpu, param_ref, path, clock, ref_fn, seed, tol_f=1e-5, tol_g=1e-4):
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer_gpu(p, c, readout="prefix")
    torch.cuda.synchronize()
    print(f"  GPU rows {tuple(out.shape)}", flush=True)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = ref_fn(pr, cr, param_ref())
    e = relerr(out, ref)
    w = torch.tensor(np.random.default_rng(seed).normal(size=tuple(ref.shape)) / np.sqrt(ref.shape[-1]))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = [relerr(p.grad, pr.grad), relerr(c.grad, cr.grad)]
    errs += [relerr(g.grad, h.grad) for g, h in zip(param_gpu.parameters(), param_ref.parameters())]
    print(f"  forward {e:.2e}, gradients (path, clock, parameters) {['%.2e' % x for x in errs]}", flush=True)
    assert e < tol_f, e
    assert max(errs) < tol_g, errs


def test_ppg_block_shape():
    """ppg_results/config.json: depth 1, m = 64 of 16 complex chains of size 4, leaf jordan_closed with jordan_flows,
    a clamped-gate clock (per-step increments, some gates closed); B = 8, L = 49,920."""
    B, L, K = 8, 49920, 16
    rng = np.random.default_rng(2025)
    gpu, ref = _jordan_param(K, 4, rng)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 4 * K)) / np.sqrt(L), 1), dtype=torch.float32)
    inc = np.clip(rng.normal(0.5, 0.6, size=(B, L)), 0.0, 1.0) * (2.0 / L)
    clock = torch.tensor(np.cumsum(inc, 1), dtype=torch.float32)
    layer = E.EWS(gpu, N=1, leaf="jordan_closed", combine="block_kernel", jordan_flows=True)
    print(f"ppg block B={B} L={L} K={K}", flush=True)
    _layer_check(layer, gpu, ref, path, clock, lambda p, c, A: CO.chain_depth1(p, c, A, "complex", 4), seed=1)


@pytest.mark.parametrize("q", [24, 48])
def test_weather_block_shape(q):
    """weather_results/config.json: depth 1, m = 64 of 16 complex chains of size 4, the series leaf (orders up to
    series_q_max = 48), exact flows, the time clock; B = 16, L = 720."""
    B, L, K = 16, 720, 16
    rng = np.random.default_rng(q)
    gpu, ref = _jordan_param(K, 4, rng, 0.2, 1.5, 1.8)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 4 * K)) * 0.05, 1), dtype=torch.float32)
    clock = torch.tensor(np.broadcast_to(np.arange(L, dtype=np.float64) / 24.0, (B, L)).copy(), dtype=torch.float32)
    layer = E.EWS(gpu, N=1, leaf="series", series_q=q, combine="block_kernel", chen_expm="exact")
    print(f"weather block B={B} L={L} K={K} q={q}", flush=True)
    _layer_check(layer, gpu, ref, path, clock,
                 lambda p, c, A: CO.chain_depth1(p, c, A, "complex", 4, series_q=q), seed=2)


@pytest.mark.parametrize("mode", ["displacement", "displacement_uniform", "displacement_uniform_basepoint"])
def test_wide_planes_van_loan(mode):
    """Rotation planes at m = 64 with the reference's default leaf (van_loan, M = 4, exact exponentials) at depth 1:
    the formal-language blocks' configuration (formal_language_results/even_pairs/config.json), every reweighting
    mode (flows and the leaf's step shared in the uniform modes)."""
    B, L, K = 64, 130, 32
    rng = np.random.default_rng(3)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    gpu = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0).to(DEV)
    ref = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 2 * K)) * 0.2, 1), dtype=torch.float32)
    clock = torch.tensor(np.broadcast_to(np.arange(L, dtype=np.float64) / 29.4837, (B, L)).copy(),
                         dtype=torch.float32)
    layer = E.EWS(gpu, N=1, leaf="van_loan", M=4, van_loan_expm="exact", chen_expm="exact", reweighting_mode=mode)
    step = {"displacement": "per_interval", "displacement_uniform": "cached",
            "displacement_uniform_basepoint": "cached_basepoint"}[mode]
    print(f"planes m={2 * K} van_loan {mode}", flush=True)
    _layer_check(layer, gpu, ref, path, clock,
                 lambda p, c, A: CO.chain_depth1(p, c, A, "complex", 2, step, step), seed=3)


@pytest.mark.parametrize("leaf", ["van_loan", "series"])
def test_formal_language_token_block(leaf):
    """formal_language_results/even_pairs/config.json: the token-cached block at depth 1, m = 64 rotation planes,
    Van Loan M = 4 with exact exponentials (and the series leaf); B = 256 sequences of 512 tokens, vocabulary 8,
    padded tails. build_token_cache (the chain kernels) then token_cached_prefix_scan (the depth-1 cached scan)
    against oracle/token_oracle.py (the cache from the oracle's Van Loan / series leaf and matrix_exp flows; the
    batched depth-1 scan pinned to the packed Chen loop): forward and the gradients of the token displacements,
    clock increments and plane parameters."""
    from oracle import token_oracle as TO

    B, n, V, K = 256, 512, 8, 32
    d = 2 * K
    rng = np.random.default_rng(77)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    gpu = E.AParamDampedRotation(v.clone(), u.clone(), d, omega_scale=2.0).to(DEV)
    ref = E.AParamDampedRotation(v.double(), u.double(), d, omega_scale=2.0)
    dx = torch.tensor(rng.normal(size=(V, d)) * 0.3, dtype=torch.float32)
    dth = torch.tensor(rng.uniform(0.05, 0.4, size=V), dtype=torch.float32)
    tok = torch.tensor(rng.integers(0, V, size=(B, n)), dtype=torch.int64)
    lens = rng.integers(n // 4, n + 1, size=B)
    mask = torch.tensor(np.arange(n)[None, :] < lens[:, None])
    q = 3 if leaf == "series" else None  # an order low enough that the truncation shows at these steps
    print(f"token block m={d} V={V} B={B} n={n} leaf={leaf}", flush=True)
    gx = dx.to(DEV).requires_grad_(True)
    gt = dth.to(DEV).requires_grad_(True)
    P, Dc = E.build_token_cache(gx, gt, gpu(), 4, 1, "exact", "exact", leaf, q)
    out = E.token_cached_prefix_scan(tok.to(DEV), mask.to(DEV), P, Dc, d, 1)
    rx = dx.double().requires_grad_(True)
    rt = dth.double().requires_grad_(True)
    Pr, Dr = TO.build_token_cache(rx, rt, ref(), 4, 1, "exact", "exact", leaf, q)
    want = TO.token_cached_prefix_scan_depth1(tok, mask, Pr, Dr)
    errs = dict(P=relerr(P, Pr), D=relerr(Dc, Dr), fwd=relerr(out, want))
    w = torch.tensor(rng.normal(size=tuple(want.shape)) / np.sqrt(d))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (want * w).sum().backward()
    errs.update(ddx=relerr(gx.grad, rx.grad), ddtheta=relerr(gt.grad, rt.grad))
    errs.update({f"dA_{i}": relerr(g.grad, h.grad) for i, (g, h) in enumerate(zip(gpu.parameters(),
                                                                               ref.parameters()))})
    print("  " + ", ".join(f"{k} {x:.2e}" for k, x in errs.items()), flush=True)
    assert max(errs["P"], errs["D"], errs["fwd"]) < 1e-5, errs
    assert max(x for k, x in errs.items() if k not in ("P", "D", "fwd")) < 1e-4, errs
    # the cache is block-diagonal (planes: blocks of 2), which the scan above exploited; the dense route on the same
    # caches (block=0: every flow entry read, the full dense token gradients) gives the same rows and gradients
    gx2 = dx.to(DEV).requires_grad_(True)
    gt2 = dth.to(DEV).requires_grad_(True)
    P2, D2 = E.build_token_cache(gx2, gt2, gpu(), 4, 1, "exact", "exact", leaf, q)
    assert getattr(D2, "_ews_block", 0) == 2
    out2 = E.token_cached_prefix_scan(tok.to(DEV), mask.to(DEV), P2, D2, d, 1, block=0)
    (out2 * w.to(DEV, torch.float32)).sum().backward()
    e2 = [relerr(out2, want), relerr(gx2.grad, rx.grad), relerr(gt2.grad, rt.grad)]
    print(f"  dense route: forward {e2[0]:.2e}, ddx {e2[1]:.2e}, ddtheta {e2[2]:.2e}", flush=True)
    assert e2[0] < 1e-5 and max(e2[1:]) < 1e-4, e2
