"""The series leaves on rotation planes and real diagonals at low order: the GPU layer computes the order-q
truncated series the reference computes (ews/core/leaf.py:99-175; series_leaf.py:8-25; blockdiag_engine.py:88-155),
not the closed forms.

Unit clock steps (the block default clock) put ||A|| h near 1-3, where an order-6 series differs from the exact
integrals by far more than float32 resolution. Each case checks the GPU layer against the float64 oracle at the
same q (oracle.series_local_terms / block_series_local_terms, pinned to the truncated defining integral in
tests/test_oracle_math.py), forward and gradients (path, clock, generator parameters), and checks that the
exact closed forms would have failed the same bar. Bars: forward <= 1e-5, gradients <= 1e-4 (max|a-b| / max|b|).
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _params(structure, K, seed, leaf="series"):
    rng = np.random.default_rng(seed)
    if structure == "real" and leaf == "block_series":
        # the block-series leaf needs a block-diagonal parametrisation (ews/core/kernels/combine.py:37-58): 1x1
        # blocks
        lam = rng.uniform(0.1, 2.0, size=K)
        gpu = E.AParamBlockDiag([torch.tensor([[x]], dtype=torch.float32) for x in lam], [1] * K).to(DEV)
        ref = E.AParamBlockDiag([torch.tensor([[x]], dtype=torch.float64) for x in lam], [1] * K)
        return gpu, ref, "diag_closed", K
    if structure == "planes":
        v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
        u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
        gpu = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=2.0).to(DEV)
        ref = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=2.0)
        return gpu, ref, "plane_closed", 2 * K
    th = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    return E.AParamEFM(th.clone()).to(DEV), E.AParamEFM(th.double()), "diag_closed", K


CASES = [
    # structure, K, leaf, q, N, L, clock
    ("planes", 4, "series", 6, 2, 130, "unit"),
    ("planes", 4, "block_series", 6, 2, 130, "unit"),
    ("planes", 8, "series", 3, 2, 200, "unit"),       # d = 16: the pair-group kernels stand aside for the series
    ("planes", 3, "series", 5, 1, 90, "unit"),
    ("real", 6, "series", 3, 2, 130, "unit"),
    ("real", 6, "block_series", 4, 2, 130, "unit"),
    ("real", 5, "series", 8, 2, 150, "irregular"),    # exact per-step coefficients
    ("planes", 3, "block_series", 2, 2, 150, "irregular"),
]


@pytest.mark.parametrize("case", CASES, ids=[f"{c[0]}-K{c[1]}-{c[2]}-q{c[3]}-N{c[4]}-{c[6]}" for c in CASES])
@pytest.mark.parametrize("readout", ["prefix", "terminal"])
def test_low_order_series_leaf(case, readout):
    structure, K, leaf, q, N, L, clk = case
    gpu, ref, closed_leaf, d = _params(structure, K, 17 + K + q, leaf)
    B = 2
    rng = np.random.default_rng(q * 10 + K)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1), dtype=torch.float32)
    if clk == "unit":
        clock = torch.arange(L, dtype=torch.float32).expand(B, L).contiguous()
    else:
        clock = torch.tensor(np.cumsum(rng.uniform(0.3, 1.5, size=(B, L)), 1), dtype=torch.float32)
    layer = E.EWS(gpu, N=N, leaf=leaf, series_q=q, combine="block_kernel" if structure == "planes" else "assoc")
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer(p, c, readout=readout)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    A = ref()
    want = O.ews(pr, cr, A, N, readout, leaf=leaf, series_q=q, terminal_reduce="tree", chen_expm="exact")
    e = relerr(out, want)
    exact = O.ews(path.double(), clock.double(), A.detach(), N, readout, leaf=closed_leaf, terminal_reduce="tree")
    e_closed = relerr(exact, want)
    print(f"{case} {readout}: forward relerr {e:.2e} (closed forms: {e_closed:.2e})", flush=True)
    assert e < 1e-5, e
    assert e_closed > 1e-4, e_closed  # the truncation is visible: the closed forms would not pass
    w = torch.tensor(np.random.default_rng(5).normal(size=tuple(want.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (want * w).sum().backward()
    errs = [relerr(p.grad, pr.grad), relerr(c.grad, cr.grad)]
    errs += [relerr(a.grad, b.grad) for a, b in zip(gpu.parameters(), ref.parameters())]
    print(f"  gradient relerrs {errs}", flush=True)
    assert max(errs) < 1e-4, errs
