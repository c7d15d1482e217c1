"""GPU parity of the per-sample sequential kernels (real diagonal, depth 2, d <= 32): the flat prefix rows and the
LogEWS prefix rows written straight from the scan, forward and gradients (path, clock, diagonal), against the float64
oracle (ews/layer.py:154-265 and 488-517 restated in oracle/ews_oracle.py, pinned in tests/test_oracle_*.py).

Cases cover d = 32 (1,024 lanes per sample), narrow and odd widths (idle lanes, a padded pair row), lengths with a
partial last checkpoint block and an exact multiple of it, the three clock modes (every step equal: one set of
coefficients; equal to float32 rounding: first-order models; irregular: exact per-step coefficients), a bfloat16 path, the series leaf, and the c4 block at its full
shape (B = 256, L = 512, d = 32) through the LogEWS layer, where the default plan picks these kernels. Bars: forward
<= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|.
"""

import numpy as np
import pytest
import torch

import bench
import ews_mi355x as E
from ews_mi355x import _native as nat
from ews_mi355x import ops
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
SEQ = nat.CHUNK_SEQUENTIAL


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _data(B, L, K, seed, clock):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, K)) / np.sqrt(K), 1).astype(np.float32)
    if clock == "unit":  # every step exactly 1: one set of coefficients
        th = np.broadcast_to(np.arange(L, dtype=np.float32), (B, L)).copy()
    elif clock == "frac":  # k / L in float32: steps equal to rounding, first-order coefficient models
        th = np.broadcast_to((np.arange(L) / L).astype(np.float32), (B, L)).copy()
    else:
        th = np.cumsum(rng.uniform(0.3, 1.5, size=(B, L)), 1).astype(np.float32)
    lam = rng.uniform(0.1, 2.0, size=K).astype(np.float32)
    return path, th, lam


def _oracle(path, th, lam, log, leaf="diag_closed", **kw):
    A = torch.diag(lam)
    if log:
        return torch.stack([O.log_ews_single(path[b], th[b], A, 2, "prefix", leaf=leaf, **kw)
                            for b in range(path.shape[0])])
    return O.ews(path, th, A, 2, "prefix", leaf=leaf, **kw)


CASES = [
    # K, L, clock, log
    (32, 100, "unit", False),
    (32, 100, "unit", True),
    (32, 65, "irregular", True),   # 64 steps: whole checkpoint blocks
    (16, 120, "frac", False),
    (32, 90, "frac", True),
    (8, 150, "irregular", False),
    (5, 70, "unit", True),         # odd width: a padded pair row
    (7, 33, "irregular", False),
    (1, 40, "unit", False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"K{c[0]}-L{c[1]}-{c[2]}-{'log' if c[3] else 'rows'}" for c in CASES])
def test_sequential_matches_oracle(case):
    K, L, clk, log = case
    B = 3
    path, th, lam = _data(B, L, K, 100 + K + L, clk)
    print(f"sequential K={K} L={L} {clk} {'log' if log else 'rows'}", flush=True)
    p = torch.tensor(path, device=DEV).requires_grad_(True)
    c = torch.tensor(th, device=DEV).requires_grad_(True)
    lg = torch.tensor(lam, device=DEV).requires_grad_(True)
    out = ops.diag_scan(p, c, lg, 2, "real_diag", "per_interval", "log_prefix" if log else "prefix", True,
                        chunk=SEQ)
    pr = torch.tensor(path, dtype=torch.float64, requires_grad=True)
    cr = torch.tensor(th, dtype=torch.float64, requires_grad=True)
    lr = torch.tensor(lam, dtype=torch.float64, requires_grad=True)
    ref = _oracle(pr, cr, lr, log)
    assert out.shape == ref.shape, (out.shape, ref.shape)
    e = relerr(out, ref)
    w = torch.tensor(np.random.default_rng(K * L).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = (relerr(p.grad, pr.grad), relerr(c.grad, cr.grad), relerr(lg.grad, lr.grad))
    print(f"  forward {e:.2e}, gradients {errs}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


def test_sequential_equals_chunked_rows():
    """The sequential and the chunk kernels give the same prefix rows and gradients (to float32 rounding), with and
    without the clock gradient."""
    K, B, L = 32, 4, 300
    path, th, lam = _data(B, L, K, 7, "unit")
    outs, grads = [], []
    for chunk in (SEQ, 16):
        for clock_grad in (True, False):
            p = torch.tensor(path, device=DEV).requires_grad_(True)
            c = torch.tensor(th, device=DEV).requires_grad_(clock_grad)
            lg = torch.tensor(lam, device=DEV).requires_grad_(True)
            o = ops.diag_scan(p, c, lg, 2, "real_diag", "per_interval", "prefix", True, chunk=chunk)
            g = torch.tensor(np.random.default_rng(3).normal(size=tuple(o.shape)), dtype=torch.float32, device=DEV)
            (o * g).sum().backward()
            outs.append(o.detach())
            grads.append((p.grad, c.grad, lg.grad))
    e = relerr(outs[0], outs[2])
    print(f"sequential vs chunked rows: {e:.2e}", flush=True)
    assert e < 1e-5
    for i in (0, 1):
        errs = [relerr(a, b) for a, b in zip(grads[i], grads[2 + i]) if a is not None]
        print(f"  gradients (clock grad {i == 0}): {errs}", flush=True)
        assert max(errs) < 1e-4, errs
    assert grads[1][1] is None


def test_sequential_bf16_and_series_leaf():
    K, B, L = 12, 2, 90
    path, th, lam = _data(B, L, K, 11, "unit")
    pb = torch.tensor(path).to(torch.bfloat16)
    out = ops.diag_scan(pb.to(DEV), torch.tensor(th, device=DEV), torch.tensor(lam, device=DEV), 2, "real_diag",
                        "per_interval", "log_prefix", True, chunk=SEQ)
    ref = _oracle(pb.double(), torch.tensor(th, dtype=torch.float64), torch.tensor(lam, dtype=torch.float64), True)
    e = relerr(out, ref)
    print(f"bf16 log rows: {e:.2e}", flush=True)
    assert e < 1e-5
    # the order-3 series leaf at unit steps (lambda h up to 2: the truncation is far above float32 resolution)
    p = torch.tensor(path, device=DEV).requires_grad_(True)
    lg = torch.tensor(lam, device=DEV).requires_grad_(True)
    out = ops.diag_scan(p, torch.tensor(th, device=DEV), lg, 2, "real_diag", "per_interval", "prefix", True,
                        chunk=SEQ, leaf="series", series_q=3)
    pr = torch.tensor(path, dtype=torch.float64, requires_grad=True)
    lr = torch.tensor(lam, dtype=torch.float64, requires_grad=True)
    ref = _oracle(pr, torch.tensor(th, dtype=torch.float64), lr, False, leaf="series", series_q=3,
                  terminal_reduce="tree", chen_expm="exact")
    exact = _oracle(pr.detach(), torch.tensor(th, dtype=torch.float64), lr.detach(), False)
    w = torch.tensor(np.random.default_rng(4).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    e, e_exact = relerr(out, ref), relerr(exact, ref)
    errs = (relerr(p.grad, pr.grad), relerr(lg.grad, lr.grad))
    print(f"series q=3 rows: {e:.2e} (closed forms {e_exact:.2e}), gradients {errs}", flush=True)
    assert e < 1e-5 and e_exact > 1e-4
    assert max(errs) < 1e-4, errs


def test_c4_full_shape_log_layer():
    """The c4 block at B = 256, L = 512, d = 32 through the LogEWS layer (the default plan takes the sequential
    kernels and the fused log rows): samples 0-1 against the float64 oracle (forward and path gradients), and the
    whole batch against the chunk kernels followed by the separate log readout (forward, path and A gradients)."""
    path, clock, lam = bench.c4_inputs()
    B, L, d = path.shape
    assert (B, L, d) == (256, 512, 32)
    Ag = E.AParamEFM(torch.log(torch.expm1(torch.tensor(lam, dtype=torch.float32)))).to(DEV)
    assert torch.allclose(Ag().diagonal().cpu(), torch.tensor(lam), rtol=1e-5)
    # a real diagonal reaches the diagonal kernels through the series leaf; at order 40 and lambda h <= 2 its
    # truncation (below 1e-20) is invisible, so the closed forms are the reference here
    layer = E.LogEWS(Ag, N=2, leaf="series", series_q=40)
    p = torch.tensor(path, device=DEV).requires_grad_(True)
    c = torch.tensor(clock, device=DEV)
    print("c4 full shape through LogEWS", flush=True)
    got = layer(p, c, readout="prefix")
    g = torch.tensor(np.random.default_rng(8).normal(size=tuple(got.shape)), dtype=torch.float32, device=DEV)
    (got * g).sum().backward()
    gA = [q.grad.clone() for q in Ag.parameters()]
    # the chunk kernels, then the separate log readout, on the same inputs
    p2 = torch.tensor(path, device=DEV).requires_grad_(True)
    lam_t = Ag().diagonal().detach().clone().requires_grad_(True)
    rows = ops.diag_scan(p2, c, lam_t, 2, "real_diag", "per_interval", "prefix", True, chunk=16)
    alt = ops.log_rows(rows, d, 2, True, "prefix")
    (alt * g).sum().backward()
    e_fwd, e_dp = relerr(got, alt), relerr(p.grad, p2.grad)
    # the layer's parameter gradient through A = diag(softplus(theta)): chain the chunked dlambda the same way
    theta = [q for q in Ag.parameters()][0]
    dth = lam_t.grad * torch.sigmoid(theta.detach())
    e_dA = relerr(gA[0], dth)
    print(f"c4 sequential vs chunked: fwd {e_fwd:.2e} dpath {e_dp:.2e} dA {e_dA:.2e}", flush=True)
    assert e_fwd < 1e-5 and e_dp < 1e-4 and e_dA < 1e-4
    # two samples against the float64 oracle
    pr = torch.tensor(path[:2], dtype=torch.float64, requires_grad=True)
    ref = _oracle(pr, torch.tensor(clock[:2], dtype=torch.float64), Ag().diagonal().detach().double().cpu(), True)
    (ref * g[:2].double().cpu()).sum().backward()
    e, e_g = relerr(got[:2], ref), relerr(p.grad[:2], pr.grad)
    print(f"c4 samples 0-1 vs oracle: fwd {e:.2e} dpath {e_g:.2e}", flush=True)
    assert e < 1e-5 and e_g < 1e-4
