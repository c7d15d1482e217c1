"""GPU parity of the exact-integral leaves, the Jordan-chain leaves (leaf="jordan_closed" / "jordan_closed_tables")
with jordan_flows and the block-series leaf on general blocks, against the float64 oracle's exact local integrals (its
series leaf at order 40 at small steps, and its augmented-exponential leaf at any step, both pinned against
quadrature in tests/test_oracle_*.py). The reference pins its closed forms the same way: tests/test_jordan_engine.py:
66-91 holds them to the series leaf (q = 24 at 1e-7, q = 60 at 1e-10).

Bars: forward max relative error <= 1e-5, gradients <= 1e-4 (metric max|a-b| / max|b|). Cases: real chains of 2-4
and complex chains of 4, 6, 8 (two blocks each), depths 1 and 2, prefix / terminal / mean readouts, with and
without jordan_flows, small steps, and steps with clock step x ||A||_1 from 5 to 60.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _params(kind, K, seed):
    rng = np.random.default_rng(seed)
    return [np.array([rng.normal(-1.5, 0.7)] if kind == "real"
                     else [rng.normal(-1.5, 0.7), rng.uniform(0.3, 1.5) * rng.choice([-1.0, 1.0])]) for _ in range(K)]


CASES = [("real", 2), ("real", 3), ("real", 4), ("complex", 4), ("complex", 6), ("complex", 8)]


@pytest.mark.parametrize("flows", [False, True])
@pytest.mark.parametrize("N", [1, 2])
@pytest.mark.parametrize("kind,size", CASES)
def test_jordan_leaf_matches_exact_integrals(kind, size, N, flows):
    K, B, L = 2, 2, 13
    d = size * K
    ps = _params(kind, K, size * 10 + N)
    A = E.AParamJordanRepeated([size] * K, [kind] * K, [torch.tensor(p, dtype=torch.float32) for p in ps]).to(DEV)
    Ar = E.AParamJordanRepeated([size] * K, [kind] * K, [torch.tensor(p, dtype=DT) for p in ps])
    rng = np.random.default_rng(size + N)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1), dtype=torch.float32)
    clock = torch.tensor(np.cumsum(rng.uniform(0.05, 0.15, size=(B, L)), 1), dtype=torch.float32)
    for leaf in ("jordan_closed", "jordan_closed_tables"):
        layer = E.EWS(A, N=N, leaf=leaf, combine="block_kernel", jordan_flows=flows,
                      chen_expm="cayley" if flows else "exact")
        for readout in ("prefix", "terminal", "mean"):
            p = path.to(DEV).requires_grad_(True)
            c = clock.to(DEV).requires_grad_(True)
            out = layer(p, c, readout=readout)
            pr = path.double().requires_grad_(True)
            cr = clock.double().requires_grad_(True)
            ref = O.ews(pr, cr, Ar(), N, readout, leaf="series", series_q=40, chen_expm="exact",
                        terminal_reduce="assoc")
            assert relerr(out, ref) < 1e-5, (leaf, readout, relerr(out, ref))
            w = torch.tensor(np.random.default_rng(1).normal(size=tuple(ref.shape)))
            (out * w.to(DEV, torch.float32)).sum().backward()
            (ref * w).sum().backward()
            assert relerr(p.grad, pr.grad) < 1e-4, (leaf, readout, relerr(p.grad, pr.grad))
            assert relerr(c.grad, cr.grad) < 1e-4, (leaf, readout, relerr(c.grad, cr.grad))
            for q, qr in zip(A.parameters(), Ar.parameters()):
                assert relerr(q.grad, qr.grad) < 1e-4, (leaf, readout, relerr(q.grad, qr.grad))
                q.grad = None
                qr.grad = None


@pytest.mark.parametrize("kind,size", CASES)
def test_jordan_leaf_at_large_steps(kind, size):
    """Clock steps with h ||A||_1 from 5 to 60, where a series of any practical order fails: the chains' tables are
    exact at any argument (jordan_engine.py:175-243). Forward and gradients (path, clock, the chain parameters)
    against the oracle's exact local terms (one augmented exponential per interval, pinned against graded
    quadrature in tests/test_oracle_math.py); two backward calls give identical gradients."""
    K, B, L = 2, 2, 9
    ps = _params(kind, K, 100 + size)
    A = E.AParamJordanRepeated([size] * K, [kind] * K, [torch.tensor(p, dtype=torch.float32) for p in ps]).to(DEV)
    Ar = E.AParamJordanRepeated([size] * K, [kind] * K, [torch.tensor(p, dtype=DT) for p in ps])
    norm = float(Ar().detach().abs().sum(0).max())
    rng = np.random.default_rng(size + 50)
    d = size * K
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)), 1), dtype=torch.float32)
    clock = torch.tensor(np.cumsum(rng.uniform(5.0, 60.0, size=(B, L)) / norm, 1), dtype=torch.float32)
    layer = E.EWS(A, N=2, leaf="jordan_closed_tables", combine="block_kernel", jordan_flows=True)
    grads = []
    for rep in range(2):
        p = path.to(DEV).requires_grad_(True)
        c = clock.to(DEV).requires_grad_(True)
        out = layer(p, c, readout="prefix")
        w = torch.tensor(np.random.default_rng(4).normal(size=tuple(out.shape)))
        (out * w.to(DEV, torch.float32)).sum().backward()
        grads.append([p.grad.clone(), c.grad.clone()] + [q.grad.clone() for q in A.parameters()])
        for q in A.parameters():
            q.grad = None
    for g0, g1 in zip(grads[0], grads[1]):
        assert torch.equal(g0, g1)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = O.ews(pr, cr, Ar(), 2, "prefix", leaf="exact", chen_expm="exact")
    (ref * w).sum().backward()
    e = relerr(out, ref)
    errs = [relerr(grads[0][0], pr.grad), relerr(grads[0][1], cr.grad)]
    errs += [relerr(q, qr.grad) for q, qr in zip(grads[0][2:], Ar.parameters())]
    print(f"{kind} {size} at h||A|| 5-60: forward {e:.2e}, gradients {errs}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


@pytest.mark.parametrize("N", [1, 2])
@pytest.mark.parametrize("sizes", [(2, 2, 2), (2, 3, 1), (4, 4), (3, 4)])
def test_block_series_leaf_on_general_blocks(N, sizes):
    """leaf="block_series" on block-diagonal generators that are neither planes nor diagonals (the cases of the
    reference's tests/test_engines.py:240-248, which hold the leaf to the series leaf at q = 24 within 1e-7)."""
    B, L = 2, 11
    rng = np.random.default_rng(sum(sizes) * 10 + N)
    blocks = []
    for n in sizes:
        S = rng.normal(size=(n, n)) * 0.4
        blocks.append(np.diag(rng.uniform(0.2, 1.0, n)) + (S - S.T) / 2 + 0.1 * rng.normal(size=(n, n)))
    A = E.AParamBlockDiag([torch.tensor(b, dtype=torch.float32) for b in blocks], sizes).to(DEV)
    Ar = E.AParamBlockDiag([torch.tensor(b, dtype=DT) for b in blocks], sizes)
    d = sum(sizes)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1), dtype=torch.float32)
    clock = torch.tensor(np.cumsum(rng.uniform(0.05, 0.2, size=(B, L)), 1), dtype=torch.float32)
    layer = E.EWS(A, N=N, leaf="block_series", series_q=24 if N == 2 else None)
    for readout in ("prefix", "terminal"):
        p = path.to(DEV).requires_grad_(True)
        out = layer(p, clock.to(DEV), readout=readout)
        pr = path.double().requires_grad_(True)
        ref = O.ews(pr, clock.double(), Ar(), N, readout, leaf="series", series_q=40, chen_expm="exact",
                    terminal_reduce="assoc")
        assert relerr(out, ref) < 1e-5, (readout, relerr(out, ref))
        w = torch.tensor(np.random.default_rng(2).normal(size=tuple(ref.shape)))
        (out * w.to(DEV, torch.float32)).sum().backward()
        (ref * w).sum().backward()
        assert relerr(p.grad, pr.grad) < 1e-4, (readout, relerr(p.grad, pr.grad))
        for q, qr in zip(A.parameters(), Ar.parameters()):
            assert relerr(q.grad, qr.grad) < 1e-4, (readout, relerr(q.grad, qr.grad))
            q.grad = None
            qr.grad = None


@pytest.mark.parametrize("scheme", ["cayley", "euler", "pade"])
def test_plane_closed_leaf_with_approximate_flows(scheme):
    """leaf="plane_closed" with chen_expm other than "exact": the closed-form local terms with the scheme's flows
    (ews/layer.py:172-265), on the dense kernels, against the oracle's plane closed forms and the same scheme."""
    K, B, L = 4, 2, 40
    rng = np.random.default_rng(11)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    A = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0).to(DEV)
    Ar = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 2 * K)) * 0.3, 1), dtype=torch.float32)
    clock = torch.tensor(np.cumsum(rng.uniform(0.01, 0.05, size=(B, L)), 1), dtype=torch.float32)
    layer = E.EWS(A, N=2, leaf="plane_closed", chen_expm=scheme)
    p = path.to(DEV).requires_grad_(True)
    out = layer(p, clock.to(DEV), readout="prefix")
    pr = path.double().requires_grad_(True)
    ref = O.ews(pr, clock.double(), Ar(), 2, "prefix", leaf="plane_closed", chen_expm=scheme)
    assert relerr(out, ref) < 1e-5, relerr(out, ref)
    w = torch.tensor(np.random.default_rng(3).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    assert relerr(p.grad, pr.grad) < 1e-4, relerr(p.grad, pr.grad)
