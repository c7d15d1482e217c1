"""GPU parity of the block-series leaf on general block-diagonal generators (ews/core/leaf.py:138-175,
ews/core/kernels/blockdiag_engine.py:88-155): the exact level 1 G v, G = phi(-h A), at any clock step, and the
order-q series at level 2, on the dense kernels, forward and path / clock / A gradients, against the float64 oracle
(oracle/ews_oracle.py block_series_local_terms: the augmented matrix exponential for level 1, pinned in
tests/test_oracle_math.py). Bars: forward <= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|.

Level 1 alone (depth 1) runs at clock step x ||A||_1 from 5 to 60, where the scaled Taylor polynomial needs up to six
doublings; depth 2 runs at a low order (q = 6) where the truncation of level 2 is far above float32 resolution (the
oracle's q = 6 and its exact level 2 differ by more than 1e-4), so that the test fixes the order the kernels use.
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
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _blocks(sizes, seed):
    rng = np.random.default_rng(seed)
    out = []
    for n in sizes:
        S = rng.normal(size=(n, n)) * 0.6
        out.append(np.diag(rng.uniform(0.2, 1.0, n)) + (S - S.T) / 2 + 0.2 * rng.normal(size=(n, n)))
    return out


def _case(sizes, seed, B, L, step_norm):
    """Block generator, path and a clock whose steps h satisfy h ||A||_1 in step_norm (a (lo, hi) range)."""
    blocks = _blocks(sizes, seed)
    A = E.AParamBlockDiag([torch.tensor(b, dtype=torch.float32) for b in blocks], sizes).to(DEV)
    Ar = E.AParamBlockDiag([torch.tensor(b, dtype=DT) for b in blocks], sizes)
    anorm = float(Ar().abs().sum(0).max())
    rng = np.random.default_rng(seed + 1)
    d = sum(sizes)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1), dtype=torch.float32)
    steps = rng.uniform(step_norm[0], step_norm[1], size=(B, L)) / anorm
    clock = torch.tensor(np.cumsum(steps, 1), dtype=torch.float32)
    return A, Ar, path, clock


def _run(A, Ar, path, clock, N, q, readout="prefix", chen_expm="exact"):
    layer = E.EWS(A, N=N, leaf="block_series", series_q=q, chen_expm=chen_expm)
    p = path.to(DEV).requires_grad_(True)
    c = clock.to(DEV).requires_grad_(True)
    out = layer(p, c, readout=readout)
    pr = path.double().requires_grad_(True)
    cr = clock.double().requires_grad_(True)
    ref = O.ews(pr, cr, Ar(), N, readout, leaf="block_series", series_q=q, chen_expm=chen_expm,
                terminal_reduce="assoc")
    w = torch.tensor(np.random.default_rng(7).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = [relerr(p.grad, pr.grad), relerr(c.grad, cr.grad)]
    errs += [relerr(g.grad, gr.grad) for g, gr in zip(A.parameters(), Ar.parameters())]
    grads = [p.grad.clone(), c.grad.clone()] + [g.grad.clone() for g in A.parameters()]
    for g in A.parameters():
        g.grad = None
    return out, ref, errs, grads


@pytest.mark.parametrize("sizes", [(2, 3, 1), (4, 4), (3, 4, 5)])
def test_level1_exact_at_large_steps(sizes):
    A, Ar, path, clock = _case(sizes, sum(sizes), 2, 40, (5.0, 60.0))
    print(f"block series depth 1 sizes {sizes} at h||A||_1 5-60", flush=True)
    out, ref, errs, g1 = _run(A, Ar, path, clock, 1, None)
    e = relerr(out, ref)
    print(f"  forward {e:.2e}, gradients {['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs
    # the same call again: bit-identical gradients (fixed-order reductions)
    _, _, _, g2 = _run(A, Ar, path, clock, 1, None)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("sizes,readout", [((2, 3, 1), "prefix"), ((4, 4), "terminal"), ((3, 4), "mean")])
def test_depth2_low_order(sizes, readout):
    A, Ar, path, clock = _case(sizes, 3 * sum(sizes), 2, 30, (1.0, 3.0))
    print(f"block series depth 2 q=6 sizes {sizes} {readout}", flush=True)
    out, ref, errs, _ = _run(A, Ar, path, clock, 2, 6, readout)
    exact = O.ews(path.double(), clock.double(), Ar().detach(), 2, readout, leaf="exact", chen_expm="exact",
                  terminal_reduce="assoc")
    e, e_trunc = relerr(out, ref), relerr(exact, ref)
    print(f"  forward {e:.2e} (order-6 vs exact: {e_trunc:.2e}), gradients {['%.2e' % x for x in errs]}",
          flush=True)
    assert e_trunc > 1e-4
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs


def test_approximate_flows_on_planes():
    """block_series on rotation planes with chen_expm="cayley" (the dense route): exact level 1, order-8 level 2,
    Cayley flows, against the oracle."""
    K, B, L = 3, 2, 35
    rng = np.random.default_rng(21)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    A = E.AParamDampedRotation(v.clone(), u.clone(), 2 * K, omega_scale=3.0).to(DEV)
    Ar = E.AParamDampedRotation(v.double(), u.double(), 2 * K, omega_scale=3.0)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, 2 * K)) * 0.3, 1), dtype=torch.float32)
    clock = torch.tensor(np.cumsum(rng.uniform(0.2, 0.6, size=(B, L)), 1), dtype=torch.float32)
    out, ref, errs, _ = _run(A, Ar, path, clock, 2, 8, "prefix", chen_expm="cayley")
    e = relerr(out, ref)
    print(f"planes cayley: forward {e:.2e}, gradients {['%.2e' % x for x in errs]}", flush=True)
    assert e < 1e-5, e
    assert max(errs) < 1e-4, errs
