"""Pins of oracle/chain_oracle.py (the vectorised depth-1 chain checker used at full size on the GPU) to
oracle/ews_oracle.py by independent routes, forward and autograd gradients, float64:
  - the exact leaf: one augmented matrix exponential per interval (ews_oracle.exact_local_terms, itself pinned against
    quadrature in tests/test_oracle_math.py), flows by torch.linalg.matrix_exp, the sequential Chen loop;
  - the series leaf of order q from its letters (ews_oracle.series_local_terms);
  - the Van Loan leaf with exact exponentials in the three reweighting modes (ews_oracle.van_loan_local_terms).
Real chains of 1-4 coordinates, complex chains of 1-4 complex coordinates (size 2: rotation planes), steps with
h |c| up to 6 (the recurrence branch of phi^(r)), prefix / terminal / mean / max readouts.
"""

import numpy as np
import pytest
import torch

from oracle import chain_oracle as CO
from oracle import ews_oracle as O

DT = torch.float64


def relerr(a, b):
    a, b = a.detach(), b.detach()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _chain_A(kind, size, params):
    """Block-diagonal A of uniform chains from per-chain (c or (a, b), eps) tensors: real lambda I + eps Nil;
    complex blocks [[a, -b], [b, a]] with eps times the 2x2 identity above them."""
    blocks = []
    for p in params:
        if kind == "real":
            lam, eps = p[0], p[1]
            blk = torch.diag(lam.expand(size))
            if size > 1:
                blk = blk + eps * torch.diag(torch.ones(size - 1, dtype=DT), 1)
        else:
            a, b, eps = p[0], p[1], p[2]
            R = torch.stack([torch.stack([a, -b]), torch.stack([b, a])])
            k = size // 2
            blk = torch.kron(torch.eye(k, dtype=DT), R)
            if k > 1:
                blk = blk + eps * torch.kron(torch.diag(torch.ones(k - 1, dtype=DT), 1), torch.eye(2, dtype=DT))
        blocks.append(blk)
    return torch.block_diag(*blocks)


def _case(kind, size, K, B, L, seed, scale=0.1):
    rng = np.random.default_rng(seed)
    d = size * K
    params = []
    for _ in range(K):
        if kind == "real":
            params.append(torch.tensor([rng.uniform(0.2, 2.0), rng.normal()], dtype=DT, requires_grad=True))
        else:
            params.append(torch.tensor([rng.uniform(0.2, 2.0), rng.normal() * 2.0, rng.normal()], dtype=DT,
                                       requires_grad=True))
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)), 1), dtype=DT, requires_grad=True)
    clock = torch.tensor(np.cumsum(rng.uniform(0.2, 1.0, size=(B, L)) * scale, 1), dtype=DT, requires_grad=True)
    return params, path, clock


def _grads(out, wts, tensors):
    (out * wts).sum().backward()
    g = [t.grad.clone() for t in tensors]
    for t in tensors:
        t.grad = None
    return g


CHAINS = [("real", 1), ("real", 2), ("real", 3), ("real", 4), ("complex", 2), ("complex", 4), ("complex", 6),
          ("complex", 8)]


@pytest.mark.parametrize("scale", [0.1, 2.0], ids=["small_steps", "large_steps"])
@pytest.mark.parametrize("kind,size", CHAINS)
def test_chain_checker_equals_exact_leaf(kind, size, scale):
    params, path, clock = _case(kind, size, 3, 2, 11, size * 7 + int(scale * 10), scale)
    tensors = [path, clock, *params]
    for readout in ("prefix", "terminal", "mean", "max"):
        A = _chain_A(kind, size, params)
        got = CO.chain_depth1(path, clock, A, kind, size, readout=readout)
        want = O.ews(path, clock, A, 1, readout, leaf="exact", chen_expm="exact")
        assert relerr(got, want) < 1e-12, (readout, relerr(got, want))
        w = torch.tensor(np.random.default_rng(3).normal(size=tuple(want.shape)), dtype=DT)
        g1 = _grads(got, w, tensors)
        A = _chain_A(kind, size, params)
        g2 = _grads(O.ews(path, clock, A, 1, readout, leaf="exact", chen_expm="exact"), w, tensors)
        for x, y in zip(g1, g2):
            assert relerr(x, y) < 1e-10, (readout, relerr(x, y))


@pytest.mark.parametrize("q", [1, 3, 8])
@pytest.mark.parametrize("kind,size", [("real", 3), ("complex", 4), ("complex", 2)])
def test_chain_checker_series_leaf(kind, size, q):
    params, path, clock = _case(kind, size, 2, 2, 9, q, 1.0)
    A = _chain_A(kind, size, params)
    got = CO.chain_depth1(path, clock, A, kind, size, series_q=q)
    want = O.ews(path, clock, A, 1, "prefix", leaf="series", series_q=q, chen_expm="exact")
    assert relerr(got, want) < 1e-12, relerr(got, want)
    # the truncation matters at these steps: the exact leaf differs
    exact = O.ews(path, clock, A, 1, "prefix", leaf="exact", chen_expm="exact")
    assert relerr(exact, want) > 1e-9  # far above the 1e-12 agreement with the series
    tensors = [path, clock, *params]
    w = torch.tensor(np.random.default_rng(4).normal(size=tuple(want.shape)), dtype=DT)
    g1 = _grads(got, w, tensors)
    A = _chain_A(kind, size, params)
    g2 = _grads(O.ews(path, clock, A, 1, "prefix", leaf="series", series_q=q, chen_expm="exact"), w, tensors)
    for x, y in zip(g1, g2):
        assert relerr(x, y) < 1e-10, relerr(x, y)


@pytest.mark.parametrize("mode", ["displacement", "displacement_uniform", "displacement_uniform_basepoint"])
@pytest.mark.parametrize("kind,size", [("real", 2), ("complex", 4), ("complex", 2)])
def test_chain_checker_van_loan_modes(kind, size, mode):
    params, path, clock = _case(kind, size, 2, 2, 10, 5, 0.5)
    A = _chain_A(kind, size, params)
    step = {"displacement": "per_interval", "displacement_uniform": "cached",
            "displacement_uniform_basepoint": "cached_basepoint"}[mode]
    got = CO.chain_depth1(path, clock, A, kind, size, flow_mode=step, leaf_mode=step)
    want = O.ews(path, clock, A, 1, "prefix", leaf="van_loan", M=4, van_loan_expm="exact", chen_expm="exact",
                 reweighting_mode=mode)
    assert relerr(got, want) < 1e-11, relerr(got, want)
    tensors = [path, clock, *params]
    w = torch.tensor(np.random.default_rng(6).normal(size=tuple(want.shape)), dtype=DT)
    g1 = _grads(got, w, tensors)
    A = _chain_A(kind, size, params)
    g2 = _grads(O.ews(path, clock, A, 1, "prefix", leaf="van_loan", M=4, van_loan_expm="exact", chen_expm="exact",
                      reweighting_mode=mode), w, tensors)
    for x, y in zip(g1, g2):
        assert relerr(x, y) < 1e-9, relerr(x, y)
