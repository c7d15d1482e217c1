"""GPU parity of the token-cached scan (csrc/ews_dense.hip: ews_token_scan, ews_token_scan_backward,
ews_dense_local_terms_backward) against the float64 oracle (oracle/token_oracle.py, pinned in
tests/test_oracle_token.py to the ordinary EWS scan, the reference's own claim for this path).

Bars: forward max relative error <= 1e-5, gradients <= 1e-4 (metric max|a-b| / max|b|,
the reference's tests/test_engines.py:31-33). Cases: depths 1-3, d from 2 to 16, one and several chunks, masks
with different lengths per sample, vocabularies of 1, 5, 40 and 128 tokens (up to eight groups of the gradient's
token accumulators; 128 is the vocabulary of the reference's set task, experiments/fl/tasks/set.py), more than 1024 steps (several gradient chunks), the Van Loan and series leaves of the cache, and the
chain build_token_cache -> token_cached_prefix_scan against the ordinary dense EWS layer on the expanded path.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import ews_oracle as O
from oracle import token_oracle as TO

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _cache(V, d, N, seed):
    rng = np.random.default_rng(seed)
    D = sum(d**k for k in range(1, N + 1))
    P = rng.normal(size=(V, D)) * 0.3
    S = rng.normal(size=(V, d, d)) * 0.2
    Dc = np.eye(d)[None] * rng.uniform(0.6, 0.95, size=(V, 1, 1)) + (S - S.transpose(0, 2, 1)) / 2
    return torch.tensor(P), torch.tensor(Dc)


SCANS = [
    # V, d, N, B, n, mask lengths
    (5, 4, 2, 3, 300, (300, 177, 1)),
    (1, 3, 3, 2, 70, None),
    (40, 2, 2, 2, 150, (150, 90)),
    (5, 16, 2, 2, 130, (130, 64)),
    (3, 6, 1, 2, 1500, (1500, 1100)),
    (7, 8, 3, 1, 80, None),
    (128, 8, 2, 2, 700, (700, 333)),  # the vocabulary of the reference's set task: 8 groups of token accumulators
    (128, 4, 3, 1, 300, None),
]


@pytest.mark.parametrize("case", SCANS, ids=[f"V{c[0]}-d{c[1]}-N{c[2]}-B{c[3]}-n{c[4]}-{'mask' if c[5] else 'nomask'}"
                                             for c in SCANS])
def test_token_scan_forward_and_cache_grads(case):
    V, d, N, B, n, lens = case
    rng = np.random.default_rng(V * 100 + d)
    P, Dc = _cache(V, d, N, V + d)
    ids = torch.tensor(rng.integers(0, V, size=(B, n)))
    mask = None
    if lens is not None:
        mask = torch.zeros(B, n, dtype=torch.bool)
        for i, k in enumerate(lens):
            mask[i, :k] = True
    Pg = P.float().to(DEV).requires_grad_(True)
    Dg = Dc.float().to(DEV).requires_grad_(True)
    out = E.token_cached_prefix_scan(ids.to(DEV), None if mask is None else mask.to(DEV), Pg, Dg, d, N)
    Pr = P.clone().requires_grad_(True)
    Dr = Dc.clone().requires_grad_(True)
    ref = torch.stack([TO.token_cached_prefix_scan(ids[b], None if mask is None else mask[b], Pr, Dr, d, N)
                       for b in range(B)])
    assert out.shape == ref.shape
    assert relerr(out, ref) < 1e-5, relerr(out, ref)
    w = torch.tensor(np.random.default_rng(1).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    assert relerr(Pg.grad, Pr.grad) < 1e-4, relerr(Pg.grad, Pr.grad)
    assert relerr(Dg.grad, Dr.grad) < 1e-4, relerr(Dg.grad, Dr.grad)


CACHES = [
    # leaf, d, N, V, kwargs
    ("van_loan", 4, 2, 5, dict(M=4, expm_method="exact")),
    ("van_loan", 3, 3, 3, dict(M=6, expm_method="cayley", chen_expm_method="exact")),
    ("series", 5, 2, 6, dict(M=1, series_q=12)),
    ("series", 16, 2, 4, dict(M=1, series_q=10)),
]


def _vocab(V, d, seed):
    rng = np.random.default_rng(seed)
    dx = torch.tensor(rng.normal(size=(V, d)) * 0.4)
    dth = torch.tensor(rng.uniform(0.05, 0.5, size=V))
    S = rng.normal(size=(d, d)) * 0.3
    A = torch.tensor(np.diag(rng.uniform(0.2, 1.0, d)) + (S - S.T) / 2)
    return dx, dth, A


@pytest.mark.parametrize("case", CACHES, ids=[f"{c[0]}-d{c[1]}-N{c[2]}-V{c[3]}" for c in CACHES])
def test_build_token_cache_and_chain(case):
    leaf, d, N, V, kw = case
    dx, dth, A = _vocab(V, d, d * 10 + N)
    M = kw["M"]
    expm = kw.get("expm_method", "exact")
    chen = kw.get("chen_expm_method")
    q = kw.get("series_q")
    g = [t.float().to(DEV).requires_grad_(True) for t in (dx, dth, A)]
    P, Dc = E.build_token_cache(g[0], g[1], g[2], M, N, expm, chen, leaf, q)
    r = [t.clone().requires_grad_(True) for t in (dx, dth, A)]
    Pr, Dr = TO.build_token_cache(r[0], r[1], r[2], M, N, expm, chen, leaf, q)
    assert relerr(P, Pr) < 1e-5 and relerr(Dc, Dr) < 1e-5, (relerr(P, Pr), relerr(Dc, Dr))
    # the chain: tokens -> cached scan, against the oracle chain
    B, n = 2, 90
    ids = torch.tensor(np.random.default_rng(3).integers(0, V, size=(B, n)))
    mask = torch.ones(B, n, dtype=torch.bool)
    mask[1, 60:] = False
    out = E.token_cached_prefix_scan(ids.to(DEV), mask.to(DEV), P, Dc, d, N)
    ref = torch.stack([TO.token_cached_prefix_scan(ids[b], mask[b], Pr, Dr, d, N) for b in range(B)])
    assert relerr(out, ref) < 1e-5, relerr(out, ref)
    w = torch.tensor(np.random.default_rng(2).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    for a, b, nm in zip(g, r, ("vocab_dx", "vocab_dtheta", "A")):
        assert relerr(a.grad, b.grad) < 1e-4, (nm, relerr(a.grad, b.grad))


def test_token_scan_equals_dense_layer_on_expanded_path():
    """The reference's equivalence (ews/core/token_scan.py:1-7) on the GPU: the cached scan and the dense EWS kernels
    on the path whose increments are the tokens' give the same prefix rows."""
    V, d, N, L = 4, 4, 2, 200
    dx, dth, A = _vocab(V, d, 5)
    ids = torch.tensor(np.random.default_rng(6).integers(0, V, size=L))
    P, Dc = E.build_token_cache(dx.float().to(DEV), dth.float().to(DEV), A.float().to(DEV), 20, N, "cayley",
                                "exact", "van_loan")
    cached = E.token_cached_prefix_scan(ids.to(DEV), None, P, Dc, d, N)
    path = torch.cat([torch.zeros(1, d, dtype=DT), torch.cumsum(dx[ids], 0)], 0)
    clock = torch.cat([torch.zeros(1, dtype=DT), torch.cumsum(dth[ids], 0)], 0)
    layer = E.EWS(E.AParamConstant(A.float()), N=N, M=20, leaf="van_loan", van_loan_expm="cayley",
                  chen_expm="exact").to(DEV)
    flat = layer(path.float().to(DEV)[None], clock.float().to(DEV)[None], readout="prefix")[0]
    ref = O.ews_single(path, clock, A, N, "prefix", leaf="van_loan", M=20, van_loan_expm="cayley",
                       chen_expm="exact", output_format="flat")[:, 1:]
    assert relerr(cached, ref) < 1e-5, relerr(cached, ref)
    assert relerr(flat[:, 1:], ref) < 1e-4, relerr(flat[:, 1:], ref)
