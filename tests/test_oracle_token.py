"""CPU pins of the token-cache oracle (oracle/token_oracle.py) by the reference's own claim for this path
(ews/core/token_scan.py:1-7 and tests/test_token_cache.py:96-111): for the same per-position segments the
token-cached scan reproduces the ordinary EWS prefix scan, forward and gradient. The ordinary scan here is the
oracle's EWS on the path whose increments are the tokens' displacements and clock increments (padded steps: zero
increments, as the increment path and the frozen clock give them), an independent route through the leaf on
every interval and the Chen recursion."""

import numpy as np
import pytest
import torch

from oracle import ews_oracle as O
from oracle import token_oracle as TO

DT = torch.float64


def _setup(V, d, seed):
    rng = np.random.default_rng(seed)
    dx = torch.tensor(rng.normal(size=(V, d)) * 0.4, dtype=DT, requires_grad=True)
    dth = torch.tensor(rng.uniform(0.05, 0.6, size=V), dtype=DT, requires_grad=True)
    S = rng.normal(size=(d, d)) * 0.3
    A = torch.tensor(np.diag(rng.uniform(0.2, 1.0, d)) + (S - S.T) / 2, dtype=DT, requires_grad=True)
    return dx, dth, A


def _expanded(ids, mask, dx, dth):
    on = torch.ones(len(ids), dtype=DT) if mask is None else mask.to(DT)
    inc = dx[ids] * on[:, None]
    dinc = dth[ids] * on
    path = torch.cat([torch.zeros(1, dx.shape[1], dtype=DT), torch.cumsum(inc, 0)], 0)
    clock = torch.cat([torch.zeros(1, dtype=DT), torch.cumsum(dinc, 0)], 0)
    return path, clock


@pytest.mark.parametrize("leaf", ["van_loan", "series"])
@pytest.mark.parametrize("masked", [False, True])
def test_token_scan_equals_ordinary_scan(leaf, masked):
    V, d, N, L = 4, 3, 2, 12
    dx, dth, A = _setup(V, d, 3)
    ids = torch.tensor(np.random.default_rng(4).integers(0, V, size=L))
    mask = (torch.arange(L) < 8) if masked else None
    kw = dict(M=4, expm_method="exact", leaf=leaf, series_q=10)
    P, D = TO.build_token_cache(dx, dth, A, kw["M"], N, kw["expm_method"], None, leaf, kw["series_q"])
    got = TO.token_cached_prefix_scan(ids, mask, P, D, d, N)
    path, clock = _expanded(ids, mask, dx, dth)
    ref = O.ews_single(path, clock, A, N, "prefix", leaf=leaf, M=4, van_loan_expm="exact", chen_expm="exact",
                       series_q=10, output_format="flat")[:, 1:]
    np.testing.assert_allclose(got.detach().numpy(), ref.detach().numpy(), rtol=1e-12, atol=1e-13)
    w = torch.tensor(np.random.default_rng(5).normal(size=tuple(ref.shape)))
    g1 = torch.autograd.grad((got * w).sum(), (dx, dth, A))
    g2 = torch.autograd.grad((ref * w).sum(), (dx, dth, A))
    for a, b in zip(g1, g2):
        np.testing.assert_allclose(a.numpy(), b.numpy(), rtol=1e-10, atol=1e-12)
    if masked:  # padded steps are the identity: the prefix is frozen past the mask
        assert torch.equal(got[8:], got[7:8].expand(L - 8, -1))


def test_one_token_stream_is_a_geometric_recursion():
    """All steps the same token g: S_t = mult(apply_M(S_{t-1}, D_g), P_g), level 1 = sum_{s<t} D_g^s p1 (the
    depth-1 affine recursion)."""
    dx, dth, A = _setup(3, 4, 7)
    P, D = TO.build_token_cache(dx, dth, A, 4, 1, "exact", None, "van_loan")
    got = TO.token_cached_prefix_scan(torch.full((6,), 2), None, P, D, 4, 1)
    x = torch.zeros(4, dtype=DT)
    for t in range(6):
        x = D[2] @ x + P[2]
        np.testing.assert_allclose(got[t].detach().numpy(), x.detach().numpy(), rtol=1e-12)


def test_depth1_batched_scan_equals_the_packed_chen_loop():
    """The batched depth-1 form (D S + P) against the per-sample packed Chen loop, with masks, forward and
    gradients."""
    rng = np.random.default_rng(31)
    B, L, d, V = 3, 17, 5, 4
    P = torch.tensor(rng.normal(size=(V, d)), dtype=DT, requires_grad=True)
    Dc = torch.tensor(rng.normal(size=(V, d, d)) * 0.4, dtype=DT, requires_grad=True)
    tok = torch.tensor(rng.integers(0, V, size=(B, L)))
    mask = torch.tensor(np.arange(L)[None, :] < np.array([L, 11, 5])[:, None])
    a = TO.token_cached_prefix_scan_depth1(tok, mask, P, Dc)
    b = torch.stack([TO.token_cached_prefix_scan(tok[i], mask[i], P, Dc, d, 1) for i in range(B)])
    assert float((a - b).abs().max()) < 1e-13
    w = torch.tensor(rng.normal(size=(B, L, d)), dtype=DT)
    ga = torch.autograd.grad((a * w).sum(), [P, Dc])
    gb = torch.autograd.grad((b * w).sum(), [P, Dc])
    for x, y in zip(ga, gb):
        assert float((x - y).abs().max()) < 1e-12
