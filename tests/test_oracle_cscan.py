"""The C restatement (oracle/cpu_scan.c, the full-size checker and CPU baseline) against the torch float64
oracle: forward prefix rows and the gradients of a random-weighted loss, in the three flow modes."""

import numpy as np
import pytest
import torch

from oracle import cbuild
from oracle import cpu_scan_py as C
from oracle import ews_oracle as O


@pytest.fixture(scope="module", autouse=True)
def _built():
    cbuild.build(verbose=False)


def _case(seed, B=2, L=23, K=3):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, 2 * K)) * 0.4, 1)
    clock = np.cumsum(rng.uniform(0.05, 0.4, size=(B, L)), 1)
    dw = np.stack([rng.uniform(0.05, 1.0, K), rng.uniform(-2, 2, K)], -1)
    return path, clock, dw


def _dense(dw):
    K = dw.shape[0]
    A = torch.zeros((2 * K, 2 * K), dtype=torch.float64)
    for j in range(K):
        A = A.index_put((torch.tensor([2 * j, 2 * j, 2 * j + 1, 2 * j + 1]),
                         torch.tensor([2 * j, 2 * j + 1, 2 * j, 2 * j + 1])),
                        torch.stack([dw[j, 0], dw[j, 1], -dw[j, 1], dw[j, 0]]))
    return A


@pytest.mark.parametrize("mode,flow", [("displacement", "per_interval"), ("displacement_uniform", "cached"),
                                       ("displacement_uniform_basepoint", "cached_basepoint")])
def test_c_scan_matches_torch_oracle(mode, flow):
    path, clock, dw = _case(1)
    got = C.planes_forward(path, clock, dw, flow)
    pt = torch.tensor(path, requires_grad=True)
    ct = torch.tensor(clock, requires_grad=True)
    wt = torch.tensor(dw, requires_grad=True)
    ref = O.ews(pt, ct, _dense(wt), 2, "prefix", leaf="plane_closed", reweighting_mode=mode)
    np.testing.assert_allclose(got, ref.detach().numpy(), rtol=0, atol=1e-12 * np.abs(got).max())
    g = np.random.default_rng(5).normal(size=got.shape)
    (ref * torch.tensor(g)).sum().backward()
    dp, dc, dd = C.planes_backward(path, clock, dw, g, flow)
    for a, b in ((dp, pt.grad), (dc, ct.grad), (dd, wt.grad)):
        b = b.numpy()
        assert np.abs(a - b).max() <= 1e-10 * max(1.0, np.abs(b).max())


def test_c_scan_gradients_at_bench_shape():
    """d = 16 planes, float32-uniform clock (the bench's c2 shape at L = 400): the checker's coefficient derivatives
    are analytic, so its clock gradient (a difference of adjacent step gradients) stays exact to ~1e-11."""
    rng = np.random.default_rng(11)
    B, L = 1, 400
    path = np.cumsum(rng.normal(0.0, np.sqrt(1.0 / L), size=(B, L, 16)), 1)
    clock = np.broadcast_to((np.arange(L) / L).astype(np.float32).astype(np.float64), (B, L)).copy()
    dw = np.stack([rng.uniform(0.01, 1.0, 8), rng.uniform(0.0, np.pi, 8)], -1)
    pt = torch.tensor(path, requires_grad=True)
    ct = torch.tensor(clock, requires_grad=True)
    wt = torch.tensor(dw, requires_grad=True)
    ref = O.ews(pt, ct, _dense(wt), 2, "prefix", leaf="plane_closed")
    np.testing.assert_allclose(C.planes_forward(path, clock, dw), ref.detach().numpy(), rtol=0,
                               atol=1e-10 * float(ref.abs().max()))
    g = np.random.default_rng(5).normal(size=tuple(ref.shape))
    (ref * torch.tensor(g)).sum().backward()
    dp, dc, dd = C.planes_backward(path, clock, dw, g)
    for a, b in ((dp, pt.grad), (dc, ct.grad), (dd, wt.grad)):
        b = b.numpy()
        assert np.abs(a - b).max() <= 1e-10 * np.abs(b).max()
