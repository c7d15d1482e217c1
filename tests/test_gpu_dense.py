"""GPU parity of the dense-generator kernels (series leaf, exact flows, MFMA Chen scan) against the float64 oracle.

Bars: forward max relative error <= 1e-5 with the reference's metric
max|a-b| / max|b| (tests/test_engines.py:31-33). The oracle restates ews/core/series_leaf.py:55-126 with the
coefficient tensor, the flows of ews/core/chen_scan.py:155-168 with a float64 matrix exponential, and the
sequential Chen recursion; the kernels compute the same truncated series through nested degree sums, so the
two differ by float32 rounding only. Cases: the leaf alone, the combine alone on oracle inputs, the layer for
every readout and reweighting mode, depths 1-3, d = 16 and a padded d, single- and multi-chunk lengths, steps
with h ||A|| above 1 (scaled-and-squared flows), and the c3 recipe at reduced length.
"""

import numpy as np
import pytest
import torch

import bench
import ews_mi355x as E
from ews_mi355x import ops
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def c3_inputs(B, L):
    """BASELINE.json configs[2] recipe, from the bench (bench.c3_inputs), as float32 tensors."""
    path, clock, A = bench.c3_inputs(B, L)
    return torch.tensor(path), torch.tensor(clock), torch.tensor(A)


def _random(B, L, d, seed, hscale=0.05, ascale=1.0):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1)
    clock = np.cumsum(rng.uniform(0.5, 1.5, size=(B, L)) * hscale, 1)
    A = rng.normal(size=(d, d)) * ascale / np.sqrt(d) + np.eye(d) * 0.5 * ascale
    return (torch.tensor(path, dtype=torch.float32), torch.tensor(clock, dtype=torch.float32),
            torch.tensor(A, dtype=torch.float32))


def _oracle_levels(path, clock, A, N, q, mode="displacement"):
    """Per-sample oracle leaf + flows (float64)."""
    lv, fl = [], []
    cached = mode != "displacement"
    basepoint = mode == "displacement_uniform_basepoint"
    for b in range(path.shape[0]):
        p, c = path[b].double(), clock[b].double()
        levels = O.series_local_terms(p[1:] - p[:-1], c[1:] - c[:-1], A.double(), N, q)
        lv.append(O.pack(levels))
        fl.append(O.flows(c[1:] - c[:-1], A.double(), "exact", cached, basepoint))
    return torch.stack(lv), torch.stack(fl)


@pytest.mark.parametrize("N,d,q,hscale", [(1, 16, 8, 0.05), (2, 16, 12, 0.05), (3, 16, 20, 0.05),
                                          (3, 5, 16, 0.05), (3, 16, 24, 0.6), (2, 9, 40, 0.3)])
def test_dense_local_terms(N, d, q, hscale):
    path, clock, A = _random(2, 37, d, seed=10 + N + d, hscale=hscale)
    lv, fl = ops.dense_local_terms(path.to(DEV), clock.to(DEV), A.to(DEV), N, q)
    rlv, rfl = _oracle_levels(path, clock, A, N, q)
    print(f"local N={N} d={d} q={q} h={hscale}: levels {relerr(lv, rlv):.2e} flows {relerr(fl, rfl):.2e}")
    assert relerr(fl, rfl) < 1e-5
    off = 0
    for k in range(1, N + 1):  # every level on its own scale
        n = d**k
        assert relerr(lv[..., off:off + n], rlv[..., off:off + n]) < 1e-5, k
        off += n


@pytest.mark.parametrize("N,d,n,chunk", [(1, 16, 50, 8), (2, 16, 50, 8), (3, 16, 50, 8), (3, 16, 130, 0),
                                         (3, 7, 45, 16), (2, 3, 33, 4)])
def test_dense_combine_on_oracle_inputs(N, d, n, chunk):
    path, clock, A = _random(2, n + 1, d, seed=20 + N + d)
    rlv, rfl = _oracle_levels(path, clock, A, N, 10)
    ref = torch.stack([O.chen_scan_prefix(O.unpack(rlv[b], d, N), rfl[b]) for b in range(2)])
    got = ops.dense_combine(rlv.float().to(DEV), rfl.float().to(DEV), N, "prefix", level0=False, chunk=chunk)
    print(f"combine N={N} d={d} n={n} chunk={chunk}: {relerr(got, ref):.2e}")
    assert relerr(got, ref) < 1e-5
    term = ops.dense_combine(rlv.float().to(DEV), rfl.float().to(DEV), N, "terminal", level0=True, chunk=chunk)
    assert relerr(term[:, 1:], ref[:, -1]) < 1e-5
    assert torch.all(term[:, 0] == 1.0)


@pytest.mark.parametrize("readout", ["prefix", "terminal", "mean", "max"])
@pytest.mark.parametrize("mode", ["displacement", "displacement_uniform", "displacement_uniform_basepoint"])
def test_dense_layer_parity(readout, mode):
    B, L, d, N, q = 2, 90, 16, 3, 16
    path, clock, A = _random(B, L, d, seed=31, hscale=0.04)
    if mode != "displacement":
        clock = torch.linspace(0.0, 3.0, L).expand(B, L).contiguous()
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=N, leaf="series", series_q=q, reweighting_mode=mode,
                  terminal_reduce="assoc")
    out = layer(path.to(DEV), clock.to(DEV), readout=readout)
    ref = O.ews(path.double(), clock.double(), A.double(), N, readout, leaf="series", series_q=q,
                reweighting_mode=mode, terminal_reduce="assoc")
    print(f"layer {readout} {mode}: {relerr(out, ref):.2e}")
    assert out.shape == ref.shape
    assert relerr(out, ref) < 1e-5


def test_dense_layer_list_format_and_tree_terminal():
    B, L, d, N, q = 2, 70, 6, 3, 12
    path, clock, A = _random(B, L, d, seed=41)
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=N, leaf="series", series_q=q)  # tree terminal: per-interval flows
    lv = layer(path.to(DEV), clock.to(DEV), readout="terminal", output_format="list")
    ref = O.ews(path.double(), clock.double(), A.double(), N, "terminal", leaf="series", series_q=q)[:, 1:]
    assert [tuple(x.shape) for x in lv] == [(B,) + (d,) * k for k in range(1, N + 1)]
    off = 0
    for k in range(N):
        n = d ** (k + 1)
        assert relerr(lv[k].reshape(B, n), ref[:, off:off + n]) < 1e-5
        off += n
    single = layer(path[0].to(DEV), clock[0].to(DEV), readout="prefix")
    assert single.shape == (L - 1, 1 + d + d * d + d**3)


def test_dense_planes_at_depth3_route_to_dense_kernels():
    K = 4
    rng = np.random.default_rng(5)
    v = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    u = torch.tensor(rng.normal(size=K), dtype=torch.float32)
    path, clock, _ = _random(2, 40, 2 * K, seed=51)
    layer = E.EWS(E.AParamDampedRotation(v, u, 2 * K).to(DEV), N=3, leaf="series", series_q=20)
    out = layer(path.to(DEV), clock.to(DEV), readout="prefix")
    A = E.AParamDampedRotation(v.double(), u.double(), 2 * K)()
    ref = O.ews(path.double(), clock.double(), A, 3, "prefix", leaf="series", series_q=20)
    assert relerr(out, ref) < 1e-5


def test_dense_c3_recipe():
    """BASELINE.json configs[2] at B=2 and L=700 (the full L=4096 runs in the bench)."""
    B, L, q = 2, 700, 24
    path, clock, A = c3_inputs(B, L)
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=3, leaf="series", series_q=q)
    out = layer(path.to(DEV), clock.to(DEV), readout="prefix")
    ref = O.ews(path.double(), clock.double(), A.double(), 3, "prefix", leaf="series", series_q=q)
    e = relerr(out, ref)
    print(f"c3 recipe L={L}: {e:.2e}; max h||A||_1 = {float((clock[:, 1:] - clock[:, :-1]).max()):.3f} x "
          f"{float(A.abs().sum(0).max()):.3f}")
    assert e < 1e-5


def test_dense_backward_through_the_layer():
    """The layer's backward runs the dense adjoint kernels (parity: tests/test_gpu_dense_bwd.py)."""
    path, clock, A = _random(1, 10, 4, seed=61)
    p = path.to(DEV).requires_grad_(True)
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=2, leaf="series", series_q=8)
    out = layer(p, clock.to(DEV), readout="prefix")
    out.sum().backward()
    assert p.grad is not None and torch.isfinite(p.grad).all()
