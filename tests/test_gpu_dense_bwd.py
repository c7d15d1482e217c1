"""GPU parity of the dense-generator backward against torch float64 autograd of the oracle.

Bar: gradients within max relative error 1e-4 (max|a-b| / max|b|, the reference's
metric, tests/test_engines.py:31-33), each gradient (and each level) on its own scale. The oracle's Chen scan is
the plain sequential recursion of ews/core/chen_scan.py:98-152 in float64, differentiated by torch autograd, so
the adjoint scan (local reverse scans, the carry scan over chunk summaries, the emitting reverse scan) is checked
against the chain rule itself; multi-chunk lengths exercise the carries, every readout its cotangent routing.
"""

import numpy as np
import pytest
import torch
from scipy.linalg import expm

from ews_mi355x import ops
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _inputs(B, n, d, N, seed):
    rng = np.random.default_rng(seed)
    D = sum(d**k for k in range(1, N + 1))
    lv = rng.normal(size=(B, n, D)) * 0.3
    off = d
    for k in range(2, N + 1):  # higher levels smaller, as local terms are
        lv[..., off:off + d**k] *= 0.3 ** (k - 1)
        off += d**k
    A = rng.normal(size=(d, d)) / np.sqrt(d) + 0.5 * np.eye(d)
    h = rng.uniform(0.02, 0.1, size=(B, n))
    fl = np.stack([np.stack([expm(-hh * A) for hh in h[b]]) for b in range(B)])
    return torch.tensor(lv), torch.tensor(fl)


def _combine_ref(lv, fl, d, N, readout, level0):
    B = lv.shape[0]
    prefix = torch.stack([O.chen_scan_prefix(O.unpack(lv[b], d, N), fl[b]) for b in range(B)])
    flat = torch.cat([torch.ones(prefix.shape[:-1] + (1,), dtype=prefix.dtype), prefix], -1)
    if readout == "prefix":
        return flat if level0 else prefix
    if readout == "terminal":
        return flat[:, -1] if level0 else prefix[:, -1]
    if readout == "mean":
        return flat.mean(1)
    return flat.max(1).values


def _check_levels(got, ref, d, N, bar, tag):
    off = 0
    for k in range(1, N + 1):
        n = d**k
        e = relerr(got[..., off:off + n], ref[..., off:off + n])
        assert e < bar, (tag, k, e)
        off += n


@pytest.mark.parametrize("readout", ["prefix", "terminal", "mean", "max"])
@pytest.mark.parametrize("N,d,n,chunk", [(1, 16, 50, 8), (2, 16, 50, 8), (3, 16, 50, 16), (3, 16, 130, 0),
                                         (3, 7, 45, 16), (2, 3, 33, 4)])
def test_dense_combine_backward(readout, N, d, n, chunk):
    B = 2
    lv, fl = _inputs(B, n, d, N, seed=700 + 10 * N + d)
    level0 = readout in ("mean", "max") or N != 2
    lv64 = lv.clone().requires_grad_(True)
    fl64 = fl.clone().requires_grad_(True)
    out = _combine_ref(lv64, fl64, d, N, readout, level0)
    rng = np.random.default_rng(1)
    gout = torch.tensor(rng.normal(size=out.shape))
    rlv, rfl = torch.autograd.grad(out, (lv64, fl64), gout)
    glv, gfl = ops.dense_combine_backward(lv.float().to(DEV), fl.float().to(DEV), gout.float().to(DEV), N,
                                          readout, level0, chunk)
    print(f"combine bwd {readout} N={N} d={d} n={n} chunk={chunk}: levels {relerr(glv, rlv):.2e} "
          f"flows {relerr(gfl, rfl):.2e}")
    _check_levels(glv, rlv, d, N, 1e-4, "levels")
    assert relerr(gfl, rfl) < 1e-4


# ------------------------------------------------------------------------------------------------ full backward
def _random(B, L, d, seed, hscale=0.05, ascale=1.0, uniform=False):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1)
    if uniform:
        clock = np.broadcast_to(np.arange(L) * hscale, (B, L)).copy()
    else:
        clock = np.cumsum(rng.uniform(0.5, 1.5, size=(B, L)) * hscale, 1)
    A = rng.normal(size=(d, d)) * ascale / np.sqrt(d) + np.eye(d) * 0.5 * ascale
    return torch.tensor(path), torch.tensor(clock), torch.tensor(A)


_FLOW = {"displacement": "per_interval", "displacement_uniform": "cached",
         "displacement_uniform_basepoint": "cached_basepoint"}


def _grads(path, clock, A, N, q, readout, mode, level0=True, clock_grad=True, seed=3):
    """(GPU grads, float64 autograd grads of the oracle) for (path, clock, A)."""
    p64, c64, A64 = (x.clone().requires_grad_(True) for x in (path, clock, A))
    ref_out = O.ews(p64, c64, A64, N, readout, leaf="series", series_q=q, reweighting_mode=mode,
                    terminal_reduce="assoc")
    if not level0:
        ref_out = ref_out[..., 1:]
    gout = torch.tensor(np.random.default_rng(seed).normal(size=ref_out.shape))
    ref = torch.autograd.grad(ref_out, (p64, c64, A64), gout)
    pg = path.float().to(DEV).requires_grad_(True)
    cg = clock.float().to(DEV).requires_grad_(clock_grad)
    Ag = A.float().to(DEV).requires_grad_(True)
    out = ops.dense_scan(pg, cg, Ag, N, q, _FLOW[mode], readout, level0)
    got = torch.autograd.grad(out, (pg, cg, Ag) if clock_grad else (pg, Ag), gout.float().to(DEV))
    if not clock_grad:
        got = (got[0], None, got[1])
    return got, ref


@pytest.mark.parametrize("readout", ["prefix", "terminal", "mean", "max"])
@pytest.mark.parametrize("N,d,q,L", [(1, 16, 8, 40), (2, 16, 12, 70), (3, 16, 16, 70), (3, 5, 10, 45)])
def test_dense_backward_series(readout, N, d, q, L):
    path, clock, A = _random(2, L, d, seed=800 + N + d)
    got, ref = _grads(path, clock, A, N, q, readout, "displacement", level0=readout in ("mean", "max") or N != 2)
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd {readout} N={N} d={d} q={q}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4


@pytest.mark.parametrize("mode", ["displacement_uniform", "displacement_uniform_basepoint"])
def test_dense_backward_cached_flows(mode):
    path, clock, A = _random(2, 60, 8, seed=820, uniform=True)
    got, ref = _grads(path, clock, A, 3, 12, "prefix", mode)
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd {mode}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4


def test_dense_backward_large_steps_and_no_clock_grad():
    """h ||A||_1 above 1 (flows scaled and squared, whose adjoint runs through the squarings), and a data clock
    (no clock gradient: the kernels skip it)."""
    path, clock, A = _random(2, 40, 16, seed=830, hscale=0.6)
    got, ref = _grads(path, clock, A, 3, 24, "terminal", "displacement")
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd large steps: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4
    got2, _ = _grads(path, clock, A, 3, 24, "terminal", "displacement", clock_grad=False)
    assert got2[1] is None
    assert relerr(got2[0], ref[0]) < 1e-4 and relerr(got2[2], ref[2]) < 1e-4


def _grads_kw(path, clock, A, N, readout, mode, leaf_kw, level0=True, seed=5):
    """(GPU grads, float64 autograd grads of the oracle) for (path, clock, A) under the leaf options leaf_kw."""
    p64, c64, A64 = (x.clone().requires_grad_(True) for x in (path, clock, A))
    ref_out = O.ews(p64, c64, A64, N, readout, reweighting_mode=mode, terminal_reduce="assoc", **leaf_kw)
    gout = torch.tensor(np.random.default_rng(seed).normal(size=ref_out.shape))
    ref = torch.autograd.grad(ref_out, (p64, c64, A64), gout)
    pg, cg, Ag = (x.float().to(DEV).requires_grad_(True) for x in (path, clock, A))
    kind = leaf_kw.get("leaf", "van_loan")
    leaf = ops.DenseLeaf(kind, q=leaf_kw.get("series_q", 0), M=leaf_kw.get("M", 20),
                         van_loan_expm=leaf_kw.get("van_loan_expm", "cayley"), reweighting_mode=mode,
                         chen_expm=leaf_kw.get("chen_expm", "exact"))
    out = ops.dense_scan(pg, cg, Ag, N, leaf.q, _FLOW[mode], readout, level0, leaf=leaf)
    got = torch.autograd.grad(out, (pg, cg, Ag), gout.float().to(DEV))
    return got, ref


@pytest.mark.parametrize("scheme", ["exact", "cayley", "euler", "pade"])
@pytest.mark.parametrize("N", [1, 2, 3])
def test_dense_backward_van_loan(scheme, N):
    path, clock, A = _random(2, 30, 16 if N < 3 else 6, seed=900 + N)
    got, ref = _grads_kw(path, clock, A, N, "prefix", "displacement",
                         dict(leaf="van_loan", M=7, van_loan_expm=scheme))
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd van loan {scheme} N={N}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4


@pytest.mark.parametrize("mode", ["displacement_uniform", "displacement_uniform_basepoint"])
@pytest.mark.parametrize("scheme", ["exact", "cayley"])
def test_dense_backward_van_loan_uniform(mode, scheme):
    path, clock, A = _random(2, 40, 8, seed=910, uniform=True)
    got, ref = _grads_kw(path, clock, A, 3, "terminal", mode, dict(leaf="van_loan", M=20, van_loan_expm=scheme))
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd van loan {scheme} {mode}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4


def test_dense_backward_van_loan_large_steps():
    """delta ||A||_1 above the series radii: Gauss-Jordan step matrices and scaled exponentials (their doublings)."""
    path, clock, A = _random(2, 20, 8, seed=920, hscale=3.0, ascale=0.4)
    for scheme in ("exact", "cayley", "pade", "euler"):
        got, ref = _grads_kw(path, clock, A, 2, "terminal", "displacement",
                             dict(leaf="van_loan", M=2, van_loan_expm=scheme))
        errs = [relerr(g, r) for g, r in zip(got, ref)]
        print(f"dense bwd van loan large {scheme}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
        assert max(errs) < 1e-4, scheme


@pytest.mark.parametrize("chen", ["cayley", "pade", "euler"])
@pytest.mark.parametrize("flow_mode", ["displacement", "displacement_uniform"])
def test_dense_backward_flow_schemes(chen, flow_mode):
    path, clock, A = _random(2, 30, 8, seed=930, hscale=0.2, uniform=flow_mode != "displacement")
    got, ref = _grads_kw(path, clock, A, 2, "prefix", flow_mode, dict(leaf="series", series_q=12, chen_expm=chen))
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd flows {chen} {flow_mode}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4
    # larger steps: the Gauss-Jordan inverse instead of the series
    path, clock, A = _random(2, 12, 8, seed=931, hscale=1.5, ascale=0.5)
    got, ref = _grads_kw(path, clock, A, 2, "terminal", "displacement",
                         dict(leaf="series", series_q=30, chen_expm=chen))
    errs = [relerr(g, r) for g, r in zip(got, ref)]
    print(f"dense bwd flows large {chen}: path {errs[0]:.2e} clock {errs[1]:.2e} A {errs[2]:.2e}")
    assert max(errs) < 1e-4


@pytest.mark.parametrize("B,L,d,N", [(1, 2, 1, 1), (1, 2, 3, 3), (3, 3, 2, 2), (1, 65, 4, 3), (2, 129, 16, 2)])
def test_dense_backward_edge_shapes(B, L, d, N):
    """One interval, width 1, the basepoint minimum length, chunk-boundary lengths (64 + 1, 128 + 1)."""
    path, clock, A = _random(B, L, d, seed=950 + L + d)
    for readout in ("prefix", "terminal"):
        got, ref = _grads(path, clock, A, N, 6, readout, "displacement")
        errs = [relerr(g, r) for g, r in zip(got, ref)]
        print(f"dense bwd edge B={B} L={L} d={d} N={N} {readout}: {max(errs):.2e}")
        assert max(errs) < 1e-4
    got, ref = _grads_kw(path, clock, A, N, "mean", "displacement", dict(leaf="van_loan", M=3, van_loan_expm="cayley"))
    assert max(relerr(g, r) for g, r in zip(got, ref)) < 1e-4


@pytest.mark.parametrize("leaf,N,mode", [("van_loan", 3, "displacement_uniform"), ("van_loan", 2, "displacement"),
                                         ("series", 3, "displacement_uniform_basepoint"),
                                         ("series", 2, "displacement_uniform")])
def test_dense_backward_is_deterministic(leaf, N, mode):
    """Two backward calls in one process give bit-identical gradients of A, the clock and the path: every sum in
    the dense backward runs in a fixed order (per-wavefront partials, per-interval terms reduced by one workgroup
    per sample), with no float atomics. The cached modes take the shared-step reduction; depth 3 of the Van Loan
    leaf the cross-wavefront column sums."""
    B, L, d = 3, 300, 16
    rng = np.random.default_rng(77)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.2, 1), dtype=torch.float32, device=DEV)
    clock = torch.tensor(np.broadcast_to(np.arange(L) / L, (B, L)).copy(), dtype=torch.float32, device=DEV)
    A = torch.tensor(rng.normal(size=(d, d)) / np.sqrt(d) + np.eye(d), dtype=torch.float32, device=DEV)
    dl = ops.DenseLeaf(leaf, q=12, M=8, reweighting_mode=mode)
    flow = {"displacement": "per_interval", "displacement_uniform": "cached",
            "displacement_uniform_basepoint": "cached_basepoint"}[mode]
    g = torch.tensor(rng.normal(size=(B, L - 1, 1 + sum(d**k for k in range(1, N + 1)))), dtype=torch.float32,
                     device=DEV)
    grads = []
    for _ in range(2):
        p = path.clone().requires_grad_(True)
        c = clock.clone().requires_grad_(True)
        a = A.clone().requires_grad_(True)
        out = ops.dense_scan(p, c, a, N, dl.q, flow, "prefix", True, leaf=dl)
        (out * g).sum().backward()
        torch.cuda.synchronize()
        grads.append((p.grad.clone(), c.grad.clone(), a.grad.clone()))
    for name, x, y in zip(("path", "clock", "A"), grads[0], grads[1]):
        assert torch.equal(x, y), f"{name} gradient differs between two identical calls"


@pytest.mark.parametrize("leaf,N,readout", [("series", 3, "prefix"), ("van_loan", 2, "max"), ("series", 2, "mean"),
                                            ("block_series", 1, "terminal")])
def test_kept_forward_backward_equals_recompute(leaf, N, readout):
    """The training pair ews_dense_forward_keep / ews_dense_backward_kept (the forward's leaf, flows, summaries and
    carries kept for the backward) gives the gradients of ews_dense_backward (which recomputes them) bit for bit:
    both run the same kernels on the same data. A second backward of the same graph (retain_graph) finds the kept
    data consumed and recomputes; it matches too."""
    B, L, d = 2, 200, 16
    rng = np.random.default_rng(91)
    path = torch.tensor(np.cumsum(rng.normal(size=(B, L, d)) * 0.2, 1), dtype=torch.float32, device=DEV)
    clock = torch.tensor(np.cumsum(rng.uniform(0.01, 0.05, size=(B, L)), 1), dtype=torch.float32, device=DEV)
    A = torch.tensor(rng.normal(size=(d, d)) / np.sqrt(d) + np.eye(d), dtype=torch.float32, device=DEV)
    dl = ops.DenseLeaf(leaf, q=10, M=6)
    p = path.clone().requires_grad_(True)
    c = clock.clone().requires_grad_(True)
    a = A.clone().requires_grad_(True)
    out = ops.dense_scan(p, c, a, N, 10, "per_interval", readout, True, leaf=dl)
    g = torch.tensor(rng.normal(size=tuple(out.shape)), dtype=torch.float32, device=DEV)
    kept = torch.autograd.grad(out, (p, c, a), g, retain_graph=True)
    again = torch.autograd.grad(out, (p, c, a), g)  # the kept data is consumed: this one recomputes
    # the recomputing entry point on its own
    from ews_mi355x import _native as nat
    import ctypes
    lib = nat.load()
    desc = ops.make_dense_desc(B, L, d, N, 10, "per_interval", readout, True, 0, dl)
    ws = torch.empty(int(lib.ews_dense_backward_workspace_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    gp, gc, ga = torch.empty_like(path), torch.empty_like(clock), torch.empty_like(A)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.check(lib.ews_dense_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                     g.contiguous().data_ptr(), gp.data_ptr(), gc.data_ptr(), ga.data_ptr(),
                                     ws.data_ptr(), st), "ews_dense_backward")
    torch.cuda.synchronize()
    for name, x, y, z in zip(("path", "clock", "A"), kept, again, (gp, gc, ga)):
        assert torch.equal(x, z), f"{name}: kept backward differs from the recomputing one"
        assert torch.equal(y, z), f"{name}: second backward differs from the recomputing one"
