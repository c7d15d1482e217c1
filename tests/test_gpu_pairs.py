"""GPU parity of the plane pair-group kernels (rotation planes, d = 16, depth 2, prefix readout, per-interval
flows, chunks with a float32-uniform clock) against the float64 C checker (oracle/cpu_scan.c, itself pinned to
the torch oracle by tests/test_oracle_cscan.py).

Bars: forward max relative error <= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|
(the reference's tests/test_engines.py:31-33). Each case also reads the per-chunk classification the forward
leaves in its residual, so a case asserts which chunks ran in the pair-group kernels and which in the generic
ones: all-uniform clocks, clocks with non-uniform chunks mixed in, strong damping (steps not invertible: the
generic recomputing adjoint), partial last chunks and workgroups, tiny lengths, and bfloat16 paths.
"""

import ctypes

import numpy as np
import pytest
import torch

import ews_mi355x as E
from ews_mi355x import _native as nat
from ews_mi355x.ops import make_desc
from oracle import cbuild
from oracle import cpu_scan_py as C

pytestmark = pytest.mark.gpu

DEV = "cuda"
D16 = 16
T_DEFAULT = 64


@pytest.fixture(scope="module", autouse=True)
def _built():
    cbuild.build(verbose=False)


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _inputs(B, L, seed, damp=(0.01, 1.0), jitter_chunks=(), den=None):
    """c2-style inputs: Brownian 6-channel paths lifted to d = 16, planes (d_j, w_j), clock k/L (or k/den) in
    float32."""
    rng = np.random.default_rng(seed)
    inc = rng.normal(0.0, np.sqrt(1.0 / L), size=(B, L - 1, 6))
    pc = np.concatenate([np.zeros((B, 1, 6)), np.cumsum(inc, 1)], 1)
    Wl = rng.normal(0.0, np.sqrt(1.0 / 6), size=(D16, 6))
    path = (pc @ Wl.T).astype(np.float32)
    dw = np.stack([rng.uniform(*damp, 8), rng.uniform(0.0, np.pi, 8)], -1).astype(np.float32)
    clock = np.broadcast_to(np.arange(L, dtype=np.float64) / (den or L), (B, L)).copy()
    for c in jitter_chunks:
        clock[:, c * T_DEFAULT + 5] += 0.3 / L
    return path, clock.astype(np.float32), dw


def _align(x):
    return (x + 255) // 256 * 256


def _run(path, clock, dw, g, bf16=False, clock_grad=True):
    """Forward + backward through the C ABI; returns out, dpath, dclock, ddw and the chunk flags (clock_grad=False
    passes a null grad_clock: the clock gradient is not requested)."""
    lib = nat.load()
    B, L, d = path.shape
    dt = nat.DTYPE_BF16 if bf16 else nat.DTYPE_F32
    desc = make_desc(B, L, d, 2, nat.STRUCT_PLANES, nat.FLOW_PER_INTERVAL, "prefix", True, dt)
    W = 1 + d + d * d
    tp = torch.tensor(path, device=DEV)
    if bf16:
        tp = tp.to(torch.bfloat16)
    tc = torch.tensor(clock, device=DEV)
    tw = torch.tensor(dw, device=DEV)
    tg = torch.tensor(g, device=DEV, dtype=torch.float32)
    ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    rs = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    out = torch.empty((B, L - 1, W), device=DEV)
    dpath = torch.empty((B, L, d), device=DEV)
    dclock = torch.empty((B, L), device=DEV)
    ddw = torch.empty_like(tw)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    nat.check(lib.ews_diag_forward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), out.data_ptr(),
                                   rs.data_ptr(), ws.data_ptr(), st), "forward")
    nat.check(lib.ews_diag_backward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), rs.data_ptr(),
                                    tg.data_ptr(), dpath.data_ptr(), dclock.data_ptr() if clock_grad else None,
                                    ddw.data_ptr(), ws.data_ptr(), st), "backward")
    torch.cuda.synchronize()
    # residual layout (ews_diag.hip): float64 carries (B, C+1, D) | argmax (B, W) int32 | chunk flags (B, C) int32
    Cn = (L - 1 + T_DEFAULT - 1) // T_DEFAULT
    off = _align(B * (Cn + 1) * (d + d * d) * 8) + _align(B * W * 4)
    flags = rs[off: off + B * Cn * 4].view(torch.int32).reshape(B, Cn).cpu().numpy()
    return (out.cpu().numpy(), dpath.cpu().numpy(), dclock.cpu().numpy(), ddw.cpu().numpy(), flags)


def _check(path, clock, dw, bf16=False, seed=7):
    B, L, d = path.shape
    W = 1 + d + d * d
    g = (np.random.default_rng(seed).normal(size=(B, L - 1, W)) / np.sqrt(W)).astype(np.float32)
    src = path
    if bf16:
        src = torch.tensor(path).to(torch.bfloat16).to(torch.float64).numpy()
    out, dp, dc, dd, flags = _run(path, clock, dw, g, bf16)
    ref = C.planes_forward(src.astype(np.float64), clock.astype(np.float64), dw.astype(np.float64), kind="f64")
    rdp, rdc, rdd = C.planes_backward(src.astype(np.float64), clock.astype(np.float64), dw.astype(np.float64),
                                      g.astype(np.float64), kind="f64")
    errs = dict(fwd=relerr(out, ref), dpath=relerr(dp, rdp), dclock=relerr(dc, rdc), dparams=relerr(dd, rdd))
    # without the clock gradient the invertible chunks take the split adjoint (local adjoint + closed-form carry)
    _, dp2, _, dd2, _ = _run(path, clock, dw, g, bf16, clock_grad=False)
    errs.update(dpath_split=relerr(dp2, rdp), dparams_split=relerr(dd2, rdd))
    print(f"B={B} L={L} bf16={bf16} flags={np.bincount(flags.ravel(), minlength=8).tolist()} errs={errs}", flush=True)
    assert errs["fwd"] < 1e-5, errs
    assert errs["dpath"] < 1e-4 and errs["dclock"] < 1e-4 and errs["dparams"] < 1e-4, errs
    assert errs["dpath_split"] < 1e-4 and errs["dparams_split"] < 1e-4, errs
    return flags


@pytest.mark.parametrize("B,L", [(3, 300), (2, 2000), (2, 66), (1, 2), (5, 1 + 64 * 4 * 2 + 37)])
def test_uniform_chunks_run_in_pair_kernels(B, L):
    path, clock, dw = _inputs(B, L, seed=L)
    flags = _check(path, clock, dw)
    assert (flags & 1).all(), flags
    assert (flags & 4).all(), flags  # a uniform clock: every chunk takes the shared coefficient table
    if L >= 300:  # chunk span 64 / L with damping <= 1: the adjoint inverts the steps (2 d tau <= ln 2)
        assert (flags & 3 == 3).all(), flags


def test_multi_segment_carry_scans():
    # the carry scans stage 72 quads (288 chunks) per segment, in 8 wavefront blocks: 145 quads make two full
    # segments and a last one of a single quad, whose other seven blocks are empty
    L = 1 + 64 * 4 * 144 + 37
    path, clock, dw = _inputs(1, L, seed=11)
    flags = _check(path, clock, dw)
    assert (flags & 3 == 3).all(), flags


def test_mixed_chunks():
    path, clock, dw = _inputs(2, 600, seed=3, jitter_chunks=(1, 4))
    flags = _check(path, clock, dw)
    assert (flags[:, [1, 4]] & 5 == 0).all(), flags
    assert (flags[:, [0, 2, 3, 5]] & 3 == 3).all(), flags


def test_strong_damping_uses_recomputing_adjoint():
    # steps of exactly 2^-8 keep the chunks uniform at damping 60; a chunk then contracts by e^{-15}, too much to
    # invert the steps, so the adjoint recomputes the states forward (generic kernel) while the rest stays
    path, clock, dw = _inputs(2, 300, seed=4, damp=(40.0, 60.0), den=256)
    flags = _check(path, clock, dw)
    assert (flags & 3 == 1).all(), flags


def test_bf16_path():
    path, clock, dw = _inputs(2, 400, seed=5)
    flags = _check(path, clock, dw, bf16=True)
    assert (flags & 3 == 3).all(), flags


def test_layer_api_on_pair_kernels():
    """The EWS layer (ews/layer.py:43-307 call contract) over the same kernels, gradients wrt the plane
    parametrisation through autograd."""
    B, L = 2, 260
    path, clock, dw = _inputs(B, L, seed=9)
    v = torch.tensor(np.random.default_rng(1).normal(size=8), dtype=torch.float32)
    u = torch.tensor(np.random.default_rng(2).normal(size=8), dtype=torch.float32)
    A = E.AParamDampedRotation(v.clone(), u.clone(), 16, omega_scale=3.0).to(DEV)
    layer = E.EWS(A, N=2, leaf="plane_closed", combine="block_kernel")
    p = torch.tensor(path, device=DEV, requires_grad=True)
    out = layer(p, torch.tensor(clock, device=DEV), readout="prefix")
    g = np.random.default_rng(3).normal(size=tuple(out.shape))
    (out * torch.tensor(g, device=DEV, dtype=torch.float32)).sum().backward()
    Aref = E.AParamDampedRotation(v.double(), u.double(), 16, omega_scale=3.0)
    dwr = Aref.plane_params().detach().numpy()
    ref = C.planes_forward(path.astype(np.float64), clock.astype(np.float64), dwr, kind="f64")
    rdp, _, rdd = C.planes_backward(path.astype(np.float64), clock.astype(np.float64), dwr, g, kind="f64")
    assert relerr(out.detach().cpu().numpy(), ref) < 1e-5
    assert relerr(p.grad.cpu().numpy(), rdp) < 1e-4
    # chain the (d_j, w_j) gradient through the parametrisation on the CPU
    pp = Aref.plane_params()
    (pp * torch.tensor(rdd)).sum().backward()
    for g_gpu, g_ref in zip([A.v.grad, A.u.grad], [Aref.v.grad, Aref.u.grad]):
        assert relerr(g_gpu.cpu().numpy(), g_ref.numpy()) < 1e-4


def test_null_clock_gradient_leaves_the_other_gradients_unchanged():
    """grad_clock = NULL selects the adjoint without clock terms (its own arithmetic): the forward is the same bits,
    and the path and parameter gradients meet the same bar against the float64 checker."""
    B, L = 2, 700
    path, clock, dw = _inputs(B, L, seed=11)
    W = 1 + path.shape[2] + path.shape[2] ** 2
    g = (np.random.default_rng(5).normal(size=(B, L - 1, W)) / np.sqrt(W)).astype(np.float32)
    out1, dp1, _, dd1, _ = _run(path, clock, dw, g, clock_grad=True)
    out2, dp2, _, dd2, _ = _run(path, clock, dw, g, clock_grad=False)
    assert np.array_equal(out1, out2)
    rdp, _, rdd = C.planes_backward(path.astype(np.float64), clock.astype(np.float64), dw.astype(np.float64),
                                    g.astype(np.float64), kind="f64")
    errs = dict(dpath=relerr(dp2, rdp), dparams=relerr(dd2, rdd), dpath_vs_clock=relerr(dp2, dp1),
                dparams_vs_clock=relerr(dd2, dd1))
    print(errs)
    assert errs["dpath"] < 1e-4 and errs["dparams"] < 1e-4, errs
