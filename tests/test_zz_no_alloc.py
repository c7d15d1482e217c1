"""The allocation-free forward (ews_diag_forward_noalloc) through the C ABI against ews_diag_forward on the same
inputs: bit-identical outputs on calls in a row, each later one using less scratch (the scratch keeps the previous
call's contents, which the next must not depend on), on the pair-group, generic and sequential kernels, and the size
limit reported as an error code without any launch."""

import ctypes

import numpy as np
import pytest
import torch

import bench
from ews_mi355x import _native as nat
from ews_mi355x.ops import make_desc

pytestmark = pytest.mark.gpu

DEV = "cuda"
EWS_ERR_SCRATCH = -6


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _both(path, clock, params, structure, readout, bf16=False, chunk=0):
    """(allocating forward, allocation-free forward) outputs for one input."""
    lib = nat.load()
    B, L, d = path.shape
    dt = nat.DTYPE_BF16 if bf16 else nat.DTYPE_F32
    desc = make_desc(B, L, d, 2, structure, nat.FLOW_PER_INTERVAL, readout, True, dt, chunk=chunk)
    W = d + d * (d - 1) // 2 if readout == "log_prefix" else 1 + d + d * d
    shape = (B, L - 1, W) if readout in ("prefix", "log_prefix") else (B, W)
    tp = torch.tensor(path, device=DEV)
    if bf16:
        tp = tp.to(torch.bfloat16)
    tc = torch.tensor(clock, device=DEV)
    tw = torch.tensor(params, device=DEV)
    ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    rs = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    ref = torch.full(shape, float("nan"), device=DEV)
    got = torch.full(shape, float("nan"), device=DEV)
    nat.check(lib.ews_diag_forward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), ref.data_ptr(),
                                   rs.data_ptr(), ws.data_ptr(), _stream()), "ews_diag_forward")
    nat.check(lib.ews_diag_forward_noalloc(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(),
                                           got.data_ptr(), _stream()), "ews_diag_forward_noalloc")
    torch.cuda.synchronize()
    return ref, got


def test_noalloc_forward_matches_allocating_forward_twice():
    # call 1: the c2 recipe at B = 4, L = 17,984 (pair-group kernels, quad carry scans)
    path, clock, dw = bench.make_inputs(B=4)
    print("noalloc call 1: c2 recipe B=4 L=17984 d=16 planes prefix", flush=True)
    ref, got = _both(path, clock, dw, nat.STRUCT_PLANES, "prefix")
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)
    # call 2, smaller: 12 planes with a bfloat16 path (generic kernels), then a real diagonal with the mean readout
    path, clock, dw = bench.c5_inputs(B=2, L=3001)
    print("noalloc call 2: c5 recipe B=2 L=3001 d=24 planes bf16 prefix", flush=True)
    ref, got = _both(path, clock, dw, nat.STRUCT_PLANES, "prefix", bf16=True)
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)
    path, clock, lam = bench.c1_inputs(B=3, L=515)
    print("noalloc call 3: c1 recipe B=3 L=515 d=8 real diagonal mean", flush=True)
    ref, got = _both(path, clock, lam, nat.STRUCT_REAL_DIAG, "mean")
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)
    # the per-sample sequential kernels (no checkpoints kept by the allocation-free call), LogEWS rows
    rng = np.random.default_rng(5)
    path = np.cumsum(rng.normal(size=(2, 300, 32)) / 8.0, 1).astype(np.float32)
    clock = np.broadcast_to(np.arange(300, dtype=np.float32), (2, 300)).copy()
    lam = rng.uniform(0.1, 2.0, size=32).astype(np.float32)
    print("noalloc call 4: sequential kernels B=2 L=300 d=32 real diagonal log_prefix", flush=True)
    ref, got = _both(path, clock, lam, nat.STRUCT_REAL_DIAG, "log_prefix", chunk=nat.CHUNK_SEQUENTIAL)
    assert torch.isfinite(ref).all()
    assert torch.equal(ref, got)


def test_noalloc_forward_rejects_oversized_calls():
    """The c4 block shape on the chunk kernels (chunk = 16: float64 chunk carries of 69 MB alone) needs more than the
    64 MiB scratch: an error code, nothing launched. The size is checked on the host through the library's own
    query before the call, and every buffer has the call's real size, so the call stays in bounds whatever the
    entry point decides."""
    lib = nat.load()
    B, L, d = 256, 512, 32
    desc = make_desc(B, L, d, 2, nat.STRUCT_REAL_DIAG, nat.FLOW_PER_INTERVAL, "prefix", True, nat.DTYPE_F32,
                     chunk=16)
    need = int(lib.ews_diag_residual_bytes(ctypes.byref(desc)))
    assert need > 64 << 20, need
    path = torch.zeros(B, L, d, device=DEV)
    clock = torch.arange(L, dtype=torch.float32, device=DEV).expand(B, L).contiguous()
    lam = torch.ones(d, device=DEV)
    out = torch.empty(B, L - 1, 1 + d + d * d, device=DEV)
    rc = lib.ews_diag_forward_noalloc(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), lam.data_ptr(),
                                      out.data_ptr(), _stream())
    torch.cuda.synchronize()
    assert rc == EWS_ERR_SCRATCH
    assert b"scratch" in lib.ews_error_string(rc)
