"""The allocation-free forward (ews_diag_forward_noalloc) through the C ABI against ews_diag_forward on the same
inputs: bit-identical outputs on two calls in a row, the second with a smaller input (the scratch keeps the first
call's contents, which the second must not depend on), and the size limit reported as an error code without any
launch."""

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


def _both(path, clock, params, structure, readout, bf16=False):
    """(allocating forward, allocation-free forward) outputs for one input."""
    lib = nat.load()
    B, L, d = path.shape
    dt = nat.DTYPE_BF16 if bf16 else nat.DTYPE_F32
    desc = make_desc(B, L, d, 2, structure, nat.FLOW_PER_INTERVAL, readout, True, dt)
    W = 1 + d + d * d
    shape = (B, L - 1, W) if readout == "prefix" else (B, W)
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


def test_noalloc_forward_rejects_oversized_calls():
    """The c4 block shape at B = 256 needs more than the 64 MiB scratch: an error code, nothing launched (the
    pointers are never dereferenced on the host, and the check precedes every launch)."""
    lib = nat.load()
    desc = make_desc(256, 512, 32, 2, nat.STRUCT_REAL_DIAG, nat.FLOW_PER_INTERVAL, "prefix", True, nat.DTYPE_F32)
    buf = torch.empty(16, device=DEV)
    rc = lib.ews_diag_forward_noalloc(ctypes.byref(desc), buf.data_ptr(), buf.data_ptr(), buf.data_ptr(),
                                      buf.data_ptr(), _stream())
    assert rc == EWS_ERR_SCRATCH
    assert b"scratch" in lib.ews_error_string(rc)
