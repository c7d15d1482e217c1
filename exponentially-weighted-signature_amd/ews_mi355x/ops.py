"""torch autograd binding of the diagonal / rotation-plane scan (forward + hand-written backward).

This is the torch-side analogue of the reference's ``jax.custom_vjp`` pair around its fused kernels
(ews/core/kernels/pallas_combine.py:1673-1801): the forward saves only the inputs and the float64
chunk-start states the library returns; the backward recomputes the rest inside the kernels.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat


def _stream_handle(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def make_desc(B, L, d, N, structure, flow_mode, readout, level0, path_dtype, chunk=0):
    return nat.DiagDesc(B, L, d, N, structure, flow_mode, nat.READOUTS[readout], int(level0), path_dtype,
                        int(chunk))


def _check_inputs(path, clock, params):
    if not path.is_cuda:
        raise RuntimeError("ews_mi355x runs on a HIP device only: move path/clock/A to the GPU (no CPU path)")
    if path.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"path dtype must be float32 or bfloat16, got {path.dtype}")
    if clock.dtype != torch.float32 or params.dtype != torch.float32:
        raise TypeError("clock and A must be float32")


class DiagScan(torch.autograd.Function):
    """out = EWS readout of (path, clock) under a diagonal / rotation-plane generator with parameters
    ``params`` ((d/2, 2) rows (d_j, w_j) for planes, (d,) for a real diagonal)."""

    @staticmethod
    def forward(ctx, path, clock, params, N, structure, flow_mode, readout, level0, chunk):
        lib = nat.load()
        _check_inputs(path, clock, params)
        path = path.contiguous()
        clock = clock.contiguous()
        params = params.contiguous()
        B, L, d = path.shape
        dt = nat.DTYPE_BF16 if path.dtype == torch.bfloat16 else nat.DTYPE_F32
        desc = make_desc(B, L, d, N, structure, flow_mode, readout, level0, dt, chunk)
        D = d + (d * d if N == 2 else 0)
        W = D + (1 if level0 else 0)
        shape = (B, L - 1, W) if readout == "prefix" else (B, W)
        dev = path.device
        out = torch.empty(shape, device=dev, dtype=torch.float32)
        resid = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        rc = lib.ews_diag_forward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), params.data_ptr(),
                                  out.data_ptr(), resid.data_ptr(), ws.data_ptr(), _stream_handle(dev))
        nat.check(rc, "ews_diag_forward")
        ctx.save_for_backward(path, clock, params, resid)
        ctx.desc = (B, L, d, N, structure, flow_mode, readout, level0, dt, chunk)
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, params, resid = ctx.saved_tensors
        B, L, d, N, structure, flow_mode, readout, level0, dt, chunk = ctx.desc
        desc = make_desc(B, L, d, N, structure, flow_mode, readout, level0, dt, chunk)
        gout = gout.contiguous().to(torch.float32)
        dev = path.device
        dpath = torch.empty((B, L, d), device=dev, dtype=torch.float32)
        dclock = torch.empty((B, L), device=dev, dtype=torch.float32)
        dparams = torch.empty_like(params)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        rc = lib.ews_diag_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), params.data_ptr(),
                                   resid.data_ptr(), gout.data_ptr(), dpath.data_ptr(), dclock.data_ptr(),
                                   dparams.data_ptr(), ws.data_ptr(), _stream_handle(dev))
        nat.check(rc, "ews_diag_backward")
        return dpath.to(path.dtype), dclock, dparams, None, None, None, None, None, None


def diag_scan(path, clock, params, N, structure, flow_mode="per_interval", readout="prefix", level0=True,
              chunk=0):
    fm = {"per_interval": nat.FLOW_PER_INTERVAL, "cached": nat.FLOW_CACHED,
          "cached_basepoint": nat.FLOW_CACHED_BASEPOINT}[flow_mode]
    st = {"planes": nat.STRUCT_PLANES, "real_diag": nat.STRUCT_REAL_DIAG}[structure]
    return DiagScan.apply(path, clock, params, int(N), st, fm, readout, bool(level0), int(chunk))
