"""ctypes binding of the HIP library ``libews_mi355x.so`` (C ABI in include/ews_hip.h).

The library is the only compute path: if it is missing or fails to load, every call raises. There is no
CPU fallback.
"""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_NAME = "libews_mi355x.so"
LIB_PATH = os.path.join(_HERE, LIB_NAME)

EWS_OK = 0
STRUCT_PLANES = 1
STRUCT_REAL_DIAG = 2
FLOW_PER_INTERVAL = 0
FLOW_CACHED = 1
FLOW_CACHED_BASEPOINT = 2
READOUTS = {"prefix": 0, "terminal": 1, "mean": 2, "max": 3, "log_prefix": 4}  # log_prefix: diag scan only
CHUNK_SEQUENTIAL = -1  # ews_diag_desc.chunk: the per-sample sequential kernels
LEAF_SERIES = 0
LEAF_VAN_LOAN = 1
LEAF_BLOCK_SERIES = 2
DIAG_LEAVES = {"plane_closed": 0, "block_series": 1, "series": 2}
EXPM_SCHEMES = {"exact": 0, "euler": 1, "cayley": 2, "pade": 3}
DTYPE_F32 = 0
DTYPE_BF16 = 1

EXPORTED = (
    "ews_diag_workspace_bytes",
    "ews_diag_residual_bytes",
    "ews_diag_forward",
    "ews_diag_backward",
    "ews_diag_forward_pass",
    "ews_diag_backward_pass",
    "ews_diag_num_passes",
    "ews_diag_forward_noalloc",
    "ews_diag_forward_status",
    "ews_error_string",
    "ews_version",
    "ews_dense_workspace_bytes",
    "ews_dense_forward",
    "ews_dense_forward_pass",
    "ews_dense_num_passes",
    "ews_dense_local_terms",
    "ews_dense_combine",
    "ews_dense_backward_workspace_bytes",
    "ews_dense_combine_backward",
    "ews_dense_backward",
    "ews_dense_forward_keep",
    "ews_dense_backward_kept",
    "ews_log_dim",
    "ews_log_workspace_bytes",
    "ews_log_forward",
    "ews_log_backward",
    "ews_mixer_residual_bytes",
    "ews_mixer_forward",
    "ews_mixer_backward",
    "ews_mixer_backward_workspace_bytes",
    "ews_mixer_backward_weight",
    "ews_clock_residual_bytes",
    "ews_clock_workspace_bytes",
    "ews_clock_num_params",
    "ews_clock_forward",
    "ews_clock_backward",
    "ews_lift_residual_bytes",
    "ews_lift_workspace_bytes",
    "ews_lift_forward",
    "ews_lift_backward",
    "ews_dense_local_terms_backward",
    "ews_token_scan_workspace_bytes",
    "ews_token_scan",
    "ews_token_scan_backward",
    "ews_jordan_local_terms",
    "ews_jordan_workspace_bytes",
    "ews_jordan_local_terms_backward",
    "ews_chain_residual_bytes",
    "ews_chain_workspace_bytes",
    "ews_chain_forward",
    "ews_chain_backward",
    "ews_token1_workspace_bytes",
    "ews_token1_scan",
    "ews_token1_scan_backward",
    "ews_diag_mixer_forward",
    "ews_diag_uses_chunk_kernels",
)

JORDAN_KINDS = {"real": 0, "complex": 1}

CLOCK_MODES = {"time": 0, "blended_variation": 1, "blended_learn": 1, "blended_quad_variation": 2,
               "token_gated": 3, "clamped_gate": 4}
CLOCK_SCALINGS = {"none": 0, "[0,1]": 1, "[-1,1]": 2, "steps": 3}
LIFT_NONE = 0
LIFT_FULL = 1
LIFT_PRESERVE = 2

GRADED_VARIANTS = {"live_rms": 0, "static_gain": 1, "dilation": 2}


class DiagDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("structure", ctypes.c_int32),
        ("flow_mode", ctypes.c_int32),
        ("readout", ctypes.c_int32),
        ("level0", ctypes.c_int32),
        ("path_dtype", ctypes.c_int32),
        ("chunk", ctypes.c_int32),
        ("leaf", ctypes.c_int32),
        ("series_q", ctypes.c_int32),
    ]


class DenseDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("series_q", ctypes.c_int32),
        ("flow_mode", ctypes.c_int32),
        ("readout", ctypes.c_int32),
        ("level0", ctypes.c_int32),
        ("chunk", ctypes.c_int32),
        ("leaf", ctypes.c_int32),
        ("vl_steps", ctypes.c_int32),
        ("vl_expm", ctypes.c_int32),
        ("vl_mode", ctypes.c_int32),
        ("chen_expm", ctypes.c_int32),
    ]


class JordanDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("kind", ctypes.c_int32),
        ("size", ctypes.c_int32),
    ]


class ChainDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("kind", ctypes.c_int32),
        ("size", ctypes.c_int32),
        ("flow_mode", ctypes.c_int32),
        ("leaf_mode", ctypes.c_int32),
        ("readout", ctypes.c_int32),
        ("level0", ctypes.c_int32),
        ("series_q", ctypes.c_int32),
        ("chunk", ctypes.c_int32),
    ]


class Token1Desc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("steps", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("vocab", ctypes.c_int32),
        ("block", ctypes.c_int32),
    ]


class LogDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("level0", ctypes.c_int32),
        ("readout", ctypes.c_int32),
    ]


class MixerDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("rows", ctypes.c_int32),
        ("dim", ctypes.c_int32),
        ("depth", ctypes.c_int32),
        ("level0", ctypes.c_int32),
        ("hidden", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("prepend", ctypes.c_int32),
        ("prescale", ctypes.c_int32),
        ("eps", ctypes.c_float * 3),
    ]


class ClockDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("channels", ctypes.c_int32),
        ("mode", ctypes.c_int32),
        ("scaling", ctypes.c_int32),
        ("normalize", ctypes.c_int32),
        ("gates", ctypes.c_int32),
        ("has_mask", ctypes.c_int32),
        ("increment_driver", ctypes.c_int32),
        ("has_time_denominator", ctypes.c_int32),
        ("basepoint", ctypes.c_int32),
        ("learned_alpha", ctypes.c_int32),
        ("alpha", ctypes.c_float),
        ("norm_constant", ctypes.c_float),
        ("time_denominator", ctypes.c_float),
        ("variation_eps", ctypes.c_float),
        ("in_scale", ctypes.c_float),
    ]


class LiftDesc(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int32),
        ("length", ctypes.c_int32),
        ("branch_dim", ctypes.c_int32),
        ("append", ctypes.c_int32),
        ("out_dim", ctypes.c_int32),
        ("lift", ctypes.c_int32),
        ("increment", ctypes.c_int32),
        ("has_mask", ctypes.c_int32),
        ("basepoint", ctypes.c_int32),
    ]


class NativeLibraryError(RuntimeError):
    pass


_lib = None


def load():
    """Load the HIP library once; raise if it is absent (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950)"
        )
    lib = ctypes.CDLL(LIB_PATH)
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    dp = ctypes.POINTER(DiagDesc)
    lib.ews_diag_workspace_bytes.argtypes = [dp]
    lib.ews_diag_workspace_bytes.restype = sz
    lib.ews_diag_residual_bytes.argtypes = [dp]
    lib.ews_diag_residual_bytes.restype = sz
    lib.ews_diag_forward.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_diag_forward.restype = i32
    lib.ews_diag_backward.argtypes = [dp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_diag_backward.restype = i32
    lib.ews_diag_forward_pass.argtypes = [dp, i32, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_diag_forward_pass.restype = i32
    lib.ews_diag_backward_pass.argtypes = [dp, i32, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_diag_backward_pass.restype = i32
    lib.ews_diag_num_passes.argtypes = [i32]
    lib.ews_diag_num_passes.restype = i32
    lib.ews_diag_forward_noalloc.argtypes = [dp, vp, vp, vp, vp, vp]
    lib.ews_diag_forward_noalloc.restype = i32
    lib.ews_diag_forward_status.argtypes = [dp, vp, ctypes.POINTER(ctypes.c_int), vp]
    lib.ews_diag_forward_status.restype = i32
    lib.ews_error_string.argtypes = [i32]
    lib.ews_error_string.restype = ctypes.c_char_p
    lib.ews_version.argtypes = []
    lib.ews_version.restype = ctypes.c_char_p
    ddp = ctypes.POINTER(DenseDesc)
    lib.ews_dense_workspace_bytes.argtypes = [ddp]
    lib.ews_dense_workspace_bytes.restype = sz
    lib.ews_dense_forward.argtypes = [ddp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_forward.restype = i32
    lib.ews_dense_forward_pass.argtypes = [ddp, i32, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_forward_pass.restype = i32
    lib.ews_dense_num_passes.argtypes = []
    lib.ews_dense_num_passes.restype = i32
    lib.ews_dense_local_terms.argtypes = [ddp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_local_terms.restype = i32
    lib.ews_dense_combine.argtypes = [ddp, vp, vp, vp, vp, vp]
    lib.ews_dense_combine.restype = i32
    lib.ews_dense_backward_workspace_bytes.argtypes = [ddp]
    lib.ews_dense_backward_workspace_bytes.restype = sz
    lib.ews_dense_combine_backward.argtypes = [ddp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_combine_backward.restype = i32
    lib.ews_dense_backward.argtypes = [ddp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_backward.restype = i32
    lib.ews_dense_forward_keep.argtypes = [ddp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_forward_keep.restype = i32
    lib.ews_dense_backward_kept.argtypes = [ddp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_backward_kept.restype = i32
    ldp = ctypes.POINTER(LogDesc)
    lib.ews_log_dim.argtypes = [i32, i32]
    lib.ews_log_dim.restype = i32
    lib.ews_log_workspace_bytes.argtypes = [ldp]
    lib.ews_log_workspace_bytes.restype = sz
    lib.ews_log_forward.argtypes = [ldp, vp, vp, vp, vp]
    lib.ews_log_forward.restype = i32
    lib.ews_log_backward.argtypes = [ldp, vp, vp, vp, vp, vp]
    lib.ews_log_backward.restype = i32
    mdp = ctypes.POINTER(MixerDesc)
    lib.ews_mixer_residual_bytes.argtypes = [mdp]
    lib.ews_mixer_residual_bytes.restype = sz
    lib.ews_mixer_forward.argtypes = [mdp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_mixer_forward.restype = i32
    lib.ews_mixer_backward.argtypes = [mdp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_mixer_backward.restype = i32
    lib.ews_mixer_backward_workspace_bytes.argtypes = [mdp]
    lib.ews_mixer_backward_workspace_bytes.restype = ctypes.c_size_t
    lib.ews_mixer_backward_weight.argtypes = [mdp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_mixer_backward_weight.restype = i32
    lib.ews_dense_local_terms_backward.argtypes = [ddp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_dense_local_terms_backward.restype = i32
    lib.ews_token_scan_workspace_bytes.argtypes = [ddp, i32]
    lib.ews_token_scan_workspace_bytes.restype = sz
    lib.ews_token_scan.argtypes = [ddp, vp, vp, vp, vp, i32, vp, vp, vp]
    lib.ews_token_scan.restype = i32
    lib.ews_token_scan_backward.argtypes = [ddp, vp, vp, vp, vp, i32, vp, vp, vp, vp, vp]
    lib.ews_token_scan_backward.restype = i32
    cdp = ctypes.POINTER(ClockDesc)
    lib.ews_clock_residual_bytes.argtypes = [cdp]
    lib.ews_clock_residual_bytes.restype = sz
    lib.ews_clock_workspace_bytes.argtypes = [cdp]
    lib.ews_clock_workspace_bytes.restype = sz
    lib.ews_clock_num_params.argtypes = [cdp]
    lib.ews_clock_num_params.restype = i32
    lib.ews_clock_forward.argtypes = [cdp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_clock_forward.restype = i32
    lib.ews_clock_backward.argtypes = [cdp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_clock_backward.restype = i32
    ftp = ctypes.POINTER(LiftDesc)
    lib.ews_lift_residual_bytes.argtypes = [ftp]
    lib.ews_lift_residual_bytes.restype = sz
    lib.ews_lift_workspace_bytes.argtypes = [ftp]
    lib.ews_lift_workspace_bytes.restype = sz
    lib.ews_lift_forward.argtypes = [ftp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_lift_forward.restype = i32
    lib.ews_lift_backward.argtypes = [ftp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_lift_backward.restype = i32
    jdp = ctypes.POINTER(JordanDesc)
    lib.ews_jordan_local_terms.argtypes = [jdp, vp, vp, vp, vp, vp]
    lib.ews_jordan_local_terms.restype = i32
    lib.ews_jordan_workspace_bytes.argtypes = [jdp]
    lib.ews_jordan_workspace_bytes.restype = sz
    lib.ews_jordan_local_terms_backward.argtypes = [jdp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_jordan_local_terms_backward.restype = i32
    chp = ctypes.POINTER(ChainDesc)
    lib.ews_chain_residual_bytes.argtypes = [chp]
    lib.ews_chain_residual_bytes.restype = sz
    lib.ews_chain_workspace_bytes.argtypes = [chp]
    lib.ews_chain_workspace_bytes.restype = sz
    lib.ews_chain_forward.argtypes = [chp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_chain_forward.restype = i32
    lib.ews_chain_backward.argtypes = [chp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_chain_backward.restype = i32
    lib.ews_diag_mixer_forward.argtypes = [dp, ctypes.POINTER(MixerDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_diag_mixer_forward.restype = i32
    lib.ews_diag_uses_chunk_kernels.argtypes = [dp]
    lib.ews_diag_uses_chunk_kernels.restype = i32
    t1p = ctypes.POINTER(Token1Desc)
    lib.ews_token1_workspace_bytes.argtypes = [t1p]
    lib.ews_token1_workspace_bytes.restype = sz
    lib.ews_token1_scan.argtypes = [t1p, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_token1_scan.restype = i32
    lib.ews_token1_scan_backward.argtypes = [t1p, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.ews_token1_scan_backward.restype = i32
    _lib = lib
    return lib


def check(rc: int, what: str):
    if rc != EWS_OK:
        msg = load().ews_error_string(rc).decode()
        raise NativeLibraryError(f"{what} failed: {msg} (code {rc})")
