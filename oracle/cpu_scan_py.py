"""ctypes wrapper of oracle/cpu_scan.c (test infrastructure: the float64 checker and the CPU baseline)."""

from __future__ import annotations

import ctypes

import numpy as np

from . import cbuild

_libs = {}


def _lib(kind):
    if kind not in _libs:
        path = cbuild.lib_path(kind)
        lib = ctypes.CDLL(path)
        p = ctypes.c_void_p
        lib.cpu_planes_forward.argtypes = [ctypes.c_int] * 4 + [p, p, p, p]
        lib.cpu_planes_backward.argtypes = [ctypes.c_int] * 4 + [p] * 7
        _libs[kind] = lib
    return _libs[kind]


FLOW = {"per_interval": 0, "cached": 1, "cached_basepoint": 2}


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def planes_forward(path, clock, dw, flow_mode="per_interval", kind="f64"):
    """path (B, L, m), clock (B, L), dw (m/2, 2) -> prefix rows (B, L-1, 1 + m + m^2)."""
    dt = np.float64 if kind == "f64" else np.float32
    path = np.ascontiguousarray(path, dt)
    clock = np.ascontiguousarray(clock, dt)
    dw = np.ascontiguousarray(dw, dt)
    B, L, m = path.shape
    out = np.empty((B, L - 1, 1 + m + m * m), dt)
    _lib(kind).cpu_planes_forward(B, L, m, FLOW[flow_mode], _ptr(path), _ptr(clock), _ptr(dw), _ptr(out))
    return out


def planes_backward(path, clock, dw, gout, flow_mode="per_interval", kind="f64"):
    dt = np.float64 if kind == "f64" else np.float32
    path = np.ascontiguousarray(path, dt)
    clock = np.ascontiguousarray(clock, dt)
    dw = np.ascontiguousarray(dw, dt)
    gout = np.ascontiguousarray(gout, dt)
    B, L, m = path.shape
    dpath = np.empty_like(path)
    dclock = np.empty_like(clock)
    ddw = np.empty_like(dw)
    _lib(kind).cpu_planes_backward(B, L, m, FLOW[flow_mode], _ptr(path), _ptr(clock), _ptr(dw), _ptr(gout),
                                   _ptr(dpath), _ptr(dclock), _ptr(ddw))
    return dpath, dclock, ddw
