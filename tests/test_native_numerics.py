"""The kernels' scalar coefficient numerics (csrc/ews_numerics.h), built for the host with g++ and checked
against divided differences of exp computed independently at 50 digits with mpmath: the Opitz formula,
exp of the upper-bidiagonal matrix with the nodes on the diagonal holds exp[a_i..a_j] in entry (i, j).
The float32 bar is a few ulp relative to the largest term of each quantity."""

import ctypes
import os
import subprocess

import mpmath
import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "exponentially-weighted-signature_amd", "csrc")


@pytest.fixture(scope="module")
def shim(tmp_path_factory):
    out = tmp_path_factory.mktemp("shim") / "libnumshim.so"
    subprocess.check_call(["g++", "-O2", "-shared", "-fPIC", "-I", CSRC, "-o", str(out),
                           os.path.join(HERE, "native", "numerics_shim.cpp")])
    return ctypes.CDLL(str(out))


def _dd_exact(nodes):
    """exp[nodes] by Opitz: exp of the bidiagonal matrix, entry (0, n)."""
    mpmath.mp.dps = 50
    n = len(nodes)
    J = mpmath.zeros(n, n)
    for i, a in enumerate(nodes):
        J[i, i] = a
        if i + 1 < n:
            J[i, i + 1] = 1
    return complex(mpmath.expm(J)[0, n - 1])


def _ptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _cases(rng, n, scale):
    r = rng.uniform(0, scale, n) * np.exp(1j * rng.uniform(0, 2 * np.pi, n))
    return r.astype(np.complex64)


@pytest.mark.parametrize("scale", [1e-4, 0.3, 0.9, 1.7, 6.0])
def test_complex_dd3_matches_opitz(shim, scale):
    rng = np.random.default_rng(int(scale * 1000))
    n = 40
    x = _cases(rng, n, scale)
    # y = x + x' as the kernels form it (pairs of plane nodes), plus near-coincident nodes
    y = (x + _cases(rng, n, scale)).astype(np.complex64)
    y[: n // 4] = (x[: n // 4] * (1 + 1e-3)).astype(np.complex64)
    xf = np.ascontiguousarray(np.stack([x.real, x.imag], -1).astype(np.float32))
    yf = np.ascontiguousarray(np.stack([y.real, y.imag], -1).astype(np.float32))
    out = np.zeros((n, 6), np.float32)
    shim.shim_dd3_c(n, _ptr(xf), _ptr(yf), _ptr(out))
    got = out[:, 0::2] + 1j * out[:, 1::2]
    for i in range(n):
        xi, yi = complex(xf[i, 0], xf[i, 1]), complex(yf[i, 0], yf[i, 1])
        ref = [_dd_exact([0, xi, yi]), _dd_exact([0, xi, xi, yi]), _dd_exact([0, xi, yi, yi])]
        big = max(1.0, abs(np.exp(xi)), abs(np.exp(yi)))  # largest term the quantity is built from
        for g, r in zip(got[i], ref):
            assert abs(g - r) <= 5e-7 * big, (scale, i, xi, yi, g, r)


@pytest.mark.parametrize("scale", [1e-3, 0.5, 3.0])
def test_complex_node1_matches_opitz(shim, scale):
    rng = np.random.default_rng(7)
    n = 30
    x = _cases(rng, n, scale)
    xf = np.ascontiguousarray(np.stack([x.real, x.imag], -1).astype(np.float32))
    out = np.zeros((n, 6), np.float32)
    shim.shim_node1_c(n, _ptr(xf), _ptr(out))
    got = out[:, 0::2] + 1j * out[:, 1::2]
    for i in range(n):
        xi = complex(xf[i, 0], xf[i, 1])
        ref = [np.exp(xi), _dd_exact([0, xi]), _dd_exact([0, xi, xi])]
        big = max(1.0, abs(np.exp(xi)))
        for g, r in zip(got[i], ref):
            assert abs(g - r) <= 5e-7 * big, (i, xi, g, r)


def test_real_dd3_matches_opitz(shim):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.uniform(-1, 1, 20) * 1e-3, rng.uniform(-3, 3, 20), rng.uniform(-12, 2, 20)])
    y = x + np.concatenate([rng.uniform(-1, 1, 20) * 1e-3, rng.uniform(-3, 3, 20), rng.uniform(-12, 2, 20)])
    x = x.astype(np.float32)
    y = y.astype(np.float32)
    out = np.zeros((len(x), 3), np.float32)
    shim.shim_dd3_r(len(x), _ptr(x), _ptr(y), _ptr(out))
    for i in range(len(x)):
        xi, yi = float(x[i]), float(y[i])
        ref = [_dd_exact([0, xi, yi]).real, _dd_exact([0, xi, xi, yi]).real, _dd_exact([0, xi, yi, yi]).real]
        big = max(1.0, np.exp(xi), np.exp(yi))
        for g, r in zip(out[i], ref):
            assert abs(g - r) <= 5e-7 * big, (i, xi, yi, g, r)
