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


def _trunc(nodes, q):
    """Degree-<= q part of exp[nodes] in the nodes: the Taylor coefficients of s -> exp[s * nodes] at s = 0
    (50-digit Opitz, numerical Taylor expansion), summed at s = 1."""
    mpmath.mp.dps = 50
    f = lambda s: mpmath.mpc(_dd_exact_mp([s * a for a in nodes]))  # noqa: E731
    return complex(sum(mpmath.taylor(f, 0, q)))


def _dd_exact_mp(nodes):
    n = len(nodes)
    J = mpmath.zeros(n, n)
    for i, a in enumerate(nodes):
        J[i, i] = a
        if i + 1 < n:
            J[i, i + 1] = 1
    return mpmath.expm(J)[0, n - 1]


@pytest.mark.parametrize("q", [1, 4, 9])
def test_truncated_series_coefficients(shim, q):
    """node1q / dd3q (the series leaf's order-q coefficients on planes and diagonals) against the degree-<= q
    Taylor polynomials of the exact divided differences, at nodes of modulus up to 3 where the truncation shows;
    node derivatives are the degree-<= q-1 parts of exp[0,x,x], exp[0,x,x,y], exp[0,x,y,y]."""
    rng = np.random.default_rng(40 + q)
    n = 6
    x = _cases(rng, n, 3.0)
    y = (x + _cases(rng, n, 3.0)).astype(np.complex64)
    xf = np.ascontiguousarray(np.stack([x.real, x.imag], -1).astype(np.float32))
    yf = np.ascontiguousarray(np.stack([y.real, y.imag], -1).astype(np.float32))
    o1 = np.zeros((n, 6), np.float32)
    o2 = np.zeros((n, 6), np.float32)
    shim.shim_node1q_c(n, q, _ptr(xf), _ptr(o1))
    shim.shim_dd3q_c(n, q, _ptr(xf), _ptr(yf), _ptr(o2))
    g1 = o1[:, 0::2] + 1j * o1[:, 1::2]
    g2 = o2[:, 0::2] + 1j * o2[:, 1::2]
    visible = 0.0
    for i in range(n):
        xi, yi = complex(xf[i, 0], xf[i, 1]), complex(yf[i, 0], yf[i, 1])
        big = max(1.0, abs(xi), abs(yi)) ** q
        ref1 = [np.exp(xi), _trunc([0, xi], q), _trunc([0, xi, xi], q - 1)]
        ref2 = [_trunc([0, xi, yi], q), _trunc([0, xi, xi, yi], q - 1), _trunc([0, xi, yi, yi], q - 1)]
        for g, r in zip(g1[i], ref1):
            assert abs(g - r) <= 2e-6 * max(big, abs(np.exp(xi))), (q, i, xi, g, r)
        for g, r in zip(g2[i], ref2):
            assert abs(g - r) <= 2e-6 * big, (q, i, xi, yi, g, r)
        visible = max(visible, abs(ref2[0] - _dd_exact([0, xi, yi])) / abs(ref2[0]))
    assert visible > 1e-4  # the truncation shows at these nodes
