"""numpy restatement of the counter-based PRNG draws the reference's model init makes.

TEST INFRASTRUCTURE ONLY: the product path never imports anything under ``oracle/``.

The reference builds its pinned fixture model (``tests/test_kernel_outputs_pinned.py:21-74``, through
``experiments/uea/train.py:159-240`` and ``ews/params.py:1195-1217``) from ``jax.random.PRNGKey(0)``.
``jax`` is not installed here, so the draws are restated from the published algorithms:

* Threefry-2x32 with 20 rounds (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2, 3",
  SC'11), the block cipher behind JAX's default key;
* JAX's "partitionable" key split and bit generation (the default of the pinned ``jax==0.9.0``): element ``i``
  of a draw of shape ``s`` is the cipher applied to the 64-bit counter ``i`` split into (hi, lo) words;
* uniform floats from the top mantissa bits OR'ed into the exponent of 1.0, and normals as
  ``sqrt(2) * erfinv(u)`` with ``u`` uniform on ``(nextafter(-1, 0), 1)``.

``erfinv`` is evaluated in float64 and rounded, so a float32 normal may differ from XLA's own float32
``erf_inv`` by about one ulp; the init fixture ``reference_model_init.npz`` checks every draw used here.
"""

from __future__ import annotations

import numpy as np
from scipy.special import erfinv

_M32 = np.uint64(0xFFFFFFFF)
_ROT = ((13, 15, 26, 6), (17, 29, 16, 24))


def _rotl(x, r):
    x = x.astype(np.uint64)
    return (((x << np.uint64(r)) | (x >> np.uint64(32 - r))) & _M32).astype(np.uint64)


def threefry2x32(k0, k1, x0, x1):
    """Threefry-2x32, 20 rounds, on uint32 word arrays ``x0, x1`` under key ``(k0, k1)``."""
    k0 = np.uint64(k0)
    k1 = np.uint64(k1)
    k2 = np.uint64(int(k0) ^ int(k1) ^ 0x1BD11BDA)
    ks = (k0, k1, k2)
    x0 = (np.asarray(x0, np.uint64) + k0) & _M32
    x1 = (np.asarray(x1, np.uint64) + k1) & _M32
    for group in range(5):
        for r in _ROT[group % 2]:
            x0 = (x0 + x1) & _M32
            x1 = _rotl(x1, r)
            x1 = x1 ^ x0
        # key injection after every 4 rounds: words (ks[g+1], ks[g+2] + g + 1)
        x0 = (x0 + ks[(group + 1) % 3]) & _M32
        x1 = (x1 + ks[(group + 2) % 3] + np.uint64(group + 1)) & _M32
    return x0.astype(np.uint32), x1.astype(np.uint32)


def prng_key(seed: int):
    """``PRNGKey(seed)`` as two uint32 words (hi, lo)."""
    seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return (np.uint32(seed >> 32), np.uint32(seed & 0xFFFFFFFF))


def _counters(n):
    i = np.arange(n, dtype=np.uint64)
    return (i >> np.uint64(32)).astype(np.uint32), (i & _M32).astype(np.uint32)


def split(key, num=2):
    """Partitionable split: subkey ``i`` = cipher(key, counter i)."""
    hi, lo = _counters(num)
    b0, b1 = threefry2x32(key[0], key[1], hi, lo)
    return [(b0[i], b1[i]) for i in range(num)]


def random_bits(key, bit_width, shape):
    n = int(np.prod(shape)) if len(shape) else 1
    hi, lo = _counters(n)
    b0, b1 = threefry2x32(key[0], key[1], hi, lo)
    if bit_width == 32:
        return (b0 ^ b1).reshape(shape)
    if bit_width == 64:
        return ((b0.astype(np.uint64) << np.uint64(32)) | b1.astype(np.uint64)).reshape(shape)
    raise ValueError("bit_width must be 32 or 64")


def uniform(key, shape, dtype=np.float32, minval=0.0, maxval=1.0):
    dtype = np.dtype(dtype)
    if dtype == np.float32:
        bits = random_bits(key, 32, shape)
        fb = (bits >> np.uint32(32 - 23)) | np.float32(1.0).view(np.uint32)
        floats = fb.view(np.float32) - np.float32(1.0)
        lo, hi = np.float32(minval), np.float32(maxval)
        return np.maximum(lo, floats * (hi - lo) + lo).astype(np.float32)
    if dtype == np.float64:
        bits = random_bits(key, 64, shape)
        fb = (bits >> np.uint64(64 - 52)) | np.float64(1.0).view(np.uint64)
        floats = fb.view(np.float64) - 1.0
        return np.maximum(minval, floats * (maxval - minval) + minval)
    raise ValueError(dtype)


def normal(key, shape, dtype=np.float32):
    dtype = np.dtype(dtype)
    lo = np.nextafter(np.array(-1.0, dtype), np.array(0.0, dtype))
    u = uniform(key, shape, dtype, lo, 1.0)
    return (np.sqrt(2.0) * erfinv(u.astype(np.float64))).astype(dtype)
