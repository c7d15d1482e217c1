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
