"""GPU parity of the headline configuration at its exact shape (B = 32, L = 17,984,
8 rotation planes, d = 16, depth 2, prefix readout, uniform float32 clock), the inputs `bench.py` times.

Every one of the 32 samples' forward rows, the path, clock and plane-parameter gradients are checked against the
float64 C checker (oracle/cpu_scan.c, pinned to the torch oracle by tests/test_oracle_cscan.py), for both backward
variants: the split adjoint without the clock gradient (a null grad_clock, the one the bench times) and the
adjoint with it. At this shape the one-launch look-back forward runs 2,272 quads at full occupancy across the
XCDs; a stale or missing aggregate would give wrong carries, so the forward's status word is read back as well
(a timeout of a look-back wait would set it). Bars: forward <= 1e-5, gradients <= 1e-4 (max|a-b| / max|b|).
"""

import ctypes

import numpy as np
import pytest
import torch

from ews_mi355x import _native as nat
from ews_mi355x.ops import make_desc
from oracle import cbuild
from oracle import cpu_scan_py as C

import bench

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _built():
    cbuild.build(verbose=False)


def relerr(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


@pytest.fixture(scope="module")
def headline():
    path, clock, dw = bench.make_inputs()  # B = 32, L = 17,984
    B, L, d = path.shape
    W = 1 + d + d * d
    g = (np.random.default_rng([2, 9]).normal(size=(B, L - 1, W)) / np.sqrt(W)).astype(np.float32)
    lib = nat.load()
    desc = make_desc(B, L, d, 2, nat.STRUCT_PLANES, nat.FLOW_PER_INTERVAL, "prefix", True, nat.DTYPE_F32)
    tp, tc, tw = (torch.tensor(x, device=DEV) for x in (path, clock, dw))
    tg = torch.tensor(g, device=DEV)
    ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    rs = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    out = torch.empty((B, L - 1, W), device=DEV)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"headline forward B={B} L={L}", flush=True)
    nat.check(lib.ews_diag_forward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), out.data_ptr(),
                                   rs.data_ptr(), ws.data_ptr(), st), "forward")
    status = ctypes.c_int(-1)
    nat.check(lib.ews_diag_forward_status(ctypes.byref(desc), rs.data_ptr(), ctypes.byref(status), st), "status")
    grads = {}
    for clock_grad in (False, True):
        print(f"headline backward clock_grad={clock_grad}", flush=True)
        dpath = torch.empty((B, L, d), device=DEV)
        dclock = torch.empty((B, L), device=DEV)
        ddw = torch.empty_like(tw)
        nat.check(lib.ews_diag_backward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(),
                                        rs.data_ptr(), tg.data_ptr(), dpath.data_ptr(),
                                        dclock.data_ptr() if clock_grad else None, ddw.data_ptr(), ws.data_ptr(), st),
                  "backward")
        torch.cuda.synchronize()
        grads[clock_grad] = (dpath.cpu().numpy(), dclock.cpu().numpy() if clock_grad else None, ddw.cpu().numpy())
    print("headline float64 checker", flush=True)
    p64, c64, w64 = path.astype(np.float64), clock.astype(np.float64), dw.astype(np.float64)
    ref = C.planes_forward(p64, c64, w64, kind="f64")
    rdp, rdc, rdd = C.planes_backward(p64, c64, w64, g.astype(np.float64), kind="f64")
    return dict(out=out.cpu().numpy(), status=status.value, grads=grads, ref=ref, rdp=rdp, rdc=rdc, rdd=rdd)


def test_headline_forward_every_sample(headline):
    out, ref = headline["out"], headline["ref"]
    assert headline["status"] == 0, "a look-back wait gave up (status word set)"
    assert np.isfinite(out).all()
    per_sample = [relerr(out[b], ref[b]) for b in range(out.shape[0])]
    print(f"forward relerr: whole {relerr(out, ref):.2e}, worst sample {max(per_sample):.2e}", flush=True)
    assert max(per_sample) < 1e-5, per_sample
    # the carries of the last quads fold every earlier group aggregate: check the last rows on their own scale
    assert relerr(out[:, -256:], ref[:, -256:]) < 1e-5


@pytest.mark.parametrize("clock_grad", [False, True], ids=["split_adjoint", "with_clock_grad"])
def test_headline_gradients(headline, clock_grad):
    dp, dc, dd = headline["grads"][clock_grad]
    assert np.isfinite(dp).all() and np.isfinite(dd).all()
    errs = dict(dpath=relerr(dp, headline["rdp"]), dparams=relerr(dd, headline["rdd"]),
                dpath_worst_sample=max(relerr(dp[b], headline["rdp"][b]) for b in range(dp.shape[0])))
    if clock_grad:
        assert np.isfinite(dc).all()
        errs["dclock"] = relerr(dc, headline["rdc"])
    print(f"clock_grad={clock_grad}: {errs}", flush=True)
    assert all(v < 1e-4 for v in errs.values()), errs
