"""GPU parity at the BASELINE.json configurations' own shapes (not reduced ones), against the float64 checkers.

* c5: B = 2 of the 8 samples at the full L = 49,920, d = 24 (12 rotation planes), bfloat16 path with
  float32 state, forward and backward, against the float64 C checker (oracle/cpu_scan.c, pinned to the torch
  oracle by tests/test_oracle_cscan.py) on the same bfloat16 inputs upcast. The long-L float32 error budget is
  the hard part here: the state is a nearly undiscounted 50k-term sum.
* c1: B = 8, L = 1,024, d = 8 real diagonal, the whole batch forward (c1's pass), gradients on two
  samples, against the float64 torch oracle.
* c4: B = 2 of 256 at L = 512, d = 32 real diagonal at unit clock steps, EWS rows and the LogEWS
  readout, forward and gradients, against the float64 torch oracle.

* c3: the whole batch B = 16 at L = 4,096, dense d = 16 generator, depth 3, input-dependent clock,
  forward with the series leaf (q = 24, the bench's) and with the Van Loan leaf (M = 20, cayley: the reference's
  default) on four samples; gradients of path, clock and A (series leaf) on one sample at the full L, against the
  float64 torch oracle and its autograd.

Inputs are the bench's own recipes (bench.py c1_inputs / c3_inputs / c4_inputs / c5_inputs). Bars (BASELINE.json north
star): forward max relative error <= 1e-5, gradients <= 1e-4, metric max|a-b| / max|b|.
"""

import ctypes

import numpy as np
import pytest
import torch

import bench
from ews_mi355x import _native as nat
from ews_mi355x import ops
from ews_mi355x.ops import make_desc
from oracle import cbuild
from oracle import cpu_scan_py as C
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def test_c5_full_length_bf16():
    cbuild.build(verbose=False)
    path, clock, dw = bench.c5_inputs(B=2)
    B, L, d = path.shape
    assert (L, d) == (49920, 24)
    W = 1 + d + d * d
    lib = nat.load()
    desc = make_desc(B, L, d, 2, nat.STRUCT_PLANES, nat.FLOW_PER_INTERVAL, "prefix", True, nat.DTYPE_BF16)
    tp = torch.tensor(path, device=DEV).to(torch.bfloat16)
    src = tp.double().cpu().numpy()  # the same bfloat16 inputs, upcast for the checker
    tc = torch.tensor(clock, device=DEV)
    tw = torch.tensor(dw, device=DEV)
    g = (np.random.default_rng(5).normal(size=(B, L - 1, W)) / np.sqrt(W)).astype(np.float32)
    tg = torch.tensor(g, device=DEV)
    ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    rs = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=DEV, dtype=torch.uint8)
    out = torch.empty((B, L - 1, W), device=DEV)
    dpath = torch.empty((B, L, d), device=DEV)
    dclock = torch.empty((B, L), device=DEV)
    ddw = torch.empty_like(tw)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    print(f"c5 full length: B={B} L={L} d={d} bf16", flush=True)
    nat.check(lib.ews_diag_forward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), out.data_ptr(),
                                   rs.data_ptr(), ws.data_ptr(), st), "forward")
    nat.check(lib.ews_diag_backward(ctypes.byref(desc), tp.data_ptr(), tc.data_ptr(), tw.data_ptr(), rs.data_ptr(),
                                    tg.data_ptr(), dpath.data_ptr(), dclock.data_ptr(), ddw.data_ptr(),
                                    ws.data_ptr(), st), "backward")
    torch.cuda.synchronize()
    ref = C.planes_forward(src, clock.astype(np.float64), dw.astype(np.float64), kind="f64")
    rdp, rdc, rdd = C.planes_backward(src, clock.astype(np.float64), dw.astype(np.float64), g.astype(np.float64),
                                      kind="f64")
    errs = dict(fwd=relerr(out, ref), dpath=relerr(dpath, rdp), dclock=relerr(dclock, rdc),
                dparams=relerr(ddw, rdd))
    # each level on its own scale as well (stricter than the reference's whole-row metric): level 1 is about 100x
    # smaller than level 2 here, so its own scale shows the float32 rounding of the long sum more
    o = out.cpu().numpy()
    errs["fwd_level1"] = relerr(o[..., 1:1 + d], ref[..., 1:1 + d])
    errs["fwd_level2"] = relerr(o[..., 1 + d:], ref[..., 1 + d:])
    print(f"c5 full length errors: {errs}", flush=True)
    assert errs["fwd"] < 1e-5, errs
    assert errs["fwd_level1"] < 1e-4 and errs["fwd_level2"] < 1e-5, errs
    assert errs["dpath"] < 1e-4 and errs["dclock"] < 1e-4 and errs["dparams"] < 1e-4, errs


def test_c1_exact_shape():
    path, clock, lam = bench.c1_inputs()
    B, L, d = path.shape
    assert (B, L, d) == (8, 1024, 8)
    tp = torch.tensor(path, device=DEV)
    tc = torch.tensor(clock, device=DEV)
    tl = torch.tensor(lam, device=DEV)
    out = ops.diag_scan(tp, tc, tl, 2, "real_diag", "per_interval", "prefix", True)
    A = torch.diag(torch.tensor(lam, dtype=torch.float64))
    ref = O.ews(torch.tensor(path, dtype=torch.float64), torch.tensor(clock, dtype=torch.float64), A, 2, "prefix",
                leaf="diag_closed")
    e = relerr(out, ref)
    print(f"c1 exact shape: forward relerr {e:.2e}", flush=True)
    assert e < 1e-5, e
    # gradients of two samples (path, clock, diagonal)
    p = tp[:2].clone().requires_grad_(True)
    c = tc[:2].clone().requires_grad_(True)
    lg = tl.clone().requires_grad_(True)
    o2 = ops.diag_scan(p, c, lg, 2, "real_diag", "per_interval", "prefix", True)
    w = torch.tensor(np.random.default_rng(1).normal(size=tuple(o2.shape)))
    (o2 * w.to(DEV, torch.float32)).sum().backward()
    pr = torch.tensor(path[:2], dtype=torch.float64, requires_grad=True)
    cr = torch.tensor(clock[:2], dtype=torch.float64, requires_grad=True)
    lr = torch.tensor(lam, dtype=torch.float64, requires_grad=True)
    r2 = O.ews(pr, cr, torch.diag(lr), 2, "prefix", leaf="diag_closed")
    (r2 * w).sum().backward()
    errs = (relerr(p.grad, pr.grad), relerr(c.grad, cr.grad), relerr(lg.grad, lr.grad))
    print(f"c1 exact shape: gradient relerrs {errs}", flush=True)
    assert max(errs) < 1e-4, errs


def test_c4_block_shape_with_log():
    path, clock, lam = bench.c4_inputs(B=2)
    B, L, d = path.shape
    assert (L, d) == (512, 32)
    p = torch.tensor(path, device=DEV).requires_grad_(True)
    c = torch.tensor(clock, device=DEV).requires_grad_(True)
    lg = torch.tensor(lam, device=DEV).requires_grad_(True)
    rows = ops.diag_scan(p, c, lg, 2, "real_diag", "per_interval", "prefix", True)
    logs = ops.log_rows(rows, d, 2, True, "prefix")
    pr = torch.tensor(path, dtype=torch.float64, requires_grad=True)
    cr = torch.tensor(clock, dtype=torch.float64, requires_grad=True)
    lr = torch.tensor(lam, dtype=torch.float64, requires_grad=True)
    A = torch.diag(lr)
    rref = O.ews(pr, cr, A, 2, "prefix", leaf="diag_closed")
    lref = torch.stack([O.log_ews_single(pr[b], cr[b], A, 2, "prefix", leaf="diag_closed") for b in range(B)])
    e_rows, e_log = relerr(rows, rref), relerr(logs, lref)
    print(f"c4 block shape: rows relerr {e_rows:.2e}, log relerr {e_log:.2e}", flush=True)
    assert e_rows < 1e-5 and e_log < 1e-5, (e_rows, e_log)
    w = torch.tensor(np.random.default_rng(2).normal(size=tuple(lref.shape)))
    (logs * w.to(DEV, torch.float32)).sum().backward()
    (lref * w).sum().backward()
    errs = (relerr(p.grad, pr.grad), relerr(c.grad, cr.grad), relerr(lg.grad, lr.grad))
    print(f"c4 block shape: gradient relerrs {errs}", flush=True)
    assert max(errs) < 1e-4, errs


def test_c3_exact_shape():
    path, clock, A = bench.c3_inputs()
    B, L, d = path.shape
    assert (B, L, d) == (16, 4096, 16)
    tp, tc, tA = (torch.tensor(x, device=DEV) for x in (path, clock, A))
    p64, c64, A64 = (torch.tensor(x, dtype=torch.float64) for x in (path, clock, A))
    out = ops.dense_scan(tp, tc, tA, 3, 24)
    ref = O.ews(p64, c64, A64, 3, "prefix", leaf="series", series_q=24)
    e = relerr(out, ref)
    print(f"c3 exact shape, series leaf q=24: forward relerr {e:.2e}", flush=True)
    assert e < 1e-5, e
    del out, ref
    vl = ops.DenseLeaf("van_loan", 0, M=20, van_loan_expm="cayley")
    out = ops.dense_scan(tp[:4], tc[:4], tA, 3, 0, leaf=vl)
    ref = O.ews(p64[:4], c64[:4], A64, 3, "prefix", leaf="van_loan", M=20, van_loan_expm="cayley")
    e = relerr(out, ref)
    print(f"c3 exact shape, Van Loan leaf M=20: forward relerr {e:.2e}", flush=True)
    assert e < 1e-5, e
    del out, ref
    # gradients of one sample at the full length (series leaf)
    pr, cr, Ar = (x.clone().requires_grad_(True) for x in (p64[:1], c64[:1], A64))
    r1 = O.ews(pr, cr, Ar, 3, "prefix", leaf="series", series_q=24)
    w = torch.tensor(np.random.default_rng(3).normal(size=tuple(r1.shape)))
    ref_g = torch.autograd.grad(r1, (pr, cr, Ar), w)
    pg, cg, Ag = (x.clone().requires_grad_(True) for x in (tp[:1], tc[:1], tA))
    o1 = ops.dense_scan(pg, cg, Ag, 3, 24)
    got = torch.autograd.grad(o1, (pg, cg, Ag), w.to(DEV, torch.float32))
    errs = tuple(relerr(g, r) for g, r in zip(got, ref_g))
    print(f"c3 exact shape: gradient relerrs (path, clock, A) {errs}", flush=True)
    assert max(errs) < 1e-4, errs
