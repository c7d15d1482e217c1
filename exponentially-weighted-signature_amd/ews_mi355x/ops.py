"""torch autograd binding of the diagonal / rotation-plane scan (forward + hand-written backward).

This is the torch-side analogue of the reference's ``jax.custom_vjp`` pair around its fused kernels
(ews/core/kernels/pallas_combine.py:1673-1801): the forward saves only the inputs and the float64
chunk-start states the library returns; the backward recomputes the rest inside the kernels.
"""

from __future__ import annotations

import ctypes
import os

import torch

from . import _native as nat


def _stream_handle(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def make_desc(B, L, d, N, structure, flow_mode, readout, level0, path_dtype, chunk=0, leaf=0, series_q=0):
    """leaf: 0 exact closed forms ("plane_closed"), 1 "block_series", 2 "series" (nat.DIAG_LEAVES); series_q: the
    series order of the series leaves."""
    return nat.DiagDesc(B, L, d, N, structure, flow_mode, nat.READOUTS[readout], int(level0), path_dtype,
                        int(chunk), int(leaf), int(series_q))


def _check_inputs(path, clock, params):
    if not path.is_cuda:
        raise RuntimeError("ews_mi355x runs on a HIP device only: move path/clock/A to the GPU (no CPU path)")
    if path.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError(f"path dtype must be float32 or bfloat16, got {path.dtype}")
    if clock.dtype != torch.float32 or params.dtype != torch.float32:
        raise TypeError("clock and A must be float32")


def _aligned(x):
    """The kernels read knot rows with 16-byte vector loads: copy a view whose data is not 16-byte aligned."""
    return x if x.data_ptr() % 16 == 0 else x.clone()


class DiagScan(torch.autograd.Function):
    """out = EWS readout of (path, clock) under a diagonal / rotation-plane generator with parameters
    ``params`` ((d/2, 2) rows (d_j, w_j) for planes, (d,) for a real diagonal)."""

    @staticmethod
    def forward(ctx, path, clock, params, N, structure, flow_mode, readout, level0, chunk, leaf, series_q):
        lib = nat.load()
        _check_inputs(path, clock, params)
        path = _aligned(path.contiguous())
        clock = clock.contiguous()
        params = params.contiguous()
        B, L, d = path.shape
        dt = nat.DTYPE_BF16 if path.dtype == torch.bfloat16 else nat.DTYPE_F32
        desc = make_desc(B, L, d, N, structure, flow_mode, readout, level0, dt, chunk, leaf, series_q)
        D = d + (d * d if N == 2 else 0)
        W = D + (1 if level0 else 0)
        if readout == "log_prefix":  # LogEWS rows: level 1 and the Lyndon coefficients of level 2, no level 0
            W = d + d * (d - 1) // 2
        shape = (B, L - 1, W) if readout in ("prefix", "log_prefix") else (B, W)
        dev = path.device
        out = torch.empty(shape, device=dev, dtype=torch.float32)
        resid = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        rc = lib.ews_diag_forward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), params.data_ptr(),
                                  out.data_ptr(), resid.data_ptr(), ws.data_ptr(), _stream_handle(dev))
        nat.check(rc, "ews_diag_forward")
        ctx.save_for_backward(path, clock, params, resid)
        ctx.desc = (B, L, d, N, structure, flow_mode, readout, level0, dt, chunk, leaf, series_q)
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, params, resid = ctx.saved_tensors
        B, L, d, N, structure, flow_mode, readout, level0, dt, chunk, leaf, series_q = ctx.desc
        desc = make_desc(B, L, d, N, structure, flow_mode, readout, level0, dt, chunk, leaf, series_q)
        gout = gout.contiguous().to(torch.float32)
        dev = path.device
        dpath = torch.empty((B, L, d), device=dev, dtype=torch.float32)
        # the clock gradient is computed only when the clock requires it (a null pointer skips its terms)
        dclock = torch.empty((B, L), device=dev, dtype=torch.float32) if ctx.needs_input_grad[1] else None
        dparams = torch.empty_like(params)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        rc = lib.ews_diag_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), params.data_ptr(),
                                   resid.data_ptr(), gout.data_ptr(), dpath.data_ptr(),
                                   dclock.data_ptr() if dclock is not None else None, dparams.data_ptr(),
                                   ws.data_ptr(), _stream_handle(dev))
        nat.check(rc, "ews_diag_backward")
        return dpath.to(path.dtype), dclock, dparams, None, None, None, None, None, None, None, None


def diag_scan(path, clock, params, N, structure, flow_mode="per_interval", readout="prefix", level0=True,
              chunk=0, leaf="plane_closed", series_q=0):
    """leaf "plane_closed" (exact closed forms, for planes and real diagonals alike), "block_series" (exact level 1,
    the order-series_q series at level 2) or "series" (the order-series_q series at every level). readout
    "log_prefix" (depth 2) returns the LogEWS prefix rows straight from the scan's output pass; chunk
    nat.CHUNK_SEQUENTIAL asks for the per-sample sequential kernels (real diagonal, d <= 32, per-interval flows)."""
    fm = {"per_interval": nat.FLOW_PER_INTERVAL, "cached": nat.FLOW_CACHED,
          "cached_basepoint": nat.FLOW_CACHED_BASEPOINT}[flow_mode]
    st = {"planes": nat.STRUCT_PLANES, "real_diag": nat.STRUCT_REAL_DIAG}[structure]
    return DiagScan.apply(path, clock, params, int(N), st, fm, readout, bool(level0), int(chunk),
                          nat.DIAG_LEAVES[leaf], int(series_q or 0))


# ---------------------------------------------------------------------------------------------- dense generators
_FLOW_MODES = {"per_interval": nat.FLOW_PER_INTERVAL, "cached": nat.FLOW_CACHED,
               "cached_basepoint": nat.FLOW_CACHED_BASEPOINT}


_VL_MODES = {"displacement": nat.FLOW_PER_INTERVAL, "displacement_uniform": nat.FLOW_CACHED,
             "displacement_uniform_basepoint": nat.FLOW_CACHED_BASEPOINT}


class DenseLeaf:
    """Leaf options of the dense path (ews/core/leaf.py:50-198): the series leaf of order q, the block-series leaf
    (the exact level 1 at any step and the order-q series at level 2), or the Van Loan leaf with M knots per
    interval, its exponential scheme and its reweighting mode; chen_expm is the flows' scheme."""

    def __init__(self, kind="series", q=0, M=20, van_loan_expm="cayley", reweighting_mode="displacement",
                 chen_expm="exact"):
        if kind not in ("series", "van_loan", "block_series"):
            raise ValueError(f"dense leaf must be 'series', 'block_series' or 'van_loan', got {kind!r}")
        if reweighting_mode not in _VL_MODES:
            raise ValueError(
                "reweighting_mode must be 'displacement', 'displacement_uniform', or "
                f"'displacement_uniform_basepoint', got {reweighting_mode}")
        for name, m in (("van_loan_expm", van_loan_expm), ("chen_expm", chen_expm)):
            if m not in nat.EXPM_SCHEMES:
                raise ValueError(f"{name} must be one of {tuple(nat.EXPM_SCHEMES)}, got {m!r}")
        if kind == "van_loan" and not 1 <= int(M) <= 64:
            raise NotImplementedError(f"the Van Loan leaf kernel takes 1 <= M <= 64 knots per interval, got M={M}")
        self.kind, self.q, self.M = kind, int(q), int(M)
        self.van_loan_expm, self.reweighting_mode, self.chen_expm = van_loan_expm, reweighting_mode, chen_expm

    def key(self):
        return (self.kind, self.q, self.M, self.van_loan_expm, self.reweighting_mode, self.chen_expm)


def make_dense_desc(B, L, d, N, q, flow_mode, readout, level0, chunk=0, leaf=None):
    leaf = leaf if leaf is not None else DenseLeaf("series", q)
    vl = leaf.kind == "van_loan"
    kind = {"series": nat.LEAF_SERIES, "van_loan": nat.LEAF_VAN_LOAN, "block_series": nat.LEAF_BLOCK_SERIES}[leaf.kind]
    return nat.DenseDesc(B, L, d, N, int(q) if not vl else 0, _FLOW_MODES[flow_mode], nat.READOUTS[readout],
                         int(level0), int(chunk), kind,
                         leaf.M if vl else 0, nat.EXPM_SCHEMES[leaf.van_loan_expm] if vl else 0,
                         _VL_MODES[leaf.reweighting_mode] if vl else 0, nat.EXPM_SCHEMES[leaf.chen_expm])


def _check_dense(path, clock, A):
    if not path.is_cuda:
        raise RuntimeError("ews_mi355x runs on a HIP device only: move path/clock/A to the GPU (no CPU path)")
    for name, x in (("path", path), ("clock", clock), ("A", A)):
        if x.dtype != torch.float32:
            raise TypeError(f"{name} must be float32 for the dense-generator kernels, got {x.dtype}")


class DenseScan(torch.autograd.Function):
    """out = EWS readout of (path, clock) under a dense generator A (series leaf of order q or the Van Loan leaf,
    flows of chen_expm). The backward is ews_dense_backward: the combine's adjoint scans, then the leaf's and the
    flows' adjoints per interval and one reduction for dA. When a gradient is needed the forward keeps its leaf,
    flows, chunk summaries and carries (ews_dense_forward_keep) and the first backward consumes them
    (ews_dense_backward_kept) instead of recomputing them; a second backward of the same graph recomputes.
    keep = False skips that (the workspace is then freed with the forward: 2.4 GB at c3's shape, per dense block of
    a stack, until the graph is released), at the price of the recompute in the backward."""

    @staticmethod
    def forward(ctx, path, clock, A, N, q, flow_mode, readout, level0, chunk, leaf, keep=True):
        lib = nat.load()
        _check_dense(path, clock, A)
        path, clock, A = path.contiguous(), clock.contiguous(), A.contiguous()
        B, L, d = path.shape
        desc = make_dense_desc(B, L, d, N, q, flow_mode, readout, level0, chunk, leaf)
        ctx.desc = desc
        ctx.leaf = leaf
        D = sum(d**k for k in range(1, N + 1))
        W = D + (1 if level0 else 0)
        shape = (B, L - 1, W) if readout == "prefix" else (B, W)
        dev = path.device
        out = torch.empty(shape, device=dev, dtype=torch.float32)
        keep = bool(keep) and any(ctx.needs_input_grad[:3])
        nbytes = (lib.ews_dense_backward_workspace_bytes if keep else lib.ews_dense_workspace_bytes)(
            ctypes.byref(desc))
        ws = torch.empty(int(nbytes), device=dev, dtype=torch.uint8)
        fwd = lib.ews_dense_forward_keep if keep else lib.ews_dense_forward
        rc = fwd(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(), out.data_ptr(), ws.data_ptr(),
                 _stream_handle(dev))
        nat.check(rc, "ews_dense_forward")
        ctx.kept = ws if keep else None
        # the kept backward reads the states from the output rows (prefix readout); autograd guards their version
        if keep:
            ctx.save_for_backward(path, clock, A, out)
        else:
            ctx.save_for_backward(path, clock, A)
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, A = ctx.saved_tensors[:3]
        rows = ctx.saved_tensors[3] if len(ctx.saved_tensors) > 3 else None
        desc = ctx.desc
        dev = path.device
        gout = gout.to(torch.float32).contiguous()
        gpath = torch.empty_like(path)
        need_clock = ctx.needs_input_grad[1]
        gclock = torch.empty_like(clock) if need_clock else None
        gA = torch.empty_like(A)
        ws, kept = ctx.kept, ctx.kept is not None
        ctx.kept = None  # the backward overwrites what the forward kept
        if not kept:
            ws = torch.empty(int(lib.ews_dense_backward_workspace_bytes(ctypes.byref(desc))), device=dev,
                             dtype=torch.uint8)
        args = (gout.data_ptr(), gpath.data_ptr(), gclock.data_ptr() if need_clock else None, gA.data_ptr(),
                ws.data_ptr(), _stream_handle(dev))
        if kept:
            rc = lib.ews_dense_backward_kept(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                             rows.data_ptr() if rows is not None else None, *args)
        else:
            rc = lib.ews_dense_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(), *args)
        nat.check(rc, "ews_dense_backward")
        return gpath, gclock, gA, None, None, None, None, None, None, None, None


def dense_keep_default():
    """Whether a dense forward keeps its backward workspace by default: yes unless EWS_DENSE_KEEP=0."""
    return os.environ.get("EWS_DENSE_KEEP", "1") != "0"


def dense_scan(path, clock, A, N, q, flow_mode="per_interval", readout="prefix", level0=True, chunk=0, leaf=None,
               keep=None):
    """keep: keep the forward's leaf, flows and carries for the backward (None: when grad mode is on, an input
    needs a gradient and EWS_DENSE_KEEP is not 0)."""
    leaf = leaf if leaf is not None else DenseLeaf("series", q)
    if keep is None:
        keep = torch.is_grad_enabled() and dense_keep_default()
    return DenseScan.apply(path, clock, A, int(N), int(q), flow_mode, readout, bool(level0), int(chunk), leaf,
                           bool(keep))


def dense_local_terms(path, clock, A, N, q, flow_mode="per_interval", leaf=None):
    """Leaf levels (B, L-1, sum_k d^k) packed and flows (B, L-1, d, d) on the GPU: the series leaf of order q,
    or the Van Loan leaf given by ``leaf`` (ews/core/leaf.py:86-114 and ews/core/chen_scan.py:155-168)."""
    lib = nat.load()
    _check_dense(path, clock, A)
    path, clock, A = path.contiguous(), clock.contiguous(), A.contiguous()
    B, L, d = path.shape
    desc = make_dense_desc(B, L, d, N, q, flow_mode, "prefix", False, 0, leaf)
    D = sum(d**k for k in range(1, N + 1))
    dev = path.device
    levels = torch.empty((B, L - 1, D), device=dev, dtype=torch.float32)
    flows = torch.empty((B, L - 1, d, d), device=dev, dtype=torch.float32)
    ws = torch.empty(int(lib.ews_dense_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
    rc = lib.ews_dense_local_terms(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                   levels.data_ptr(), flows.data_ptr(), ws.data_ptr(), _stream_handle(dev))
    nat.check(rc, "ews_dense_local_terms")
    return levels, flows


def dense_combine(levels, flows, N, readout="prefix", level0=True, chunk=0):
    """Chen combine of given packed levels (B, n, sum_k d^k) and flows (B, n, d, d)
    (ews/core/kernels/combine.py:259-269, kind "dense_kernel")."""
    lib = nat.load()
    if not levels.is_cuda or levels.dtype != torch.float32 or flows.dtype != torch.float32:
        raise TypeError("levels and flows must be float32 tensors on the HIP device")
    levels, flows = levels.contiguous(), flows.contiguous()
    B, n, d = flows.shape[0], flows.shape[1], flows.shape[2]
    desc = make_dense_desc(B, n + 1, d, N, 0, "per_interval", readout, level0, chunk)
    D = sum(d**k for k in range(1, N + 1))
    if levels.shape != (B, n, D):
        raise ValueError(f"levels must be {(B, n, D)}, got {tuple(levels.shape)}")
    W = D + (1 if level0 else 0)
    shape = (B, n, W) if readout == "prefix" else (B, W)
    out = torch.empty(shape, device=levels.device, dtype=torch.float32)
    ws = torch.empty(int(lib.ews_dense_workspace_bytes(ctypes.byref(desc))), device=levels.device,
                     dtype=torch.uint8)
    rc = lib.ews_dense_combine(ctypes.byref(desc), levels.data_ptr(), flows.data_ptr(), out.data_ptr(),
                               ws.data_ptr(), _stream_handle(levels.device))
    nat.check(rc, "ews_dense_combine")
    return out


def dense_combine_backward(levels, flows, grad_out, N, readout="prefix", level0=True, chunk=0):
    """Cotangents (grad_levels, grad_flows) of dense_combine's inputs for the cotangent grad_out of its output
    (the VJP of ews/core/kernels/pallas_combine.py:2628 dense_general_prefix_vjp)."""
    lib = nat.load()
    for name, x in (("levels", levels), ("flows", flows), ("grad_out", grad_out)):
        if not x.is_cuda or x.dtype != torch.float32:
            raise TypeError(f"{name} must be a float32 tensor on the HIP device")
    levels, flows, grad_out = levels.contiguous(), flows.contiguous(), grad_out.contiguous()
    B, n, d = flows.shape[0], flows.shape[1], flows.shape[2]
    desc = make_dense_desc(B, n + 1, d, N, 0, "per_interval", readout, level0, chunk)
    D = sum(d**k for k in range(1, N + 1))
    W = D + (1 if level0 else 0)
    shape = (B, n, W) if readout == "prefix" else (B, W)
    if levels.shape != (B, n, D) or grad_out.shape != shape:
        raise ValueError(f"levels must be {(B, n, D)} and grad_out {shape}")
    gl = torch.empty_like(levels)
    gf = torch.empty_like(flows)
    ws = torch.empty(int(lib.ews_dense_backward_workspace_bytes(ctypes.byref(desc))), device=levels.device,
                     dtype=torch.uint8)
    rc = lib.ews_dense_combine_backward(ctypes.byref(desc), levels.data_ptr(), flows.data_ptr(),
                                        grad_out.data_ptr(), gl.data_ptr(), gf.data_ptr(), ws.data_ptr(),
                                        _stream_handle(levels.device))
    nat.check(rc, "ews_dense_combine_backward")
    return gl, gf


# ---------------------------------------------------------------------------------------------- Jordan chains
def _jordan_desc(B, L, d, N, kind, size):
    return nat.JordanDesc(int(B), int(L), int(d), int(N), nat.JORDAN_KINDS[kind], int(size))


class JordanScan(torch.autograd.Function):
    """out = EWS readout of (path, clock) under uniform Jordan chains A (leaf jordan_closed / jordan_closed_tables,
    ews/core/kernels/jordan_engine.py:324-353): the chains' exact local terms (ews_jordan_local_terms), the flows of
    chen_expm under the reweighting mode (ews_dense_local_terms), the dense combine (ews_dense_combine). The
    backward runs the combine's adjoint, then the local terms' and the flows' adjoints, and sums them."""

    @staticmethod
    def forward(ctx, path, clock, A, N, kind, size, flow_mode, readout, level0, chunk, chen_expm):
        lib = nat.load()
        _check_dense(path, clock, A)
        path, clock, A = path.contiguous(), clock.contiguous(), A.contiguous()
        B, L, d = path.shape
        dev = path.device
        jd = _jordan_desc(B, L, d, N, kind, size)
        D = d + (d * d if N == 2 else 0)
        levels = torch.empty((B, L - 1, D), device=dev, dtype=torch.float32)
        nat.check(lib.ews_jordan_local_terms(ctypes.byref(jd), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                             levels.data_ptr(), _stream_handle(dev)), "ews_jordan_local_terms")
        fleaf = DenseLeaf("series", q=0, chen_expm=chen_expm)
        _, flows = dense_local_terms(path, clock, A, 1, 0, flow_mode, leaf=fleaf)
        out = dense_combine(levels, flows, N, readout, level0, chunk)
        ctx.save_for_backward(path, clock, A, levels, flows)
        ctx.cfg = (N, kind, size, flow_mode, readout, level0, chunk, fleaf)
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, A, levels, flows = ctx.saved_tensors
        N, kind, size, flow_mode, readout, level0, chunk, fleaf = ctx.cfg
        B, L, d = path.shape
        dev = path.device
        gl, gf = dense_combine_backward(levels, flows, gout.to(torch.float32).contiguous(), N, readout, level0,
                                        chunk)
        need_clock = ctx.needs_input_grad[1]
        jd = _jordan_desc(B, L, d, N, kind, size)
        gpath = torch.empty_like(path)
        gclock = torch.empty_like(clock) if need_clock else None
        gA = torch.empty_like(A)
        ws = torch.empty(int(lib.ews_jordan_workspace_bytes(ctypes.byref(jd))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_jordan_local_terms_backward(ctypes.byref(jd), path.data_ptr(), clock.data_ptr(),
                                                      A.data_ptr(), gl.data_ptr(), gpath.data_ptr(),
                                                      gclock.data_ptr() if need_clock else None, gA.data_ptr(),
                                                      ws.data_ptr(), _stream_handle(dev)),
                  "ews_jordan_local_terms_backward")
        # the flows' share: the leaf-and-flows adjoint with a zero level cotangent
        fdesc = make_dense_desc(B, L, d, 1, 0, flow_mode, "prefix", False, 0, fleaf)
        zl = torch.zeros((B, L - 1, d), device=dev, dtype=torch.float32)
        fpath = torch.empty_like(path)
        fclock = torch.empty_like(clock) if need_clock else None
        fA = torch.empty_like(A)
        fws = torch.empty(int(lib.ews_dense_backward_workspace_bytes(ctypes.byref(fdesc))), device=dev,
                          dtype=torch.uint8)
        nat.check(lib.ews_dense_local_terms_backward(ctypes.byref(fdesc), path.data_ptr(), clock.data_ptr(),
                                                     A.data_ptr(), zl.data_ptr(), gf.contiguous().data_ptr(),
                                                     fpath.data_ptr(), fclock.data_ptr() if need_clock else None,
                                                     fA.data_ptr(), fws.data_ptr(), _stream_handle(dev)),
                  "ews_dense_local_terms_backward")
        gA += fA
        if need_clock:
            gclock += fclock
        return gpath, gclock, gA, None, None, None, None, None, None, None, None


def jordan_scan(path, clock, A, N, kind, size, flow_mode="per_interval", readout="prefix", level0=True, chunk=0,
                chen_expm="exact"):
    """kind "real" (chain sizes 1-4) or "complex" (sizes 2, 4, 6, 8; size 2 = rotation planes)."""
    return JordanScan.apply(path, clock, A, int(N), kind, int(size), flow_mode, readout, bool(level0), int(chunk),
                            chen_expm)


# ---------------------------------------------------------------------------------------------- depth-1 chains
class ChainScan(torch.autograd.Function):
    """Depth-1 EWS of a block-diagonal A of uniform chains, any number of chains (ews_chain_forward /
    ews_chain_backward): prefix or terminal rows; the exact level 1 phi(-hA) v (series_q 0) or the series leaf's
    order-q truncation; exact flows in the chains' closed form. leaf_mode: the leaf's clock step (van_loan's
    uniform modes share one step)."""

    @staticmethod
    def forward(ctx, path, clock, A, kind, size, flow_mode, leaf_mode, readout, level0, series_q, chunk):
        lib = nat.load()
        for nm, t in (("path", path), ("clock", clock), ("A", A)):
            if not t.is_cuda:
                raise RuntimeError("ews_mi355x runs on a HIP device only: move path/clock/A to the GPU (no CPU path)")
            if t.dtype != torch.float32:
                raise TypeError(f"{nm} must be float32 for the chain kernels, got {t.dtype}")
        path, clock, A = path.contiguous(), clock.contiguous(), A.contiguous()
        B, L, d = path.shape
        desc = nat.ChainDesc(B, L, d, nat.JORDAN_KINDS[kind], int(size), _FLOW_MODES[flow_mode],
                             _FLOW_MODES[leaf_mode], nat.READOUTS[readout], int(level0), int(series_q), int(chunk))
        W = d + (1 if level0 else 0)
        dev = path.device
        out = torch.empty((B, L - 1, W) if readout == "prefix" else (B, W), device=dev, dtype=torch.float32)
        rs = torch.empty(int(lib.ews_chain_residual_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        ws = torch.empty(int(lib.ews_chain_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        if rs.numel() == 0 or ws.numel() == 0:
            raise ValueError(f"unsupported chain configuration: d={d}, kind={kind!r}, size={size}, "
                             f"series_q={series_q}, readout={readout!r}")
        nat.check(lib.ews_chain_forward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                        out.data_ptr(), rs.data_ptr(), ws.data_ptr(), _stream_handle(dev)),
                  "ews_chain_forward")
        ctx.save_for_backward(path, clock, A, rs)
        ctx.desc = desc
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, A, rs = ctx.saved_tensors
        desc = ctx.desc
        dev = path.device
        gout = gout.to(torch.float32).contiguous()
        gpath = torch.empty_like(path)
        need_clock = ctx.needs_input_grad[1]
        gclock = torch.empty_like(clock) if need_clock else None
        gA = torch.empty_like(A)
        ws = torch.empty(int(lib.ews_chain_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_chain_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                         rs.data_ptr(), gout.data_ptr(), gpath.data_ptr(),
                                         gclock.data_ptr() if need_clock else None, gA.data_ptr(), ws.data_ptr(),
                                         _stream_handle(dev)), "ews_chain_backward")
        return gpath, gclock, gA, None, None, None, None, None, None, None, None


def chain_scan(path, clock, A, kind, size, flow_mode="per_interval", leaf_mode="per_interval", readout="prefix",
               level0=True, series_q=0, chunk=0):
    """kind "real" (sizes 1-4; 1 = a real diagonal) or "complex" (sizes 2, 4, 6, 8; 2 = rotation planes); readout
    "prefix" or "terminal"."""
    return ChainScan.apply(path, clock, A, kind, int(size), flow_mode, leaf_mode, readout, bool(level0),
                           int(series_q), int(chunk))


# ---------------------------------------------------------------------------------------------- log-signature
class LogRows(torch.autograd.Function):
    """Compressed log of EWS state rows (B, R, level0 + D) with the LogEWS readout (ews/layer.py:488-517):
    ews_log_forward / ews_log_backward."""

    @staticmethod
    def forward(ctx, rows, d, N, level0, readout):
        lib = nat.load()
        if not rows.is_cuda or rows.dtype != torch.float32:
            raise TypeError("rows must be a float32 tensor on the HIP device")
        rows = rows.contiguous()
        B, R = rows.shape[0], rows.shape[1]
        desc = nat.LogDesc(B, R, d, N, int(level0), nat.READOUTS[readout])
        Dlog = int(lib.ews_log_dim(d, N))
        out = torch.empty((B, R, Dlog) if readout == "prefix" else (B, Dlog), device=rows.device,
                          dtype=torch.float32)
        ws = torch.empty(int(lib.ews_log_workspace_bytes(ctypes.byref(desc))), device=rows.device,
                         dtype=torch.uint8)
        nat.check(lib.ews_log_forward(ctypes.byref(desc), rows.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                      _stream_handle(rows.device)), "ews_log_forward")
        ctx.save_for_backward(rows)
        ctx.desc = desc
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        (rows,) = ctx.saved_tensors
        desc = ctx.desc
        gout = gout.to(torch.float32).contiguous()
        grows = torch.empty_like(rows)
        ws = torch.empty(int(lib.ews_log_workspace_bytes(ctypes.byref(desc))), device=rows.device,
                         dtype=torch.uint8)
        nat.check(lib.ews_log_backward(ctypes.byref(desc), rows.data_ptr(), gout.data_ptr(), grows.data_ptr(),
                                       ws.data_ptr(), _stream_handle(rows.device)), "ews_log_backward")
        return grows, None, None, None, None


def log_rows(rows, d, N, level0=True, readout="prefix"):
    return LogRows.apply(rows, int(d), int(N), bool(level0), readout)


# ---------------------------------------------------------------------------------------------- mixer epilogue
def _al256(x):
    return (x + 255) // 256 * 256


class MixerFn(torch.autograd.Function):
    """r = c_down(graded(prescale(levels))) of EWS prefix rows (B, R, level0 + D), fused in one pass
    (ews_mixer_forward / ews_mixer_backward; reference ews/block.py:282-306, 336-357, 405-408). The parameter
    gradients are assembled here from the kernel's per-row quantities: grad_bias = sum of grad_out, grad_gains =
    sum of row_dots times the gain factor, grad_weight per level = (scale_k grad_out)^T x_k (a plain GEMM)."""

    @staticmethod
    def forward(ctx, rows, weight, bias, gains, d, N, variant, eps, prepend, prescale, level0):
        lib = nat.load()
        for nm, t in (("rows", rows), ("weight", weight), ("bias", bias), ("gains", gains)):
            if not t.is_cuda or t.dtype != torch.float32:
                raise TypeError(f"{nm} must be a float32 tensor on the HIP device")
        rows = rows.contiguous()
        weight = weight.contiguous()
        B, R, W = rows.shape
        hidden = weight.shape[0]
        eps3 = (ctypes.c_float * 3)(*[float(e) for e in (list(eps) + [0.0] * 3)[:3]])
        desc = nat.MixerDesc(B, R, d, N, int(level0), hidden, nat.GRADED_VARIANTS[variant], int(prepend),
                             int(prescale), eps3)
        out = torch.empty((B, R + int(prepend), hidden), device=rows.device, dtype=torch.float32)
        resid = torch.empty(int(lib.ews_mixer_residual_bytes(ctypes.byref(desc))), device=rows.device,
                            dtype=torch.uint8)
        nat.check(lib.ews_mixer_forward(ctypes.byref(desc), rows.data_ptr(), weight.data_ptr(),
                                        bias.contiguous().data_ptr(), gains.contiguous().data_ptr(), out.data_ptr(),
                                        resid.data_ptr(), _stream_handle(rows.device)), "ews_mixer_forward")
        ctx.save_for_backward(rows, weight, gains, resid)
        ctx.meta = (desc, d, N, variant, int(prepend), int(level0))
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        rows, weight, gains, resid = ctx.saved_tensors
        desc, d, N, variant, prepend, level0 = ctx.meta
        gout = gout.to(torch.float32).contiguous()
        B, R, W = rows.shape
        hidden = weight.shape[0]
        M = B * R
        grows = torch.empty_like(rows)
        dots = torch.empty((B, R, N), device=rows.device, dtype=torch.float32)
        gweight, gbias, ggains = _mixer_backward(lib, desc, gout, rows, weight, gains, resid, grows, dots, d, N,
                                                 variant, prepend, level0, _stream_handle(rows.device))
        return grows, gweight, gbias, ggains, None, None, None, None, None, None, None


def _mixer_backward(lib, desc, gout, rows, weight, gains, resid, grows, dots, d, N, variant, prepend, level0, st):
    """The mixer's backward: grad_rows and row_dots, and c_down's weight gradient in the same pass over the rows
    (ews_mixer_backward_weight, hidden <= 128) or from the rows by a GEMM (wider c_down); grad_bias and grad_gains
    from grad_out and row_dots. Returns (grad_weight, grad_bias, grad_gains)."""
    nws = int(lib.ews_mixer_backward_workspace_bytes(ctypes.byref(desc)))
    if nws == 0:
        nat.check(lib.ews_mixer_backward(ctypes.byref(desc), rows.data_ptr(), weight.data_ptr(), resid.data_ptr(),
                                         gout.data_ptr(), grows.data_ptr(), dots.data_ptr(), st),
                  "ews_mixer_backward")
        return _mixer_param_grads(gout, rows, weight, gains, resid, dots, d, N, variant, prepend, level0)
    ws = torch.empty(nws, device=rows.device, dtype=torch.uint8)
    gweight = torch.empty_like(weight)
    nat.check(lib.ews_mixer_backward_weight(ctypes.byref(desc), rows.data_ptr(), weight.data_ptr(),
                                            resid.data_ptr(), gout.data_ptr(), grows.data_ptr(), dots.data_ptr(),
                                            gweight.data_ptr(), ws.data_ptr(), st), "ews_mixer_backward_weight")
    gbias, ggains = _mixer_bias_gain_grads(gout, gains, resid, dots, N, variant, weight.shape[0])
    return gweight, gbias, ggains


def _mixer_bias_gain_grads(gout, gains, resid, dots, N, variant, hidden):
    """grad_bias = sum of grad_out; grad_gains = sum over rows of row_dots times the residual's d scale / d gain."""
    M = dots.numel() // N
    F = resid[_al256(M * N * hidden * 4):].view(torch.float32)[: M * N * 3].view(M, N, 3)
    gbias = gout.sum((0, 1))
    gd = (F[:, :, 2] * dots.reshape(M, N)).sum(0)
    ggains = gd.sum().reshape(gains.shape) if variant == "dilation" else gd
    return gbias, ggains


def _mixer_param_grads(gout, rows, weight, gains, resid, dots, d, N, variant, prepend, level0):
    """c_down's and the gains' gradients from the per-row quantities of ews_mixer_backward: grad_bias = sum of
    grad_out, grad_gains = sum of row_dots times the gain factor, grad_weight per level = (scale_k grad_out)^T x_k."""
    B, R, W = rows.shape
    hidden = weight.shape[0]
    M = B * R
    # residual: level products (M, N, hidden) then factors (M, N, 3) = (scale, beta, d scale / d gain)
    F = resid[_al256(M * N * hidden * 4):].view(torch.float32)[: M * N * 3].view(M, N, 3)
    dr = gout[:, prepend:, :].reshape(M, hidden)
    gbias = gout.sum((0, 1))
    gd = (F[:, :, 2] * dots.reshape(M, N)).sum(0)
    ggains = gd.sum().reshape(gains.shape) if variant == "dilation" else gd
    gweight = torch.empty_like(weight)
    st = 0
    for k in range(N):
        n = d ** (k + 1)
        xk = rows[:, :, level0 + st: level0 + st + n].reshape(M, n)  # a strided view, no copy
        gweight[:, st: st + n] = _split_k_tn(dr * F[:, k, 0:1], xk)
        st += n
    return gweight, gbias, ggains


class ScanMixerFn(torch.autograd.Function):
    """The diagonal / rotation-plane scan's prefix rows straight into the block's mixer epilogue
    (ews_diag_mixer_forward): out = c_down(graded(prescale(levels))) with the D-wide rows never written. The
    backward regenerates the rows from the scan's float64 carries (ews_diag_forward_pass, pass 2), then runs the
    mixer's backward (ews_mixer_backward) and the scan's (ews_diag_backward)."""

    @staticmethod
    def forward(ctx, path, clock, params, weight, bias, gains, N, structure, flow_mode, leaf, series_q, variant, eps,
                prepend, prescale):
        lib = nat.load()
        _check_inputs(path, clock, params)
        for nm, t in (("weight", weight), ("bias", bias), ("gains", gains)):
            if not t.is_cuda or t.dtype != torch.float32:
                raise TypeError(f"{nm} must be a float32 tensor on the HIP device")
        path = _aligned(path.contiguous())
        clock, params, weight = clock.contiguous(), params.contiguous(), weight.contiguous()
        bias, gains = bias.contiguous(), gains.contiguous()
        B, L, d = path.shape
        hidden = weight.shape[0]
        dt = nat.DTYPE_BF16 if path.dtype == torch.bfloat16 else nat.DTYPE_F32
        sdesc = make_desc(B, L, d, N, structure, flow_mode, "prefix", True, dt, 0, leaf, series_q)
        eps3 = (ctypes.c_float * 3)(*[float(x) for x in (list(eps) + [0.0] * 3)[:3]])
        mdesc = nat.MixerDesc(B, L - 1, d, N, 1, hidden, nat.GRADED_VARIANTS[variant], int(prepend), int(prescale),
                              eps3)
        dev = path.device
        out = torch.empty((B, L - 1 + int(prepend), hidden), device=dev, dtype=torch.float32)
        mres = torch.empty(int(lib.ews_mixer_residual_bytes(ctypes.byref(mdesc))), device=dev, dtype=torch.uint8)
        sres = torch.empty(int(lib.ews_diag_residual_bytes(ctypes.byref(sdesc))), device=dev, dtype=torch.uint8)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(sdesc))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_diag_mixer_forward(ctypes.byref(sdesc), ctypes.byref(mdesc), path.data_ptr(),
                                             clock.data_ptr(), params.data_ptr(), weight.data_ptr(), bias.data_ptr(),
                                             gains.data_ptr(), out.data_ptr(), mres.data_ptr(), sres.data_ptr(),
                                             ws.data_ptr(), _stream_handle(dev)), "ews_diag_mixer_forward")
        ctx.save_for_backward(path, clock, params, weight, gains, sres, mres)
        ctx.meta = (sdesc, mdesc, d, N, variant, int(prepend))
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        path, clock, params, weight, gains, sres, mres = ctx.saved_tensors
        sdesc, mdesc, d, N, variant, prepend = ctx.meta
        gout = gout.to(torch.float32).contiguous()
        B, L, _ = path.shape
        dev = path.device
        st = _stream_handle(dev)
        ws = torch.empty(int(lib.ews_diag_workspace_bytes(ctypes.byref(sdesc))), device=dev, dtype=torch.uint8)
        # the prefix rows again, from the forward's carries (the chunk output pass)
        rows = torch.empty((B, L - 1, 1 + d + (d * d if N == 2 else 0)), device=dev, dtype=torch.float32)
        nat.check(lib.ews_diag_forward_pass(ctypes.byref(sdesc), 2, path.data_ptr(), clock.data_ptr(),
                                            params.data_ptr(), rows.data_ptr(), sres.data_ptr(), ws.data_ptr(), st),
                  "ews_diag_forward_pass")
        grows = torch.empty_like(rows)
        dots = torch.empty((B, L - 1, N), device=dev, dtype=torch.float32)
        gweight, gbias, ggains = _mixer_backward(lib, mdesc, gout, rows, weight, gains, mres, grows, dots, d, N,
                                                 variant, prepend, 1, st)
        del rows
        dpath = torch.empty((B, L, d), device=dev, dtype=torch.float32)
        dclock = torch.empty((B, L), device=dev, dtype=torch.float32) if ctx.needs_input_grad[1] else None
        dparams = torch.empty_like(params)
        nat.check(lib.ews_diag_backward(ctypes.byref(sdesc), path.data_ptr(), clock.data_ptr(), params.data_ptr(),
                                        sres.data_ptr(), grows.data_ptr(), dpath.data_ptr(),
                                        dclock.data_ptr() if dclock is not None else None, dparams.data_ptr(),
                                        ws.data_ptr(), st), "ews_diag_backward")
        return (dpath.to(path.dtype), dclock, dparams, gweight, gbias, ggains, None, None, None, None, None, None,
                None, None, None)


def scan_mixer(path, clock, params, weight, bias, gains, N, structure, flow_mode="per_interval",
               leaf="plane_closed", series_q=0, variant="live_rms", eps=(1e-3,), prepend=True, prescale=False):
    """The EWS scan's prefix rows (diagonal or rotation-plane generator) through the block's mixer epilogue, fused
    (ews_diag_mixer_forward) where the scan runs on the chunk kernels; None where it does not (the d = 16
    pair-group planes, the per-sample sequential kernels): the caller composes diag_scan and mixer_epilogue."""
    lib = nat.load()
    fm = {"per_interval": nat.FLOW_PER_INTERVAL, "cached": nat.FLOW_CACHED,
          "cached_basepoint": nat.FLOW_CACHED_BASEPOINT}[flow_mode]
    st = {"planes": nat.STRUCT_PLANES, "real_diag": nat.STRUCT_REAL_DIAG}[structure]
    B, L, d = path.shape
    if weight.shape[0] > 64 or N not in (1, 2):
        return None
    dt = nat.DTYPE_BF16 if path.dtype == torch.bfloat16 else nat.DTYPE_F32
    probe = make_desc(B, L, d, N, st, fm, "prefix", True, dt, 0, nat.DIAG_LEAVES[leaf], int(series_q or 0))
    if not lib.ews_diag_uses_chunk_kernels(ctypes.byref(probe)):
        return None
    eps = tuple(eps) if isinstance(eps, (tuple, list)) else (float(eps),) * N
    return ScanMixerFn.apply(path, clock, params, weight, bias, gains, int(N), st, fm, nat.DIAG_LEAVES[leaf],
                             int(series_q or 0), variant, eps, bool(prepend), bool(prescale))


def _split_k_tn(a, b, chunks=64):
    """a^T b for tall a (M, h) and b (M, n): a GEMM whose output is small and whose reduction runs over every
    row. A single library call tiles only the small output (a few workgroups); here the rows are cut into
    ``chunks`` batches of one batched GEMM whose partial products are then summed."""
    M = a.shape[0]
    S = min(chunks, max(1, M // 256))
    m = M // S
    out = torch.bmm(a[: S * m].reshape(S, m, -1).transpose(1, 2), b[: S * m].reshape(S, m, -1)).sum(0)
    if S * m < M:
        out = out + a[S * m:].t() @ b[S * m:]
    return out


def mixer_epilogue(rows, weight, bias, gains, d, N, variant="live_rms", eps=(1e-3,), prepend=True, prescale=False,
                   level0=True):
    eps = tuple(eps) if isinstance(eps, (tuple, list)) else (float(eps),) * N
    return MixerFn.apply(rows, weight, bias, gains, int(d), int(N), variant, eps, bool(prepend), bool(prescale),
                         bool(level0))


# ------------------------------------------------------------------------------------------------ block front
def _dev_f32(name, t):
    if not t.is_cuda or t.dtype != torch.float32:
        raise TypeError(f"{name} must be a float32 tensor on the HIP device")
    return t.contiguous()


def _mask_bytes(mask, B, L, device):
    if mask is None:
        return None
    m = mask.to(device=device)
    if m.dim() == 1:
        m = m.expand(B, L)
    if tuple(m.shape) != (B, L):
        raise ValueError("mask must be (seq_len,) or (batch, seq_len)")
    return m.to(torch.uint8).contiguous()


class ClockFn(torch.autograd.Function):
    """theta (B, L + basepoint) of one clock over a batch (ews_clock_forward / ews_clock_backward; reference
    ews/clocks.py:164-267 build_clock_jnp and :443-466 GatedClock.__call__). ``params`` is the flat parameter
    vector of the clock: [alpha] (blended_learn, after its map to [0, 1]) or [w (K c), b (K)] (gated modes)."""

    @staticmethod
    def forward(ctx, driver, params, times, mask, desc):
        lib = nat.load()
        dev = times.device
        B, L = desc.batch, desc.length
        if driver is not None:
            driver = _dev_f32("driver", driver)
        params = _dev_f32("params", params) if params is not None and params.numel() else None
        m = _mask_bytes(mask, B, L, dev)
        theta = torch.empty((B, L + desc.basepoint), device=dev, dtype=torch.float32)
        resid = torch.empty(max(1, int(lib.ews_clock_residual_bytes(ctypes.byref(desc)))), device=dev,
                            dtype=torch.uint8)
        nat.check(lib.ews_clock_forward(ctypes.byref(desc), times.data_ptr(),
                                        driver.data_ptr() if driver is not None else None,
                                        m.data_ptr() if m is not None else None,
                                        params.data_ptr() if params is not None else None, theta.data_ptr(),
                                        resid.data_ptr(), _stream_handle(dev)), "ews_clock_forward")
        ctx.save_for_backward(driver, params, times, m, resid)
        ctx.desc = desc
        return theta

    @staticmethod
    def backward(ctx, gtheta):
        lib = nat.load()
        driver, params, times, m, resid = ctx.saved_tensors
        desc = ctx.desc
        if desc.mode == nat.CLOCK_MODES["time"]:
            return None, None, None, None, None
        dev = times.device
        gtheta = gtheta.to(torch.float32).contiguous()
        gdrv = torch.empty_like(driver) if ctx.needs_input_grad[0] else None
        gprm = torch.empty_like(params) if params is not None else None
        ws = torch.empty(max(1, int(lib.ews_clock_workspace_bytes(ctypes.byref(desc)))), device=dev,
                         dtype=torch.uint8)
        nat.check(lib.ews_clock_backward(ctypes.byref(desc), times.data_ptr(), driver.data_ptr(),
                                         m.data_ptr() if m is not None else None,
                                         params.data_ptr() if params is not None else None, resid.data_ptr(),
                                         gtheta.data_ptr(), gdrv.data_ptr() if gdrv is not None else None,
                                         gprm.data_ptr() if gprm is not None else None, ws.data_ptr(),
                                         _stream_handle(dev)), "ews_clock_backward")
        return gdrv, gprm, None, None, None


class LiftFn(torch.autograd.Function):
    """The path the block hands to its EWS layer: p (B, L + basepoint, w) from the branch (B, L, H) and the
    appended clock channel (ews_lift_forward / ews_lift_backward; reference ews/block.py:284-301 with B.__call__,
    ews/params.py:1181-1191, and the increment path of ews/paths.py:126-131)."""

    @staticmethod
    def forward(ctx, branch, theta_app, matrix, mask, desc):
        lib = nat.load()
        branch = _dev_f32("branch", branch)
        dev = branch.device
        if theta_app is not None:
            theta_app = _dev_f32("theta_app", theta_app)
        if matrix is not None:
            matrix = _dev_f32("matrix", matrix)
        m = _mask_bytes(mask, desc.batch, desc.length, dev)
        path = torch.empty((desc.batch, desc.length + desc.basepoint, desc.out_dim), device=dev,
                           dtype=torch.float32)
        resid = torch.empty(max(1, int(lib.ews_lift_residual_bytes(ctypes.byref(desc)))), device=dev,
                            dtype=torch.uint8)
        nat.check(lib.ews_lift_forward(ctypes.byref(desc), branch.data_ptr(),
                                       theta_app.data_ptr() if theta_app is not None else None,
                                       m.data_ptr() if m is not None else None,
                                       matrix.data_ptr() if matrix is not None else None, path.data_ptr(),
                                       resid.data_ptr(), _stream_handle(dev)), "ews_lift_forward")
        ctx.save_for_backward(branch, theta_app, matrix, m, resid)
        ctx.desc = desc
        return path

    @staticmethod
    def backward(ctx, gpath):
        lib = nat.load()
        branch, theta_app, matrix, m, resid = ctx.saved_tensors
        desc = ctx.desc
        dev = branch.device
        gpath = gpath.to(torch.float32).contiguous()
        gbr = torch.empty_like(branch)
        gtha = torch.empty_like(theta_app) if theta_app is not None else None
        gmat = torch.empty_like(matrix) if matrix is not None else None
        ws = torch.empty(max(1, int(lib.ews_lift_workspace_bytes(ctypes.byref(desc)))), device=dev,
                         dtype=torch.uint8)
        nat.check(lib.ews_lift_backward(ctypes.byref(desc), branch.data_ptr(),
                                        theta_app.data_ptr() if theta_app is not None else None,
                                        m.data_ptr() if m is not None else None,
                                        matrix.data_ptr() if matrix is not None else None, resid.data_ptr(),
                                        gpath.data_ptr(), gbr.data_ptr(), gtha.data_ptr() if gtha is not None else None,
                                        gmat.data_ptr() if gmat is not None else None, ws.data_ptr(),
                                        _stream_handle(dev)), "ews_lift_backward")
        return gbr, gtha, gmat, None, None
