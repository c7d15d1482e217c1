"""Token-cached EWS scan on the HIP device (the reference's ews/core/token_scan.py).

With the increment path and a finite vocabulary, each step's displacement and clock increment depend on its token
alone, so the per-step local signatures and flows reduce to |V| cached ones. ``build_token_cache`` computes them
with the dense leaf kernels (one single-interval sample per token: its increments are exactly the token's, with no
cumulative sum in between), and ``token_cached_prefix_scan`` runs the dense Chen combine with each step reading its
token's cache row (csrc/ews_dense.hip, ``ews_token_scan``): no per-step levels or flows are materialised. Both are
differentiable: the scan's backward sums the per-step cotangents by token (``ews_token_scan_backward``), the cache's
goes through the leaf's adjoint (``ews_dense_local_terms_backward``).
"""

from __future__ import annotations

import ctypes

import torch

from . import _native as nat
from . import ops
from .ops import DenseLeaf, _stream_handle, make_dense_desc


class _LocalTermsFn(torch.autograd.Function):
    """levels (B, L-1, sum_k d^k), flows (B, L-1, d, d) of (path, clock, A) with their backward."""

    @staticmethod
    def forward(ctx, path, clock, A, N, leaf):
        lib = nat.load()
        for nm, t in (("path", path), ("clock", clock), ("A", A)):
            if not t.is_cuda or t.dtype != torch.float32:
                raise TypeError(f"{nm} must be a float32 tensor on the HIP device")
        path, clock, A = path.contiguous(), clock.contiguous(), A.contiguous()
        B, L, d = path.shape
        desc = make_dense_desc(B, L, d, N, leaf.q, "per_interval", "prefix", False, 0, leaf)
        D = sum(d**k for k in range(1, N + 1))
        dev = path.device
        levels = torch.empty((B, L - 1, D), device=dev, dtype=torch.float32)
        flows = torch.empty((B, L - 1, d, d), device=dev, dtype=torch.float32)
        ws = torch.empty(int(lib.ews_dense_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_dense_local_terms(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(), A.data_ptr(),
                                            levels.data_ptr(), flows.data_ptr(), ws.data_ptr(), _stream_handle(dev)),
                  "ews_dense_local_terms")
        ctx.save_for_backward(path, clock, A)
        ctx.desc = desc
        return levels, flows

    @staticmethod
    def backward(ctx, glevels, gflows):
        lib = nat.load()
        path, clock, A = ctx.saved_tensors
        desc = ctx.desc
        dev = path.device
        glevels = (torch.zeros_like(glevels) if glevels is None else glevels).to(torch.float32).contiguous()
        gflows = (torch.zeros_like(gflows) if gflows is None else gflows).to(torch.float32).contiguous()
        gpath = torch.empty_like(path)
        gclock = torch.empty_like(clock)
        gA = torch.empty_like(A)
        ws = torch.empty(int(lib.ews_dense_backward_workspace_bytes(ctypes.byref(desc))), device=dev,
                         dtype=torch.uint8)
        nat.check(lib.ews_dense_local_terms_backward(ctypes.byref(desc), path.data_ptr(), clock.data_ptr(),
                                                     A.data_ptr(), glevels.data_ptr(), gflows.data_ptr(),
                                                     gpath.data_ptr(), gclock.data_ptr(), gA.data_ptr(),
                                                     ws.data_ptr(), _stream_handle(dev)),
                  "ews_dense_local_terms_backward")
        return gpath, gclock, gA, None, None


def _chain_structure(A):
    """(kind, size) when A is rotation planes [[a, -b], [b, a]] on consecutive coordinate pairs or a real diagonal
    (the parametrisations of the formal-language blocks), read off its values; else None."""
    a = A.detach().to("cpu", torch.float64)
    d = a.shape[0]
    off = a - torch.diag(torch.diagonal(a))
    if not bool(off.any()):
        return ("real", 1)
    if d % 2:
        return None
    blk = torch.zeros_like(a, dtype=torch.bool)
    for i in range(0, d, 2):
        blk[i:i + 2, i:i + 2] = True
    if bool(a[~blk].any()):
        return None
    i = torch.arange(0, d, 2)
    if bool((a[i, i] != a[i + 1, i + 1]).any()) or bool((a[i, i + 1] != -a[i + 1, i]).any()):
        return None
    return ("complex", 2)


def _wide_cache(vocab_dx, vocab_dtheta, A, N, expm_method, chen_method, leaf, series_q, chain):
    """Depth-1 caches wider than the dense kernels for a chain-structured A, on the chain kernels: a token's level 1
    is the one-interval row of the knots (0, dx_g) at clock (0, dtheta_g); column i of its flow is the state after a
    zero-step injection of e_i and one step of dtheta_g (knots 0, e_i, e_i at clock 0, 0, dtheta_g). Both are
    differentiable through the chain kernels' adjoint."""
    if N != 1:
        raise NotImplementedError("token caches wider than 16 coordinates are built at depth 1 (the banked "
                                  "formal-language blocks); deeper ones need the dense kernels (d <= 16)")
    if chen_method != "exact" or (leaf == "van_loan" and expm_method != "exact"):
        raise NotImplementedError("token caches wider than 16 coordinates take exact exponentials")
    if chain is None:
        # the structure the parametrisation tagged its output with, else read off A's values (a copy to the host,
        # which waits for the device's queued work)
        chain = getattr(A, "_ews_chain", None) or _chain_structure(A)
    if chain is None:
        raise NotImplementedError("token caches wider than 16 coordinates need rotation planes, a real diagonal or "
                                  "uniform Jordan chains (pass chain=(kind, size))")
    kind, size = chain
    q = int(series_q) if leaf == "series" else 0
    V, d = vocab_dx.shape
    A = A.to(torch.float32).contiguous()
    zero = torch.zeros_like(vocab_dtheta)
    path = torch.stack([torch.zeros_like(vocab_dx), vocab_dx], 1).to(torch.float32)
    clock = torch.stack([zero, vocab_dtheta], 1).to(torch.float32)
    P = ops.chain_scan(path, clock, A, kind, size, readout="prefix", level0=False, series_q=q)[:, 0]
    eye = torch.eye(d, device=vocab_dx.device, dtype=torch.float32)
    basis = eye[None].expand(V, d, d).reshape(V * d, 1, d)
    kp = torch.cat([torch.zeros_like(basis), basis, basis], 1)
    th = vocab_dtheta.to(torch.float32).repeat_interleave(d)
    kc = torch.stack([torch.zeros_like(th), torch.zeros_like(th), th], 1)
    cols = ops.chain_scan(kp, kc, A, kind, size, readout="prefix", level0=False, series_q=q)[:, 1]  # (V d, d)
    D = cols.reshape(V, d, d).transpose(1, 2).contiguous()  # column i of token g's flow
    D._ews_block = int(size)  # block-diagonal with blocks of `size` coordinates: the cached scan's sparse route
    return P, D


def build_token_cache(vocab_dx, vocab_dtheta, A, M, N, expm_method="exact", chen_expm_method=None,
                      leaf="van_loan", series_q=None, chain=None):
    """ews/core/token_scan.py:44-88: P_cache (|V|, sum_k d^k), the packed local signature of each token's segment
    (its displacement vocab_dx[g], clock increment vocab_dtheta[g]), and D_cache (|V|, d, d) = exp(-dtheta_g A)
    (the flow of chen_expm, default expm_method). Differentiable in vocab_dx, vocab_dtheta and A. Above 16
    coordinates (depth 1, exact exponentials) A must be chain-structured: rotation planes or a real diagonal, read
    off A, or the uniform Jordan chains given by ``chain=(kind, size)``; the caches then come from the chain
    kernels."""
    if leaf not in ("series", "van_loan"):
        raise ValueError(f"leaf must be 'van_loan' or 'series', got {leaf!r}")
    if leaf == "series" and series_q is None:
        raise ValueError("leaf='series' requires series_q")
    if vocab_dx.shape[1] > 16:
        return _wide_cache(vocab_dx, vocab_dtheta, A, int(N), expm_method, chen_expm_method or expm_method, leaf,
                           series_q, chain)
    if leaf == "series":
        if series_q is None:
            raise ValueError("leaf='series' requires series_q")
        lf = DenseLeaf("series", int(series_q), chen_expm=chen_expm_method or expm_method)
    elif leaf == "van_loan":
        lf = DenseLeaf("van_loan", 0, M=int(M), van_loan_expm=expm_method, reweighting_mode="displacement",
                       chen_expm=chen_expm_method or expm_method)
    else:
        raise ValueError(f"leaf must be 'van_loan' or 'series', got {leaf!r}")
    V, d = vocab_dx.shape
    # one single-interval sample per token: knots (0, dx_g) and clock (0, dtheta_g)
    path = torch.stack([torch.zeros_like(vocab_dx), vocab_dx], 1)
    clock = torch.stack([torch.zeros_like(vocab_dtheta), vocab_dtheta], 1)
    levels, flows = _LocalTermsFn.apply(path, clock, A, int(N), lf)
    return levels[:, 0], flows[:, 0]


class _TokenScanFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, P_cache, D_cache, token_ids, mask, N, chunk):
        lib = nat.load()
        for nm, t in (("P_cache", P_cache), ("D_cache", D_cache)):
            if not t.is_cuda or t.dtype != torch.float32:
                raise TypeError(f"{nm} must be a float32 tensor on the HIP device")
        P_cache, D_cache = P_cache.contiguous(), D_cache.contiguous()
        V, d = D_cache.shape[0], D_cache.shape[1]
        B, n = token_ids.shape
        dev = P_cache.device
        tok = token_ids.to(device=dev, dtype=torch.int32).contiguous()
        m = None if mask is None else mask.to(device=dev).expand(B, n).to(torch.uint8).contiguous()
        desc = make_dense_desc(B, n + 1, d, N, 0, "per_interval", "prefix", False, chunk)
        D = sum(d**k for k in range(1, N + 1))
        if tuple(P_cache.shape) != (V, D):
            raise ValueError(f"P_cache must be {(V, D)}, got {tuple(P_cache.shape)}")
        out = torch.empty((B, n, D), device=dev, dtype=torch.float32)
        ws = torch.empty(int(lib.ews_token_scan_workspace_bytes(ctypes.byref(desc), V)), device=dev,
                         dtype=torch.uint8)
        nat.check(lib.ews_token_scan(ctypes.byref(desc), tok.data_ptr(), m.data_ptr() if m is not None else None,
                                     P_cache.data_ptr(), D_cache.data_ptr(), V, out.data_ptr(), ws.data_ptr(),
                                     _stream_handle(dev)), "ews_token_scan")
        ctx.save_for_backward(P_cache, D_cache, tok, m)
        ctx.desc = desc
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        P_cache, D_cache, tok, m = ctx.saved_tensors
        desc = ctx.desc
        V = D_cache.shape[0]
        dev = P_cache.device
        gout = gout.to(torch.float32).contiguous()
        gP = torch.empty_like(P_cache)
        gD = torch.empty_like(D_cache)
        ws = torch.empty(int(lib.ews_token_scan_workspace_bytes(ctypes.byref(desc), V)), device=dev,
                         dtype=torch.uint8)
        nat.check(lib.ews_token_scan_backward(ctypes.byref(desc), tok.data_ptr(),
                                              m.data_ptr() if m is not None else None, P_cache.data_ptr(),
                                              D_cache.data_ptr(), V, gout.data_ptr(), gP.data_ptr(), gD.data_ptr(),
                                              ws.data_ptr(), _stream_handle(dev)), "ews_token_scan_backward")
        return gP, gD, None, None, None, None


class _Token1ScanFn(torch.autograd.Function):
    """Depth-1 cached scan for caches of any width up to 64 (ews_token1_scan / ews_token1_scan_backward)."""

    @staticmethod
    def forward(ctx, P_cache, D_cache, token_ids, mask, block):
        lib = nat.load()
        for nm, t in (("P_cache", P_cache), ("D_cache", D_cache)):
            if not t.is_cuda or t.dtype != torch.float32:
                raise TypeError(f"{nm} must be a float32 tensor on the HIP device")
        P_cache, D_cache = P_cache.contiguous(), D_cache.contiguous()
        V, d = D_cache.shape[0], D_cache.shape[1]
        if tuple(P_cache.shape) != (V, d):
            raise ValueError(f"P_cache must be {(V, d)} at depth 1, got {tuple(P_cache.shape)}")
        B, n = token_ids.shape
        dev = P_cache.device
        tok = token_ids.to(device=dev, dtype=torch.int32).contiguous()
        m = None if mask is None else mask.to(device=dev).expand(B, n).to(torch.uint8).contiguous()
        if block and (d % block or V * (block + 1) > 64 or block not in (1, 2, 3, 4, 6, 8)):
            block = 0  # the dense route
        desc = nat.Token1Desc(B, n, d, V, int(block))
        out = torch.empty((B, n, d), device=dev, dtype=torch.float32)
        ws = torch.empty(int(lib.ews_token1_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_token1_scan(ctypes.byref(desc), tok.data_ptr(), m.data_ptr() if m is not None else None,
                                      P_cache.data_ptr(), D_cache.data_ptr(), out.data_ptr(), ws.data_ptr(),
                                      _stream_handle(dev)), "ews_token1_scan")
        ctx.save_for_backward(P_cache, D_cache, tok, m, out)
        ctx.desc = desc
        return out

    @staticmethod
    def backward(ctx, gout):
        lib = nat.load()
        P_cache, D_cache, tok, m, out = ctx.saved_tensors
        desc = ctx.desc
        dev = P_cache.device
        gout = gout.to(torch.float32).contiguous()
        gP = torch.empty_like(P_cache)
        gD = torch.empty_like(D_cache)
        ws = torch.empty(int(lib.ews_token1_workspace_bytes(ctypes.byref(desc))), device=dev, dtype=torch.uint8)
        nat.check(lib.ews_token1_scan_backward(ctypes.byref(desc), tok.data_ptr(),
                                               m.data_ptr() if m is not None else None, P_cache.data_ptr(),
                                               D_cache.data_ptr(), out.data_ptr(), gout.data_ptr(), gP.data_ptr(),
                                               gD.data_ptr(), ws.data_ptr(), _stream_handle(dev)),
                  "ews_token1_scan_backward")
        return gP, gD, None, None, None


def token_cached_prefix_scan(token_ids, mask, P_cache, D_cache, dim, trunc, chunk=0, block=None):
    """ews/core/token_scan.py:91-118, batched: token_ids (B, L) or (L,) ints, mask (B, L) / (L,) bool or None ->
    the packed prefix signatures (B, L, sum_k d^k) (no level-0 column, the layout of pack_signatures).
    S_t = mult(apply_M(S_{t-1}, D_t), P_t) from the unit; a padded step applies D = I and the unit signature.
    Above 16 coordinates, block (default: the value build_token_cache records on a chain-structured D_cache) says
    that every flow is block-diagonal with blocks of that many coordinates, which the scan then exploits."""
    single = token_ids.dim() == 1
    if single:
        token_ids = token_ids[None]
        mask = None if mask is None else mask.reshape(1, -1)
    if D_cache.shape[1] != int(dim):
        raise ValueError(f"D_cache is for dim {D_cache.shape[1]}, not {dim}")
    if int(dim) > 16:
        if int(trunc) != 1:
            raise NotImplementedError("the token-cached scan above 16 coordinates runs at depth 1")
        bs = getattr(D_cache, "_ews_block", 0) if block is None else int(block)
        out = _Token1ScanFn.apply(P_cache, D_cache, token_ids, mask, bs)
        return out[0] if single else out
    out = _TokenScanFn.apply(P_cache, D_cache, token_ids, mask, int(trunc), int(chunk))
    return out[0] if single else out
