"""CPU float64 restatement of the reference's EWS hot path (leaf -> Chen combine -> readout).

TEST INFRASTRUCTURE ONLY. Nothing in the product (the ``ews_mi355x`` package and its HIP library) imports,
links or runs this file; ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg use it as
the checker. It is written with torch float64 tensors on the CPU so that gradients come from autograd of the
same restatement.

Every function cites the reference (``/root/reference``) file:line whose behaviour it restates. Sign
convention is the reference's: the flow over an interval of clock length ``h`` is ``M = exp(-h A)``.
"""

from __future__ import annotations

import math
from fractions import Fraction
from functools import lru_cache
from itertools import product as iproduct

import torch

DT = torch.float64
CT = torch.complex128


# ============================================================== phi family (ews/core/kernels/plane_engine.py:23-78)
def _guarded(x, closed, series, tol):
    """plane_engine.py:23-26: closed form away from 0, Taylor series near 0, NaN-free gradients."""
    small = x.abs() < tol
    xs = torch.where(small, torch.ones_like(x), x)
    return torch.where(small, series(x), closed(xs))


def phi(x):
    """phi(x) = (e^x - 1)/x  (plane_engine.py:29-35)."""
    return _guarded(
        x,
        lambda x: torch.expm1(x) / x,
        lambda x: 1 + x * (1 / 2 + x * (1 / 6 + x * (1 / 24 + x * (1 / 120 + x / 720)))),
        1e-3,
    )


def dphi(x):
    """phi'(x)  (plane_engine.py:38-44)."""
    return _guarded(
        x,
        lambda x: (torch.exp(x) * (x - 1) + 1) / x**2,
        lambda x: 1 / 2 + x * (1 / 3 + x * (1 / 8 + x * (1 / 30 + x * (1 / 144 + x / 840)))),
        3e-2,
    )


def d2phi(x):
    """phi''(x)  (plane_engine.py:47-53)."""
    return _guarded(
        x,
        lambda x: (torch.exp(x) * (x**2 - 2 * x + 2) - 2) / x**3,
        lambda x: 1 / 3 + x * (1 / 4 + x * (1 / 10 + x * (1 / 36 + x * (1 / 168 + x / 960)))),
        1e-1,
    )


def d3phi(x):
    """phi'''(x)  (plane_engine.py:56-62)."""
    return _guarded(
        x,
        lambda x: (torch.exp(x) * (x**3 - 3 * x**2 + 6 * x - 6) + 6) / x**4,
        lambda x: 1 / 4 + x * (1 / 5 + x * (1 / 12 + x * (1 / 42 + x * (1 / 192 + x / 1080)))),
        2.5e-1,
    )


def divdiff_phi(x, delta, tol=4e-4):
    """D(x, delta) = (phi(x + delta) - phi(x)) / delta with a third-order Taylor branch for small delta
    (plane_engine.py:65-78; tol is the reference's float64 value). D(x, delta) is the double integral
    int_{0<s1<s2<1} e^{x(1-s1)} e^{delta(1-s2)}: x belongs to the earlier factor."""
    small = delta.abs() < tol
    ds = torch.where(small, torch.ones_like(delta), delta)
    direct = (phi(x + ds) - phi(x)) / ds
    series = dphi(x) + delta * (d2phi(x) / 2 + delta * d3phi(x) / 6)
    return torch.where(small, series, direct)


# ============================================================== layouts
def level_sizes(d, N):
    return [d**k for k in range(1, N + 1)]


def sig_dim(d, N):
    return sum(level_sizes(d, N))


def pack(levels):
    """Levels [(n,)+(d,)*k] -> (n, sum d^k)  (ews/core/chen_scan.py:33-46)."""
    n = levels[0].shape[0]
    return torch.cat([lv.reshape(n, -1) for lv in levels], dim=1)


def unpack(packed, d, N):
    """(n, sum d^k) -> levels  (chen_scan.py:81-95)."""
    out, s = [], 0
    n = packed.shape[0]
    for k in range(1, N + 1):
        out.append(packed[:, s : s + d**k].reshape((n,) + (d,) * k))
        s += d**k
    return out


# ============================================================== tensor algebra
def outer(a, b):
    """Batched outer product (n,)+sa, (n,)+sb -> (n,)+sa+sb."""
    n = a.shape[0]
    ka, kb = a.dim() - 1, b.dim() - 1
    return (a.reshape((n,) + a.shape[1:] + (1,) * kb) * b.reshape((n,) + (1,) * ka + b.shape[1:]))


def apply_M(M, T):
    """Apply M (n,d,d) along every tensor axis of T (n,)+(d,)*k  (chen_scan.py:98-121)."""
    k = T.dim() - 1
    out = T
    for ax in range(1, k + 1):
        # contract M[n, a, b] with axis `ax` of out (index b), put the new index a back in place
        out = torch.movedim(torch.einsum("nab,n...b->n...a", M, torch.movedim(out, ax, -1)), -1, ax)
    return out


def tensor_mult(X, Y):
    """Truncated tensor product of two group elements with level 0 = 1 (signax.tensor_ops.mult, used at
    chen_scan.py:146): Z_k = X_k + Y_k + sum_{j=1}^{k-1} X_j (x) Y_{k-j}."""
    N = len(X)
    Z = []
    for k in range(1, N + 1):
        z = X[k - 1] + Y[k - 1]
        for j in range(1, k):
            z = z + outer(X[j - 1], Y[k - j - 1])
        Z.append(z)
    return Z


def tensor_exp_vec(delta, N):
    """Signature of one linear segment with increment delta (n, d): level k = delta^{(x)k} / k!."""
    out, cur = [], None
    for k in range(1, N + 1):
        cur = delta if cur is None else outer(cur, delta)
        out.append(cur / math.factorial(k))
    return out


def signature_of_knots(knots, N):
    """Signature of the piecewise-linear path through knots (n, P, d), levels 1..N (level 0 omitted):
    Chen products of the segments' exponentials (what ``signax.signature`` returns for stream=False, used at
    ews/core/signature.py:20-35)."""
    S = None
    for i in range(1, knots.shape[1]):
        seg = tensor_exp_vec(knots[:, i] - knots[:, i - 1], N)
        S = seg if S is None else tensor_mult(S, seg)
    return S


# ============================================================== matrix exponential (ews/core/expm_approx.py:13-41)
def expm(X, method="exact"):
    method = method.lower()
    if method in ("pade_lite", "pade-lite"):
        method = "pade"
    eye = torch.eye(X.shape[-1], dtype=X.dtype).expand(X.shape)
    if method == "exact":
        return torch.linalg.matrix_exp(X)
    if method == "euler":
        return eye + X
    if method == "cayley":
        return torch.linalg.solve(eye - 0.5 * X, eye + 0.5 * X)
    if method == "pade":
        X2 = X @ X
        return torch.linalg.solve(eye - 0.5 * X + X2 / 12.0, eye + 0.5 * X + X2 / 12.0)
    raise ValueError(f"Unknown expm method: {method}")


def flows(dtheta, A, method="exact", cached=False, basepoint=False):
    """Per-interval flows M_t = exp(-dtheta_t A): one exponential per interval, or one shared exponential
    (from dtheta[0], or dtheta[1] with M_0 = I for a basepoint)  (chen_scan.py:155-168)."""
    n, d = dtheta.shape[0], A.shape[0]
    if not cached:
        return expm(-dtheta[:, None, None] * A[None], method)
    if basepoint:
        Ms = expm(-dtheta[1] * A, method)
        return torch.cat([torch.eye(d, dtype=A.dtype)[None], Ms[None].expand(n - 1, d, d)], 0)
    Ms = expm(-dtheta[0] * A, method)
    return Ms[None].expand(n, d, d)


# ============================================================== leaves
def plane_local_terms(v, dw, dtheta, N):
    """Closed-form local terms for rotation planes A_j = [[d_j, w_j], [-w_j, d_j]] on channels (2j, 2j+1)
    (ews/core/kernels/plane_engine.py:134-152 with the layouts of :84-128, routed by ews/core/leaf.py:116-136).
    Returns real levels [(n, m)] or [(n, m), (n, m, m)]."""
    n, m = v.shape
    K = m // 2
    z = torch.complex(dw[:, 0], dw[:, 1])  # (K,)
    zc = z.conj()
    h = dtheta[:, None].to(CT)
    p = torch.complex(v[:, 0::2], v[:, 1::2])  # (n, K)
    s1 = phi(-h * zc[None]) * p
    lvl1 = torch.stack([s1.real, s1.imag], -1).reshape(n, m)
    if N == 1:
        return [lvl1]
    x = -h[:, :, None] * zc[None, :, None]
    IA = divdiff_phi(x, -h[:, :, None] * z[None, None, :])
    IB = divdiff_phi(x, -h[:, :, None] * zc[None, None, :])
    Ac = IA * p[:, :, None] * p.conj()[:, None, :]
    Bc = IB * p[:, :, None] * p[:, None, :]
    q00 = (Ac.real + Bc.real) / 2
    q11 = (Ac.real - Bc.real) / 2
    q01 = (Bc.imag - Ac.imag) / 2
    q10 = (Ac.imag + Bc.imag) / 2
    Q = torch.stack([torch.stack([q00, q01], -1), torch.stack([q10, q11], -1)], -2)  # (n,K,K,2,2)
    lvl2 = Q.permute(0, 1, 3, 2, 4).reshape(n, m, m)
    return [lvl1, lvl2]


def diag_local_terms(v, lam, dtheta, N):
    """Closed-form local terms for a real diagonal A = diag(lam): s1_i = phi(-h lam_i) v_i and
    s2_ij = D(-h lam_i, -h lam_j) v_i v_j, the 1x1-block case of the plane closed forms
    (plane_engine.py:134-152) and the q -> infinity limit of the block-series leaf
    (ews/core/kernels/blockdiag_engine.py:88-155)."""
    h = dtheta[:, None]
    x = -h * lam[None]
    lvl1 = phi(x) * v
    if N == 1:
        return [lvl1]
    D = divdiff_phi(x[:, :, None], x[:, None, :])
    return [lvl1, D * v[:, :, None] * v[:, None, :]]


@lru_cache(maxsize=None)
def series_coeffs(depth, q):
    """c_m = prod_{j=1..k} 1/(M_j + k - j + 1), M_j = m_j + ... + m_k, for |m| <= q
    (ews/core/series_leaf.py:45-66)."""
    out = []
    for k in range(1, depth + 1):
        C = torch.zeros((q + 1,) * k, dtype=DT)
        for m in iproduct(range(q + 1), repeat=k):
            if sum(m) <= q:
                c = Fraction(1)
                for j in range(1, k + 1):
                    c /= sum(m[j - 1 :]) + k - j + 1
                C[m] = float(c)
        out.append(C)
    return tuple(out)


def series_local_terms(v, dtheta, A, N, q):
    """Series leaf: letters b_0 = v, b_p = (-h/p) A b_{p-1}; level k = sum_m c_m b_{m1} (x) ... (x) b_{mk}
    (ews/core/series_leaf.py:72-126)."""
    letters = [v]
    for p in range(1, q + 1):
        letters.append((-dtheta[:, None] / p) * (letters[-1] @ A.T))
    b = torch.stack(letters, 1)  # (n, q+1, d)
    coeffs = series_coeffs(N, q)
    levels = []
    for k in range(1, N + 1):
        C = coeffs[k - 1]
        if k == 1:
            levels.append(torch.einsum("p,npi->ni", C, b))
        elif k == 2:
            levels.append(torch.einsum("pq,npi,nqj->nij", C, b, b))
        elif k == 3:
            levels.append(torch.einsum("pqr,npi,nqj,nrk->nijk", C, b, b, b))
        else:
            raise NotImplementedError("series oracle covers depth <= 3")
    return levels


def exact_level1(v, dtheta, A):
    """Exact level-1 local term G v, G = int_0^1 e^{-h s A} ds, from the augmented exponential
    expm([[-h A, I], [0, 0]]) = [[E, G], [0, I]] (ews/core/kernels/blockdiag_engine.py:81-112)."""
    n, d = v.shape
    Z = torch.zeros((n, 2 * d, 2 * d), dtype=A.dtype)
    Z[:, :d, :d] = -dtheta[:, None, None] * A
    Z[:, :d, d:] = torch.eye(d, dtype=A.dtype)
    G = torch.linalg.matrix_exp(Z)[:, :d, d:]
    return torch.einsum("nab,nb->na", G, v)


def block_series_local_terms(v, dtheta, A, N, q):
    """Block-series leaf (ews/core/kernels/blockdiag_engine.py:88-155, routed by ews/core/leaf.py:138-175): the
    exact level 1 of the augmented exponential, and at depth 2 the series leaf's order-q level 2 (on a
    block-diagonal A the blockwise letters are the letters of A)."""
    levels = [exact_level1(v, dtheta, A)]
    if N >= 2:
        levels.append(series_local_terms(v, dtheta, A, 2, int(q))[1])
    return levels


def exact_local_terms(v, dtheta, A, N):
    """Exact local levels 1 and 2 of each interval's linear segment under any generator A, from one augmented
    exponential per interval. On the segment the state obeys S1' = -h A S1 + v and S2' = -h (A (+) A) S2 + S1 (x) v
    (S1(0) = S2(0) = 0; A (+) A = A (x) I + I (x) A acts on both factors), so with
    Z = [[-h (A (+) A), I (x) v, 0], [0, -h A, v], [0, 0, 0]] the last column of expm(Z) holds (S2(1), S1(1), 1):
    S1 = int_0^1 e^{-(1-s) h A} v ds and S2 = int_{s<t} e^{-(1-s) h A} v (x) e^{-(1-t) h A} v, the integrals every
    closed-form leaf evaluates (plane_engine.py:134-152, jordan_engine.py:1-15). The oracle of the Jordan leaves
    (jordan_closed / jordan_closed_tables), by a route independent of their derivative tables."""
    n, d = v.shape
    if N > 2:
        raise NotImplementedError("exact local terms are built for depths 1 and 2")
    eye = torch.eye(d, dtype=A.dtype)
    size = d * d + d + 1 if N == 2 else d + 1
    Z = torch.zeros((n, size, size), dtype=A.dtype)
    hA = dtheta[:, None, None] * A[None]
    o1 = d * d if N == 2 else 0
    Z[:, o1:o1 + d, o1:o1 + d] = -hA
    Z[:, o1:o1 + d, -1] = v
    if N == 2:
        Z[:, :d * d, :d * d] = -(torch.einsum("nab,cd->nacbd", hA, eye) +
                                 torch.einsum("ab,ncd->nacbd", eye, hA)).reshape(n, d * d, d * d)
        # (I (x) v) maps S1 to S1 (x) v: row (a, b), column a carries v_b
        Iv = torch.einsum("ac,nb->nabc", eye, v).reshape(n, d * d, d)
        Z[:, :d * d, d * d:d * d + d] = Iv
    E = torch.linalg.matrix_exp(Z)[:, :, -1]
    lvl1 = E[:, o1:o1 + d]
    if N == 1:
        return [lvl1]
    return [lvl1, E[:, :d * d].reshape(n, d, d)]


def _van_loan_displacement(v, dtheta, A, M, method):
    """One augmented exponential per interval (ews/core/van_loan.py:31-88)."""
    n, d = v.shape
    X = torch.zeros((n, d + 1, d + 1), dtype=DT)
    X[:, :d, :d] = A[None] * (dtheta / M)[:, None, None]
    X[:, :d, d] = v / M
    E = expm(X, method)
    powers = [torch.eye(d + 1, dtype=DT).expand(n, d + 1, d + 1)]
    for _ in range(M):
        powers.append(powers[-1] @ E)
    P = torch.stack(powers, 1)  # (n, M+1, d+1, d+1)
    Kv = P[:, :, :d, d]
    W = torch.linalg.inv(P[:, -1, :d, :d])
    return torch.einsum("nij,nmj->nmi", W, Kv)


def _van_loan_uniform(v, h0, A, M, method, eps=1e-12):
    """Shared-exponential fast path with the dt = 0 jump case (ews/core/van_loan.py:91-144)."""
    n, d = v.shape
    if not float(h0) > eps:
        frac = torch.arange(M + 1, dtype=DT) / M
        return frac[None, :, None] * v[:, None, :]
    Ad = A * (h0 / M)
    top = torch.cat([Ad, torch.eye(d, dtype=DT)], 1)
    Xb = torch.cat([top, torch.zeros((d, 2 * d), dtype=DT)], 0)
    Eb = expm(Xb, method)
    EA, F = Eb[:d, :d], Eb[:d, d:]
    Kv = (v / M) @ F.T  # (n, d)
    powers = [torch.eye(d, dtype=DT)]
    for _ in range(M):
        powers.append(powers[-1] @ EA)
    Ssum = [torch.zeros((d, d), dtype=DT)]
    for i in range(M):
        Ssum.append(Ssum[-1] + powers[i])
    S = torch.stack(Ssum, 0)  # (M+1, d, d)
    W = torch.linalg.inv(powers[-1])
    Kvals = torch.einsum("mij,tj->tmi", S, Kv)
    return torch.einsum("ij,tmj->tmi", W, Kvals)


def van_loan_local_terms(v, dtheta, A, N, M, method="cayley", mode="displacement"):
    """Van Loan leaf: M+1 reweighted knots per interval, then their signature
    (ews/core/van_loan.py:163-184, ews/core/signature.py:20-35, routed by ews/core/leaf.py:86-109)."""
    if mode == "displacement":
        knots = _van_loan_displacement(v, dtheta, A, M, method)
    elif mode == "displacement_uniform":
        knots = _van_loan_uniform(v, dtheta[0], A, M, method)
    elif mode == "displacement_uniform_basepoint":
        frac = torch.arange(M + 1, dtype=DT) / M
        k0 = frac[:, None] * v[0][None, :]
        rest = _van_loan_uniform(v[1:], dtheta[1:][0], A, M, method)
        knots = torch.cat([k0[None], rest], 0)
    else:
        raise ValueError(f"unknown reweighting_mode {mode!r}")
    return signature_of_knots(knots, N)


# ============================================================== combine (ews/core/chen_scan.py:124-298)
def chen_scan_prefix(levels, M):
    """Sequential modified Chen recursion (the math every engine implements; pallas_combine.py:300-303,
    581-588): S_k <- M^{(x)k} S_k + sum_{j<k} (M^{(x)j} S_j) (x) s_{k-j} + s_k. Returns the packed prefix
    (n, sum d^k), one row per interval end."""
    N = len(levels)
    n = levels[0].shape[0]
    state = None
    rows = []
    for t in range(n):
        loc = [lv[t : t + 1] for lv in levels]
        if state is None:
            state = loc
        else:
            Mt = M[t : t + 1]
            F = [apply_M(Mt, s) for s in state]
            state = tensor_mult(F, loc)
        rows.append(torch.cat([s.reshape(1, -1) for s in state], 1))
    return torch.cat(rows, 0)


def chen_op_packed(left, right, d, N):
    """Packed Chen operator carrying M (chen_scan.py:124-152): left flowed by M_R, truncated tensor product,
    M = M_L @ M_R."""
    pL, ML = left
    pR, MR = right
    SL = unpack(pL, d, N)
    SR = unpack(pR, d, N)
    SLf = [apply_M(MR, s) for s in SL]
    return pack(tensor_mult(SLf, SR)), ML @ MR


def chen_assoc_scan_prefix(levels, M):
    """Inclusive prefix scan with the packed operator in Hillis-Steele doubling order (any associative
    order is the reference's jax.lax.associative_scan at chen_scan.py:211 up to rounding)."""
    N = len(levels)
    d = levels[0].shape[1]
    p, Ms = pack(levels), M.clone()
    n = p.shape[0]
    off = 1
    while off < n:
        newp, newM = chen_op_packed((p[:-off], Ms[:-off]), (p[off:], Ms[off:]), d, N)
        p = torch.cat([p[:off], newp], 0)
        Ms = torch.cat([Ms[:off], newM], 0)
        off *= 2
    return p


def chen_tree_final(levels, M):
    """Terminal by pairwise tree reduction over a power-of-two padding with identities
    (chen_scan.py:244-298)."""
    N = len(levels)
    d = levels[0].shape[1]
    p, Ms = pack(levels), M
    n = p.shape[0]
    if n > 1:
        target = 1 << (n - 1).bit_length()
        if target != n:
            p = torch.cat([p, torch.zeros((target - n, p.shape[1]), dtype=p.dtype)], 0)
            Ms = torch.cat([Ms, torch.eye(d, dtype=DT)[None].expand(target - n, d, d)], 0)
    while p.shape[0] > 1:
        p, Ms = chen_op_packed((p[0::2], Ms[0::2]), (p[1::2], Ms[1::2]), d, N)
    return p[0]


# ============================================================== the layer (ews/layer.py:154-302)
def block_planes(A):
    """(K, 2) [d_j, w_j] of a rotation-plane A, read as ews/core/leaf.py:130-131 reads it."""
    ii = torch.arange(0, A.shape[0], 2)
    return torch.stack([A[ii, ii], A[ii, ii + 1]], -1)


def local_signatures(path, clock, A, N, leaf="van_loan", M=20, van_loan_expm="cayley",
                     reweighting_mode="displacement", series_q=None):
    """Leaf dispatcher (ews/core/leaf.py:50-198) for the leaves this build runs."""
    v = path[1:] - path[:-1]
    dtheta = clock[1:] - clock[:-1]
    if leaf == "van_loan":
        return van_loan_local_terms(v, dtheta, A, N, M, van_loan_expm, reweighting_mode)
    if leaf == "series":
        return series_local_terms(v, dtheta, A, N, int(series_q))
    if leaf == "block_series":
        return block_series_local_terms(v, dtheta, A, N, series_q)
    if leaf == "plane_closed":
        return plane_local_terms(v, block_planes(A), dtheta, N)
    if leaf == "diag_closed":
        return diag_local_terms(v, torch.diagonal(A), dtheta, N)
    if leaf in ("exact", "jordan_closed", "jordan_closed_tables"):
        return exact_local_terms(v, dtheta, A, N)
    raise ValueError(f"oracle has no leaf {leaf!r}")


def ews_single(path, clock, A, N, readout="prefix", leaf="van_loan", M=20, van_loan_expm="cayley",
               chen_expm="exact", reweighting_mode="displacement", series_q=None,
               terminal_reduce="assoc", output_format="flat"):
    """EWS._single_path (ews/layer.py:154-265): leaf, flows, Chen combine, level-0-prefixed readout."""
    d = path.shape[1]
    dtheta = clock[1:] - clock[:-1]
    levels = local_signatures(path, clock, A, N, leaf, M, van_loan_expm, reweighting_mode, series_q)
    cached = reweighting_mode in ("displacement_uniform", "displacement_uniform_basepoint")
    basepoint = reweighting_mode == "displacement_uniform_basepoint"
    if readout == "terminal" and terminal_reduce == "tree":
        Mt = flows(dtheta, A, chen_expm, False, False)  # the tree always takes per-interval flows (:294)
        fin = chen_tree_final(levels, Mt)
        if output_format == "list":
            return unpack(fin[None], d, N)
        return torch.cat([torch.ones(1, dtype=fin.dtype), fin])
    Mt = flows(dtheta, A, chen_expm, cached, basepoint)
    prefix = chen_scan_prefix(levels, Mt)
    if readout == "terminal":
        fin = prefix[-1]
        if output_format == "list":
            return unpack(fin[None], d, N)
        return torch.cat([torch.ones(1, dtype=fin.dtype), fin])
    if output_format == "list":
        return unpack(prefix, d, N)
    flat = torch.cat([torch.ones((prefix.shape[0], 1), dtype=prefix.dtype), prefix], 1)
    if readout == "prefix":
        return flat
    if readout == "mean":
        return flat.mean(0)
    if readout == "max":
        return flat.max(0).values
    raise ValueError(readout)


def ews(path, clock, A, N, readout="prefix", **kw):
    """Batched call (ews/layer.py:294-301): path (B, L, d), clock (B, L)."""
    return torch.stack([ews_single(path[b], clock[b], A, N, readout, **kw) for b in range(path.shape[0])])


# ============================================================== log-signature (ews/layer.py:417-517)
def lyndon_words(N, d):
    """Lyndon words of lengths 1..N over {0..d-1}, each length in lexicographic order (Duval's algorithm)."""
    words = [[] for _ in range(N)]
    w = [-1]
    while w:
        w[-1] += 1
        words[len(w) - 1].append(tuple(w))
        m = len(w)
        while len(w) < N:
            w.append(w[len(w) - m])
        while w and w[-1] == d - 1:
            w.pop()
    return [sorted(ws) for ws in words]


def tensor_log(levels):
    """Truncated log of 1 + X (X = levels 1..N): sum_{n=1}^N (-1)^{n+1} X^{(x)n} / n."""
    N = len(levels)
    out = [lv.clone() for lv in levels]
    P = [lv for lv in levels]
    for n in range(2, N + 1):
        Q = []
        for k in range(1, N + 1):
            acc = torch.zeros_like(levels[k - 1])
            for j in range(1, k):
                acc = acc + outer(P[j - 1], levels[k - j - 1])
            Q.append(acc)
        P = Q
        out = [o + ((-1) ** (n + 1)) * q / n for o, q in zip(out, P)]
    return out


def log_compress(levels, d):
    """Compressed log: each level's coefficients at its Lyndon words, concatenated (layer.py:488-517)."""
    N = len(levels)
    logs = tensor_log(levels)
    words = lyndon_words(N, d)
    n = levels[0].shape[0]
    parts = []
    for k in range(1, N + 1):
        flat = logs[k - 1].reshape(n, -1)
        idx = [sum(c * d ** (k - 1 - i) for i, c in enumerate(w)) for w in words[k - 1]]
        parts.append(flat[:, idx])
    return torch.cat(parts, 1)


def log_ews_single(path, clock, A, N, readout="terminal", **kw):
    """LogEWS._single_path (ews/layer.py:488-517): log each prefix row, then pool."""
    d = path.shape[1]
    if readout == "terminal":
        lv = ews_single(path, clock, A, N, "terminal", output_format="list", **kw)
        return log_compress(lv, d)[0]
    lv = ews_single(path, clock, A, N, "prefix", output_format="list", **kw)
    feat = log_compress(lv, d)
    if readout == "prefix":
        return feat
    if readout == "mean":
        return feat.mean(0)
    if readout == "max":
        return feat.max(0).values
    raise ValueError(readout)
