"""TEST INFRASTRUCTURE ONLY (never imported by the product): a float64 torch checker for the depth-1 EWS of a
block-diagonal generator of uniform chains, vectorised over samples and chains, for full-size parity checks where the
per-step loops of oracle/ews_oracle.py are too slow (the PPG block: L = 49,920, 16 chains).

What it restates (reference file:line):
  - chains read off A's first rows: ews/core/kernels/jordan_engine.py:324-353 (real chain lambda, eps = A[f, f+1];
    complex chain c = A[f, f] + i A[f+1, f], eps = A[f, f+2], coordinates P_i = v_2i + i v_2i+1);
  - the flows exp(-h J) = e^{-h c} sum_p (-h eps)^p / p! Nil^p: ews/core/kernels/combine.py:143-190
    (jordan_block_operators), with the step of chen_scan.py:155-168's flow modes;
  - level 1, phi(-h J) v = sum_p (-h)^p phi^(p)(-h c) / p! (eps Nil)^p v: jordan_engine.py:246-321 at N = 1, phi^(r)
    by its entire series or the recurrence from e^x (jordan_engine.py:175-243); the series leaf's level 1
    (ews/core/series_leaf.py:72-113) with phi replaced by its degree-q Taylor polynomial;
  - the depth-1 Chen combine S_t = M_t S_{t-1} + s_t (chen_scan.py:125-152 at N = 1), here by an associative
    (Hillis-Steele) scan over time, as chen_associative_scan_prefix_packed_with_M runs it (chen_scan.py:172-214).

It is pinned in tests/test_oracle_chain.py to oracle/ews_oracle.py by independent routes: the exact leaf there is
one augmented matrix exponential per interval (itself pinned against quadrature), the series leaf assembles its
letters (b_p = (-h/p) A b_{p-1}), the Van Loan leaf forms its knots, and the combine is the sequential Chen loop with
torch.linalg.matrix_exp flows; forward and autograd gradients.
"""

from __future__ import annotations

import math

import torch

C128 = torch.complex128


def chains_of(A, kind, size):
    """(c (K,) complex, eps (K,) real): the chains' eigenvalues and couplings read from their first rows."""
    d = A.shape[0]
    f = torch.arange(0, d, size)
    if kind == "real":
        c = torch.complex(A[f, f], torch.zeros_like(A[f, f]))
        eps = A[f, f + 1] if size > 1 else torch.zeros_like(A[f, f])
    else:
        c = torch.complex(A[f, f], A[f + 1, f])
        eps = A[f, f + 2] if size > 2 else torch.zeros_like(A[f, f])
    return c, eps


def u_table(x, R, q=0):
    """[phi^(r)(x) / r! for r < R] (q = 0), or of the degree-q Taylor polynomial of phi (q >= 1)."""
    if q > 0:
        out = []
        for r in range(R):
            acc = torch.zeros_like(x)
            for n in range(q, r - 1, -1):  # Horner in x over sum_{n=r..q} C(n, r) x^(n-r) / (n+1)!
                acc = acc * x + math.comb(n, r) / math.factorial(n + 1)
            out.append(acc)
        return out
    small = x.abs() <= 2.0
    xs = torch.where(small, x, torch.zeros_like(x))
    ser = [torch.zeros_like(x) for _ in range(R)]
    t = torch.ones_like(x)
    for j in range(40):
        for r in range(R):
            ser[r] = ser[r] + t / (j + r + 1)
        t = t * xs / (j + 1)
    xb = torch.where(small, torch.ones_like(x), x)
    e = torch.exp(xb)
    rec = [(e - 1) / xb]
    for r in range(1, R):
        rec.append((e - r * rec[-1]) / xb)
    return [torch.where(small, ser[r], rec[r]) / math.factorial(r) for r in range(R)]


def _mode_step(h, clock, mode):
    """Per-interval steps under a flow mode (chen_scan.py:155-168): own, theta1 - theta0, or theta2 - theta1 with
    interval 0 none."""
    if mode == "per_interval":
        return h
    if mode == "cached":
        return (clock[:, 1] - clock[:, 0])[:, None].expand_as(h)
    ref = (clock[:, 2] - clock[:, 1])[:, None].expand_as(h)
    return torch.cat([torch.zeros_like(h[:, :1]), ref[:, 1:]], 1)


def _act(a, s):
    """(E s)_i = sum_p a_p s_{i+p}: a (..., k) coefficients of Nil^p, s (..., k)."""
    k = s.shape[-1]
    out = []
    for i in range(k):
        acc = torch.zeros_like(s[..., 0])
        for p in range(k - i):
            acc = acc + a[..., p] * s[..., i + p]
        out.append(acc)
    return torch.stack(out, -1)


def _compose(a2, a1):
    """E2 E1 as coefficients of Nil^p (truncated product of polynomials in Nil)."""
    k = a1.shape[-1]
    out = []
    for r in range(k):
        acc = torch.zeros_like(a1[..., 0])
        for p in range(r + 1):
            acc = acc + a2[..., p] * a1[..., r - p]
        out.append(acc)
    return torch.stack(out, -1)


def chain_depth1(path, clock, A, kind, size, flow_mode="per_interval", leaf_mode="per_interval", readout="prefix",
                 level0=True, series_q=0):
    """path (B, L, d), clock (B, L), A (d, d), float64 -> prefix rows (B, L-1, level0 + d) or terminal (B, W)."""
    B, L, d = path.shape
    k = size if kind == "real" else size // 2
    K = d // size
    c, eps = chains_of(A, kind, size)  # (K,)
    v = path[:, 1:] - path[:, :-1]
    if kind == "real":
        P = torch.complex(v, torch.zeros_like(v)).reshape(B, L - 1, K, k)
    else:
        vv = v.reshape(B, L - 1, K, k, 2)
        P = torch.complex(vv[..., 0], vv[..., 1])
    h = clock[:, 1:] - clock[:, :-1]  # (B, n)
    hl = _mode_step(h, clock, leaf_mode)[..., None]  # (B, n, 1)
    hf = _mode_step(h, clock, flow_mode)[..., None]
    x = -hl.to(C128) * c  # (B, n, K)
    u = u_table(x, k, series_q)
    epsc = eps.to(C128)
    # level 1: s_i = sum_p (-hl)^p u_p (eps Nil)^p P
    lc = torch.stack([((-hl) ** p).to(C128) * u[p] * epsc**p for p in range(k)], -1)  # (B, n, K, k)
    s = _act(lc, P)
    # flows: a_p = e^{-hf c} (-hf eps)^p / p!
    ef = torch.exp(-hf.to(C128) * c)
    a = torch.stack([ef * ((-hf).to(C128) * epsc) ** p / math.factorial(p) for p in range(k)], -1)
    # associative scan over time: (a, s) at t composed with everything before it
    n = L - 1
    off = 1
    while off < n:
        a_new = _compose(a[:, off:], a[:, :-off])
        s_new = _act(a[:, off:], s[:, :-off]) + s[:, off:]
        a = torch.cat([a[:, :off], a_new], 1)
        s = torch.cat([s[:, :off], s_new], 1)
        off *= 2
    if kind == "real":
        rows = s.real.reshape(B, n, d)
    else:
        rows = torch.stack([s.real, s.imag], -1).reshape(B, n, d)
    if level0:
        rows = torch.cat([torch.ones_like(rows[..., :1]), rows], -1)
    if readout == "terminal":
        return rows[:, -1]
    if readout == "mean":
        return rows.mean(1)
    if readout == "max":
        return rows.max(1).values
    return rows
