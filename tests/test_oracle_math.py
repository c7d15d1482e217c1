"""Pins for the float64 oracle beyond the golden files: each check is chosen so that a plausible slip in the
oracle (a dropped term, a swapped index, a wrong sign, a transposed operand) fails it.

* local terms (plane / diagonal closed forms, series leaf) against Gauss-Legendre quadrature of their
  defining integrals with scipy's expm (the reference's own quadrature oracle, tests/test_jordan_engine.py:240-290);
* plane / diagonal closed forms against the series leaf at q = 24 (tests/test_engines.py:227-248);
* Van Loan leaf: level 1 exact for any M, level 2 converging as O(1/M^2) to the exact term;
* expm methods against scipy / their textbook formulas;
* sequential == associative == tree Chen combine (tests/test_engines.py:198-224);
* depth-1 prefix == the exact affine (Van Loan) recursion built with scipy.linalg.expm (tests/test_block.py:559-596);
* A = 0: the classical signature, whose depth-2 log is the Levy area (tests/test_log_ews.py:82-96);
* exp(log(EWS)) == EWS and the Witt dimensions (tests/test_log_ews.py:99-121);
* autograd of the oracle against central finite differences (tests/test_log_ews.py:149-175).
"""

import math

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import ews_oracle as O

DT = torch.float64


def _rng(seed=0):
    return np.random.default_rng(seed)


def _planes_A(K, rng):
    A = np.zeros((2 * K, 2 * K))
    for j in range(K):
        d, w = rng.uniform(0.05, 1.5), rng.uniform(-2.0, 2.0)
        A[2 * j : 2 * j + 2, 2 * j : 2 * j + 2] = [[d, w], [-w, d]]
    return A


def _quad_local(v, h, A, N, nodes=24):
    """Levels 1..N of the interval's local term by nested Gauss-Legendre quadrature of
    x(u) = e^{-(h-u)A} v / h over the ordered simplex of [0, h]."""
    g, w = np.polynomial.legendre.leggauss(nodes)
    d = len(v)

    def x(u):
        return scipy.linalg.expm(-(h - u) * A) @ v / h

    def lvl1(a, b):
        us = (b - a) / 2 * g + (a + b) / 2
        return sum(wi * x(ui) for wi, ui in zip(w, us)) * (b - a) / 2

    out = [lvl1(0.0, h)]
    if N >= 2:
        us = h / 2 * g + h / 2
        s2 = np.zeros((d, d))
        for wi, u2 in zip(w, us):
            s2 += wi * np.outer(lvl1(0.0, u2), x(u2))
        out.append(s2 * h / 2)
    return out


@pytest.mark.parametrize("h", [0.05, 0.7, 2.5])
def test_plane_closed_form_matches_quadrature(h):
    rng = _rng(1)
    K = 3
    A = _planes_A(K, rng)
    v = rng.normal(size=2 * K)
    got = O.plane_local_terms(torch.tensor(v[None]), O.block_planes(torch.tensor(A)), torch.tensor([h], dtype=DT), 2)
    ref = _quad_local(v, h, A, 2)
    for g_, r_ in zip(got, ref):
        np.testing.assert_allclose(g_[0].numpy(), r_, rtol=0, atol=1e-11 * max(1, np.abs(r_).max()))


@pytest.mark.parametrize("h", [1e-4, 0.3, 4.0])
def test_diag_closed_form_matches_quadrature(h):
    rng = _rng(2)
    lam = rng.uniform(-0.5, 3.0, size=5)
    v = rng.normal(size=5)
    got = O.diag_local_terms(torch.tensor(v[None]), torch.tensor(lam), torch.tensor([h], dtype=DT), 2)
    ref = _quad_local(v, h, np.diag(lam), 2)
    for g_, r_ in zip(got, ref):
        np.testing.assert_allclose(g_[0].numpy(), r_, rtol=0, atol=1e-11 * max(1, np.abs(r_).max()))


def test_series_leaf_matches_quadrature_dense_A():
    rng = _rng(3)
    d, h = 4, 0.4
    A = rng.normal(size=(d, d)) * 0.8
    v = rng.normal(size=d)
    got = O.series_local_terms(torch.tensor(v[None]), torch.tensor([h], dtype=DT), torch.tensor(A), 2, 24)
    ref = _quad_local(v, h, A, 2)
    for g_, r_ in zip(got, ref):
        np.testing.assert_allclose(g_[0].numpy(), r_, rtol=0, atol=1e-11)


def test_series_level3_matches_nested_quadrature():
    rng = _rng(4)
    d, h = 3, 0.5
    A = rng.normal(size=(d, d)) * 0.5
    v = rng.normal(size=d)
    g, w = np.polynomial.legendre.leggauss(14)

    def x(u):
        return scipy.linalg.expm(-(h - u) * A) @ v / h

    def S(level, b):
        # iterated integral of x over {0 < u1 < ... < u_level < b}
        us = b / 2 * g + b / 2
        if level == 1:
            return sum(wi * x(ui) for wi, ui in zip(w, us)) * b / 2
        acc = 0
        for wi, ui in zip(w, us):
            acc = acc + wi * np.multiply.outer(S(level - 1, ui), x(ui))
        return acc * b / 2

    got = O.series_local_terms(torch.tensor(v[None]), torch.tensor([h], dtype=DT), torch.tensor(A), 3, 26)
    np.testing.assert_allclose(got[2][0].numpy(), S(3, h), rtol=0, atol=1e-10)


def test_closed_forms_match_series_q24():
    rng = _rng(5)
    n, K = 7, 3
    A = _planes_A(K, rng) * 0.5
    v = torch.tensor(rng.normal(size=(n, 2 * K)))
    dth = torch.tensor(rng.uniform(0.05, 0.5, size=n))
    pc = O.plane_local_terms(v, O.block_planes(torch.tensor(A)), dth, 2)
    se = O.series_local_terms(v, dth, torch.tensor(A), 2, 24)
    for a, b in zip(pc, se):
        assert float((a - b).abs().max()) < 1e-10
    lam = torch.tensor(rng.uniform(0.1, 2.0, size=6))
    v6 = torch.tensor(rng.normal(size=(n, 6)))
    dc = O.diag_local_terms(v6, lam, dth, 2)
    se = O.series_local_terms(v6, dth, torch.diag(lam), 2, 24)
    for a, b in zip(dc, se):
        assert float((a - b).abs().max()) < 1e-10


def test_van_loan_level1_exact_level2_second_order():
    rng = _rng(6)
    d, n = 3, 4
    A = torch.tensor(rng.normal(size=(d, d)) * 0.7)
    v = torch.tensor(rng.normal(size=(n, d)))
    dth = torch.tensor(rng.uniform(0.3, 1.0, size=n))
    exact = O.series_local_terms(v, dth, A, 2, 30)
    errs = []
    for M in (8, 16, 32):
        vl = O.van_loan_local_terms(v, dth, A, 2, M, "exact", "displacement")
        assert float((vl[0] - exact[0]).abs().max()) < 1e-12
        errs.append(float((vl[1] - exact[1]).abs().max()))
    assert 3.5 < errs[0] / errs[1] < 4.5 and 3.5 < errs[1] / errs[2] < 4.5


def test_van_loan_uniform_equals_displacement_on_uniform_clock():
    rng = _rng(7)
    d, n = 4, 5
    A = torch.tensor(rng.normal(size=(d, d)) * 0.5)
    v = torch.tensor(rng.normal(size=(n, d)))
    dth = torch.full((n,), 0.3, dtype=DT)
    a = O.van_loan_local_terms(v, dth, A, 2, 5, "exact", "displacement")
    b = O.van_loan_local_terms(v, dth, A, 2, 5, "exact", "displacement_uniform")
    for x, y in zip(a, b):
        assert float((x - y).abs().max()) < 1e-12


# The approximate exponentials (ews/core/expm_approx.py:13-31) pinned by what the mathematics fixes, not by their
# formulas: the order of agreement with the exact exponential (error ratio under halving X), the leading error term
# (Euler X^2/2; Cayley -X^3/12; the [2/2] Pade X^5/720, the Pade error constant m! n! / ((m+n)! (m+n+1)!)),
# orthogonality on skew-symmetric X for the two diagonal Pade schemes (r(-x) = 1/r(x)), and r(X) r(-X) = I. A
# wrong sign, a dropped or mis-scaled term, or a solve against the wrong side fails one of these.
_EXPM_ORDER = {"euler": (2, 0.5), "cayley": (3, -1.0 / 12.0), "pade": (5, 1.0 / 720.0)}
_EXPM_SCALES = {"euler": (0.08, 0.04, 0.02, 0.01), "cayley": (0.08, 0.04, 0.02, 0.01), "pade": (0.2, 0.1, 0.05, 0.025)}


def test_expm_exact_is_scipy():
    X = _rng(8).normal(size=(4, 4)) * 0.3
    np.testing.assert_allclose(O.expm(torch.tensor(X), "exact").numpy(), scipy.linalg.expm(X), rtol=1e-12,
                               atol=1e-13)


@pytest.mark.parametrize("method", ["euler", "cayley", "pade"])
def test_expm_approx_order_and_leading_term(method):
    p, c = _EXPM_ORDER[method]
    rng = _rng(81)
    X0 = rng.normal(size=(5, 5))  # a general (non-normal) matrix
    X0 /= np.linalg.norm(X0, 2)
    errs = []
    for e in _EXPM_SCALES[method]:  # the [2/2] Pade error reaches float64 rounding near |X| = 0.01
        X = e * X0
        E = scipy.linalg.expm(X) - O.expm(torch.tensor(X), method).numpy()
        lead = c * np.linalg.matrix_power(X, p)
        # the leading term carries the error to relative accuracy O(|X|)
        assert np.abs(E - lead).max() <= 2.0 * e * np.abs(lead).max(), (method, e)
        errs.append(np.abs(E).max())
    for a, b in zip(errs, errs[1:]):
        assert abs(np.log2(a / b) - p) < 0.2, (method, errs)


@pytest.mark.parametrize("method", ["cayley", "pade"])
def test_expm_diagonal_pade_orthogonal_on_skew(method):
    rng = _rng(82)
    Y = rng.normal(size=(6, 6))
    S = (Y - Y.T) * 0.7  # skew-symmetric, not small
    Q = O.expm(torch.tensor(S), method).numpy()
    np.testing.assert_allclose(Q.T @ Q, np.eye(6), atol=1e-12)
    assert abs(np.linalg.det(Q) - 1.0) < 1e-12
    Y = rng.normal(size=(6, 6)) * 0.4
    R = O.expm(torch.tensor(Y), method).numpy() @ O.expm(torch.tensor(-Y), method).numpy()
    np.testing.assert_allclose(R, np.eye(6), atol=1e-12)


def test_expm_euler_is_not_symmetric():
    # Euler is the one scheme with r(X) r(-X) = I - X^2, not I
    Y = _rng(83).normal(size=(4, 4)) * 0.3
    R = O.expm(torch.tensor(Y), "euler").numpy() @ O.expm(torch.tensor(-Y), "euler").numpy()
    np.testing.assert_allclose(R, np.eye(4) - Y @ Y, atol=1e-13)


@pytest.mark.parametrize("N", [1, 2, 3])
def test_sequential_assoc_tree_agree(N):
    rng = _rng(9)
    d, n = 3, 11
    A = torch.tensor(rng.normal(size=(d, d)) * 0.4)
    v = torch.tensor(rng.normal(size=(n, d)) * 0.5)
    dth = torch.tensor(rng.uniform(0.1, 0.6, size=n))
    lv = O.series_local_terms(v, dth, A, N, 20)
    M = O.flows(dth, A)
    seq = O.chen_scan_prefix(lv, M)
    asc = O.chen_assoc_scan_prefix(lv, M)
    tree = O.chen_tree_final(lv, M)
    assert float((seq - asc).abs().max()) < 1e-12
    assert float((seq[-1] - tree).abs().max()) < 1e-12


def test_depth1_prefix_is_the_exact_affine_recursion():
    rng = _rng(10)
    d, L = 4, 12
    A = rng.normal(size=(d, d)) * 0.6
    path = np.cumsum(rng.normal(size=(L, d)), 0)
    clock = np.cumsum(rng.uniform(0.1, 0.5, size=L))
    got = O.ews_single(torch.tensor(path), torch.tensor(clock), torch.tensor(A), 1, "prefix",
                       leaf="series", series_q=30)
    y = np.zeros(d)
    rows = []
    for t in range(L - 1):
        h = clock[t + 1] - clock[t]
        v = path[t + 1] - path[t]
        Aug = np.zeros((d + 1, d + 1))
        Aug[:d, :d] = -h * A
        Aug[:d, d] = v
        E = scipy.linalg.expm(Aug)  # [[e^{-hA}, phi(-hA) v], [0, 1]]
        y = E[:d, :d] @ y + E[:d, d]
        rows.append(np.concatenate([[1.0], y]))
    np.testing.assert_allclose(got.numpy(), np.array(rows), rtol=0, atol=1e-11)


def test_zero_drift_is_the_signature_and_log_is_levy_area():
    rng = _rng(11)
    d, L = 3, 9
    path = np.cumsum(rng.normal(size=(L, d)), 0)
    clock = np.linspace(0, 1, L)
    A = torch.zeros((d, d), dtype=DT)
    for leaf in ("van_loan", "series", "diag_closed"):
        lv = O.ews_single(torch.tensor(path), torch.tensor(clock), A, 2, "terminal", leaf=leaf, M=3,
                          series_q=5, output_format="list")
        inc = np.diff(path, axis=0)
        S1 = inc.sum(0)
        # level 2 of a piecewise-linear path: sum_{s<t} D_s (x) D_t + sum_t D_t (x) D_t / 2
        S2 = sum(np.outer(inc[s], inc[t]) for s in range(L - 1) for t in range(s + 1, L - 1))
        S2 = S2 + sum(np.outer(x, x) for x in inc) / 2
        np.testing.assert_allclose(lv[0][0].numpy(), S1, atol=1e-12)
        np.testing.assert_allclose(lv[1][0].numpy(), S2, atol=1e-11)
    logf = O.log_ews_single(torch.tensor(path), torch.tensor(clock), A, 2, "terminal", leaf="series", series_q=5)
    inc = np.diff(path, axis=0)
    area = sum(np.outer(inc[s], inc[t]) - np.outer(inc[t], inc[s]) for s in range(L - 1)
               for t in range(s + 1, L - 1)) / 2
    expect = np.concatenate([inc.sum(0), [area[i, j] for i in range(d) for j in range(i + 1, d)]])
    np.testing.assert_allclose(logf.numpy(), expect, atol=1e-11)


def test_exp_of_log_recovers_ews_and_witt_dims():
    rng = _rng(12)
    d, N, L = 3, 3, 8
    path = torch.tensor(np.cumsum(0.3 * rng.normal(size=(L, d)), 0))
    clock = torch.linspace(0, 1, L, dtype=DT)
    A = torch.tensor(0.5 * rng.normal(size=(d, d)))
    lv = O.ews_single(path, clock, A, N, "terminal", leaf="series", series_q=20, output_format="list")
    lg = O.tensor_log(lv)
    # exp(X) = sum X^n / n!, truncated
    out = [x.clone() for x in lg]
    P = lg
    for n in range(2, N + 1):
        P = [sum((O.outer(P[j - 1], lg[k - j - 1]) for j in range(1, k)), torch.zeros_like(lg[k - 1]))
             for k in range(1, N + 1)]
        out = [o + p / math.factorial(n) for o, p in zip(out, P)]
    for a, b in zip(out, lv):
        assert float((a - b).abs().max()) < 1e-12
    for dd, NN, expect in [(3, 3, 14), (4, 2, 10), (2, 4, 8)]:
        assert sum(len(w) for w in O.lyndon_words(NN, dd)) == expect


def test_oracle_gradients_match_finite_differences():
    rng = _rng(13)
    K, L = 2, 7
    A0 = _planes_A(K, rng) * 0.5
    path = torch.tensor(np.cumsum(rng.normal(size=(L, 2 * K)) * 0.4, 0))
    clock = torch.tensor(np.cumsum(rng.uniform(0.2, 0.6, size=L)))
    wts = torch.tensor(rng.normal(size=(L - 1, 1 + 2 * K + 4 * K * K)))

    def loss(dw, pth, clk):
        A = torch.zeros((2 * K, 2 * K), dtype=DT)
        for j in range(K):
            A = A + torch.zeros_like(A).index_put_((torch.tensor([2 * j, 2 * j, 2 * j + 1, 2 * j + 1]),
                                                   torch.tensor([2 * j, 2 * j + 1, 2 * j, 2 * j + 1])),
                                                  torch.stack([dw[j, 0], dw[j, 1], -dw[j, 1], dw[j, 0]]))
        out = O.ews_single(pth, clk, A, 2, "prefix", leaf="plane_closed")
        return (out * wts).sum()

    dw = O.block_planes(torch.tensor(A0)).clone().requires_grad_(True)
    p = path.clone().requires_grad_(True)
    c = clock.clone().requires_grad_(True)
    gdw, gp, gc = torch.autograd.grad(loss(dw, p, c), (dw, p, c))
    eps = 1e-6
    base = [dw.detach(), p.detach(), c.detach()]
    for which, grad in enumerate((gdw, gp, gc)):
        flat = base[which].reshape(-1)
        for idx in range(0, flat.numel(), max(1, flat.numel() // 5)):
            e = torch.zeros_like(flat)
            e[idx] = eps
            args_p, args_m = list(base), list(base)
            args_p[which] = (flat + e).reshape(base[which].shape)
            args_m[which] = (flat - e).reshape(base[which].shape)
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            g = grad.reshape(-1)[idx]
            assert abs(float(fd - g)) <= 1e-6 * max(1.0, abs(float(fd))), (which, idx, float(fd), float(g))


def _quad_series(v, h, A, N, q, nodes=32):
    """The order-q series leaf by another route: the degree-<= q part in h of the defining integral of the local
    term, i.e. x(u) = e^{-h(1-u)A} v with its exponential replaced by its Taylor polynomial of degree q in h,
    integrated over the ordered simplex of [0, 1] by Gauss-Legendre quadrature (exact: polynomial integrands).
    Level 2 keeps the products of total degree <= q in h, the truncation of ews/core/series_leaf.py:8-25."""
    g, w = np.polynomial.legendre.leggauss(nodes)
    d = len(v)
    P = [np.linalg.matrix_power(-h * A, n) / math.factorial(n) for n in range(q + 1)]

    def terms(u):  # degree-n parts of x(u), n = 0..q
        return [P[n] @ v * (1.0 - u) ** n for n in range(q + 1)]

    us, ws = g / 2 + 0.5, w / 2
    lvl1 = sum(wi * sum(terms(ui)) for wi, ui in zip(ws, us))
    out = [lvl1]
    if N >= 2:
        s2 = np.zeros((d, d))
        for wi, u2 in zip(ws, us):
            t2 = terms(u2)
            # inner integral over u1 in [0, u2] of the degree-n1 parts, paired with degree n2 <= q - n1
            inner = [np.zeros(d) for _ in range(q + 1)]
            for wj, gj in zip(w, g):
                u1 = u2 * (gj + 1) / 2
                t1 = terms(u1)
                for n1 in range(q + 1):
                    inner[n1] += wj * u2 / 2 * t1[n1]
            for n1 in range(q + 1):
                for n2 in range(q + 1 - n1):
                    s2 += wi * np.outer(inner[n1], t2[n2])
        out.append(s2)
    return out


@pytest.mark.parametrize("q", [1, 3, 6, 10])
@pytest.mark.parametrize("kind", ["planes", "diag"])
def test_series_truncation_matches_truncated_integral(q, kind):
    """The oracle's order-q series leaf on a plane / diagonal generator at a unit-size step, where the truncation
    is far above float64 resolution, against the truncated defining integral."""
    rng = _rng(11)
    A = _planes_A(3, rng) if kind == "planes" else np.diag(rng.uniform(0.1, 2.0, size=6))
    v = rng.normal(size=6)
    h = 1.3
    got = O.series_local_terms(torch.tensor(v[None]), torch.tensor([h], dtype=DT), torch.tensor(A), 2, q)
    ref = _quad_series(v, h, A, 2, q)
    for g_, r_ in zip(got, ref):
        np.testing.assert_allclose(g_[0].numpy(), r_, rtol=0, atol=1e-12 * max(1, np.abs(r_).max()))
    # and the truncation is visible: the exact closed form differs at this q
    exact = O.local_signatures(torch.tensor(np.stack([np.zeros(6), v])), torch.tensor([0.0, h], dtype=DT),
                               torch.tensor(A), 2, leaf="plane_closed" if kind == "planes" else "diag_closed")
    assert (exact[1][0] - got[1][0]).abs().max() > 1e-6 * exact[1][0].abs().max()


@pytest.mark.parametrize("q", [2, 6])
def test_block_series_leaf_levels(q):
    """Block-series leaf: level 1 is exact (the closed form), level 2 is the order-q series."""
    rng = _rng(12)
    A = torch.tensor(_planes_A(3, rng))
    v = torch.tensor(rng.normal(size=(4, 6)))
    h = torch.tensor([0.2, 0.9, 1.7, 3.0], dtype=DT)
    got = O.block_series_local_terms(v, h, A, 2, q)
    closed = O.plane_local_terms(v, O.block_planes(A), h, 2)
    series = O.series_local_terms(v, h, A, 2, q)
    torch.testing.assert_close(got[0], closed[0], rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got[1], series[1], rtol=0, atol=0)


def _jordan_A(kind, size, K, rng):
    """Block-diagonal Jordan chains as AParamJordanRepeated materialises them: a real chain is lambda on the
    diagonal with ones above; a complex chain of size 2k is R = [[a, -b], [b, a]] in every 2x2 slot with the 2x2
    identity above."""
    A = np.zeros((K * size, K * size))
    for j in range(K):
        o = j * size
        if kind == "real":
            lam = rng.uniform(0.2, 2.0)
            A[o:o + size, o:o + size] = lam * np.eye(size) + np.diag(np.ones(size - 1), 1)
        else:
            a, b = rng.uniform(0.2, 2.0), rng.uniform(-3.0, 3.0)
            R = np.array([[a, -b], [b, a]])
            k = size // 2
            A[o:o + size, o:o + size] = np.kron(np.eye(k), R) + np.kron(np.diag(np.ones(k - 1), 1), np.eye(2))
    return A


def _quad_local_graded(v, h, A, N, nodes=16, panels=14):
    """_quad_local with composite Gauss-Legendre panels graded toward the interval's end (breakpoints
    h (1 - 2^-m)), for steps where e^{-(h-u) A} is concentrated near u = h."""
    g, w = np.polynomial.legendre.leggauss(nodes)
    cuts = [h * (1 - 2.0 ** -m) for m in range(panels)] + [h]

    def x(u):
        return scipy.linalg.expm(-(h - u) * A) @ v / h

    def rule(a, b):
        pts, wts = [], []
        for lo, hi in zip(cuts[:-1], cuts[1:]):
            lo, hi = max(lo, a), min(hi, b)
            if hi > lo:
                pts += list((hi - lo) / 2 * g + (hi + lo) / 2)
                wts += list(w * (hi - lo) / 2)
        return pts, wts

    def lvl1(a, b):
        pts, wts = rule(a, b)
        return sum(wi * x(ui) for wi, ui in zip(wts, pts))

    out = [lvl1(0.0, h)]
    if N >= 2:
        pts, wts = rule(0.0, h)
        out.append(sum(wi * np.outer(lvl1(0.0, u2), x(u2)) for wi, u2 in zip(wts, pts)))
    return out


@pytest.mark.parametrize("kind,size,h", [("real", 3, 12.0), ("real", 2, 30.0), ("complex", 4, 8.0)])
def test_exact_leaf_matches_graded_quadrature_jordan(kind, size, h):
    """The exact leaf (one augmented exponential per interval), the oracle of the Jordan leaves, against graded
    quadrature of the defining integrals at steps with h ||A||_1 up to about 60."""
    rng = _rng(7)
    A = _jordan_A(kind, size, 2, rng)
    v = rng.normal(size=A.shape[0])
    ref = _quad_local_graded(v, h, A, 2)
    got = O.exact_local_terms(torch.tensor(v[None]), torch.tensor([h]), torch.tensor(A), 2)
    for lvl, r in zip(got, ref):
        err = float(np.abs(lvl[0].numpy() - r).max() / np.abs(r).max())
        assert err < 1e-9, err


@pytest.mark.parametrize("h", [0.3, 4.0, 25.0])
def test_exact_leaf_matches_closed_forms(h):
    """On diagonals and rotation planes the exact leaf equals the closed forms at any step."""
    rng = _rng(3)
    v = torch.tensor(rng.normal(size=(3, 4)))
    hh = torch.full((3,), h, dtype=torch.float64)
    lam = torch.tensor(rng.uniform(0.1, 2.0, 4))
    for a, b in zip(O.exact_local_terms(v, hh, torch.diag(lam), 2), O.diag_local_terms(v, lam, hh, 2)):
        assert float((a - b).abs().max() / b.abs().max()) < 1e-11
    Ap = torch.tensor(_planes_A(2, rng))
    for a, b in zip(O.exact_local_terms(v, hh, Ap, 2), O.plane_local_terms(v, O.block_planes(Ap), hh, 2)):
        assert float((a - b).abs().max() / b.abs().max()) < 1e-11


def test_exact_leaf_matches_series_at_small_steps():
    """Any generator: at h ||A|| about 0.1 the order-30 series leaf equals the exact local terms."""
    rng = _rng(11)
    A = torch.tensor(_jordan_A("complex", 6, 1, rng) + 0.3 * rng.normal(size=(6, 6)))
    v = torch.tensor(rng.normal(size=(4, 6)))
    h = torch.tensor(rng.uniform(0.005, 0.03, 4))
    for a, b in zip(O.exact_local_terms(v, h, A, 2), O.series_local_terms(v, h, A, 2, 30)):
        assert float((a - b).abs().max() / b.abs().max()) < 1e-12
