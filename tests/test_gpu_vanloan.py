"""GPU parity of the Van Loan leaf (the reference's default leaf) and of the flow schemes on the dense kernels.

Bars: forward max relative error <= 1e-5 with the reference's metric
max|a-b| / max|b| (tests/test_engines.py:31-33), each level on its own scale.

* The reference's pinned logits (tests/golden/reference_kernel_outputs.npz, from the reference's
  tests/test_kernel_outputs_pinned.py): the fixture classifier's 13 logits are all Van Loan (M = 4, exact
  exponentials) in the three reweighting modes, both terminal reductions, mean / max readouts and the depth-2
  log-signature; here the EWS features come from the GPU layer and the head from oracle/fixture_model.py.
* The leaf alone against oracle.van_loan_local_terms, a float64 restatement of ews/core/van_loan.py:31-160
  (augmented exponentials, powers E^m, the inverse of E^M and the knots) followed by the plain signature of the
  knots. The kernel computes the same knots through the step matrices (Delta_M = V w, Delta_{m-1} = P Delta_m)
  and the levels through closed-form sums, so a wrong scheme, a wrong step or a wrong index shows up here.
  Cases: every scheme x reweighting mode, depths 1-3, d = 16 and a padded d, M from 1 to 64, steps with
  delta ||A|| above 1 (the scaled exponential), and the jump case of the uniform modes (first step 0).
* Gauss-Jordan pivoting: with M = 1 and the euler scheme the level-1 term is (I + h A)^{-1} v; A is chosen so
  that I + h A is a permuted, scaled matrix with a zero diagonal, which needs row pivoting.
* Flows of every chen_expm scheme (ews/core/expm_approx.py:13-41) against the oracle's flows, for both leaves.
* The layer end to end with its defaults (van_loan, M = 20, cayley) for every readout and reweighting mode.
"""

import os

import numpy as np
import pytest
import torch

import ews_mi355x as E
from ews_mi355x import ops
from oracle import ews_oracle as O
from oracle import fixture_model as FM

pytestmark = pytest.mark.gpu

DEV = "cuda"
SCHEMES = ("exact", "cayley", "euler", "pade")
MODES = ("displacement", "displacement_uniform", "displacement_uniform_basepoint")


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _golden(name):
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", name)


def _random(B, L, d, seed, hscale=0.05, ascale=1.0, uniform=False, shift=None):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1)
    if uniform:
        clock = np.broadcast_to(np.arange(L) * hscale, (B, L)).copy()
    else:
        clock = np.cumsum(rng.uniform(0.5, 1.5, size=(B, L)) * hscale, 1)
    A = rng.normal(size=(d, d)) * ascale / np.sqrt(d) + np.eye(d) * (0.5 * ascale if shift is None else shift)
    return (torch.tensor(path, dtype=torch.float32), torch.tensor(clock, dtype=torch.float32),
            torch.tensor(A, dtype=torch.float32))


def _check_levels(lv, rlv, d, N, bar=1e-5, tag=""):
    off = 0
    for k in range(1, N + 1):  # every level on its own scale
        n = d**k
        e = relerr(lv[..., off:off + n], rlv[..., off:off + n])
        assert e < bar, (tag, k, e)
        off += n


def _oracle_vl(path, clock, A, N, M, scheme, mode):
    out = []
    for b in range(path.shape[0]):
        p, c = path[b].double(), clock[b].double()
        out.append(O.pack(O.van_loan_local_terms(p[1:] - p[:-1], c[1:] - c[:-1], A.double(), N, M, scheme, mode)))
    return torch.stack(out)


# ------------------------------------------------------------------------------------------------ pinned logits
@pytest.mark.parametrize("name", list(FM.combinations().keys()))
def test_pinned_logits_on_gpu(name):
    ref = np.load(_golden("reference_kernel_outputs.npz"))
    mode, readout, reduce, feature = FM.combinations()[name]
    paths, clocks = FM.fixture_inputs()
    A, Bm, head = FM.fixture_params(feature=feature)
    x = torch.tensor(FM.lift(paths, Bm)).to(DEV)
    c = torch.tensor(clocks).to(DEV)
    kw = dict(M=4, van_loan_expm="exact", chen_expm="exact", reweighting_mode=mode, terminal_reduce=reduce,
              leaf="van_loan")
    At = torch.tensor(A).to(DEV)
    if feature == "signature":
        feats = E.EWS(At, N=2, **kw)(x, c, readout=readout)
    else:
        feats = E.LogEWS(At, N=2, **kw)(x, c, readout=readout)
    got = FM.head_apply(feats.cpu().double().numpy(), head)
    e = relerr(got, ref[name])
    print(f"pinned {name}: {e:.2e}")
    assert got.shape == ref[name].shape
    assert e < 1e-5


# ------------------------------------------------------------------------------------------------ the leaf alone
@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("N,d,M", [(2, 16, 20), (3, 16, 20), (3, 5, 7)])
def test_van_loan_leaf(scheme, mode, N, d, M):
    path, clock, A = _random(2, 29, d, seed=100 + N + d + M, hscale=0.05, uniform=mode != "displacement")
    leaf = ops.DenseLeaf("van_loan", M=M, van_loan_expm=scheme, reweighting_mode=mode)
    lv, _ = ops.dense_local_terms(path.to(DEV), clock.to(DEV), A.to(DEV), N, 0, leaf=leaf)
    rlv = _oracle_vl(path, clock, A, N, M, scheme, mode)
    print(f"vl leaf {scheme} {mode} N={N} d={d} M={M}: {relerr(lv, rlv):.2e}")
    _check_levels(lv, rlv, d, N, tag=f"{scheme} {mode}")


@pytest.mark.parametrize("N,d,M,hscale", [(1, 16, 1, 0.05), (3, 16, 1, 0.05), (2, 9, 4, 0.05), (3, 16, 32, 0.05),
                                          (3, 16, 64, 0.05), (2, 16, 64, 0.05), (3, 12, 3, 2.0), (2, 16, 2, 4.0)])
def test_van_loan_leaf_knots_and_large_steps(N, d, M, hscale):
    """M from 1 to 64 (one k-step to sixteen; the two-wave launch above M = 32) and delta ||A||_1 above 1 (the
    spectrum of A sits in the right half-plane, so that I + delta A stays well conditioned at large steps)."""
    path, clock, A = _random(2, 23, d, seed=200 + N + d + M, hscale=hscale, ascale=0.3, shift=1.0)
    for scheme in SCHEMES:
        leaf = ops.DenseLeaf("van_loan", M=M, van_loan_expm=scheme)
        lv, _ = ops.dense_local_terms(path.to(DEV), clock.to(DEV), A.to(DEV), N, 0, leaf=leaf)
        rlv = _oracle_vl(path, clock, A, N, M, scheme, "displacement")
        print(f"vl leaf {scheme} N={N} d={d} M={M} h={hscale}: {relerr(lv, rlv):.2e}")
        _check_levels(lv, rlv, d, N, tag=scheme)


@pytest.mark.parametrize("mode", ["displacement_uniform", "displacement_uniform_basepoint"])
def test_van_loan_uniform_jump_case(mode):
    """A first step of 0 (uniform) or a second step of 0 (basepoint) selects the linear knots
    (van_loan.py:100-102): the levels are then the plain signature of each increment, v^{(x)k} / k!."""
    B, L, d, N = 2, 12, 6, 3
    path, clock, A = _random(B, L, d, seed=301)
    clock = torch.zeros(B, L)
    leaf = ops.DenseLeaf("van_loan", M=6, van_loan_expm="cayley", reweighting_mode=mode)
    lv, _ = ops.dense_local_terms(path.to(DEV), clock.to(DEV), A.to(DEV), N, 0, leaf=leaf)
    rlv = _oracle_vl(path, clock, A, N, 6, "cayley", mode)
    pd = path.double()
    v = pd[:, 1:] - pd[:, :-1]
    plain = torch.cat([v, torch.einsum("bti,btj->btij", v, v).reshape(B, L - 1, -1) / 2,
                       torch.einsum("bti,btj,btk->btijk", v, v, v).reshape(B, L - 1, -1) / 6], -1)
    _check_levels(rlv, plain, d, N, bar=1e-12, tag="oracle")
    _check_levels(lv, rlv, d, N, tag=mode)


def test_gauss_jordan_pivoting():
    """M = 1, euler: level 1 = (I + h A)^{-1} v. With A = (Pm S - I) / h for a permutation Pm and a diagonal
    S, I + h A = Pm S has a zero diagonal: without row pivoting the elimination divides by zero."""
    d, L = 16, 6
    rng = np.random.default_rng(7)
    perm = rng.permutation(d)
    while np.any(perm == np.arange(d)):
        perm = rng.permutation(d)
    Pm = np.eye(d)[perm]
    S = np.diag(rng.uniform(0.5, 2.0, d))
    h = 0.25
    A = (Pm @ S - np.eye(d)) / h
    path = np.cumsum(rng.normal(size=(1, L, d)), 1)
    clock = np.arange(L, dtype=np.float64)[None] * h
    leaf = ops.DenseLeaf("van_loan", M=1, van_loan_expm="euler")
    t = lambda x: torch.tensor(x, dtype=torch.float32, device=DEV)
    lv, _ = ops.dense_local_terms(t(path), t(clock), t(A), 1, 0, leaf=leaf)
    v = path[0, 1:] - path[0, :-1]
    ref = np.linalg.solve(Pm @ S, v.T).T
    e = relerr(lv[0], ref)
    print(f"pivoting: {e:.2e}")
    assert e < 1e-5


# ------------------------------------------------------------------------------------------------ flow schemes
@pytest.mark.parametrize("scheme", SCHEMES)
@pytest.mark.parametrize("flow_mode,cached,basepoint", [("per_interval", False, False), ("cached", True, False),
                                                        ("cached_basepoint", True, True)])
@pytest.mark.parametrize("leaf_kind", ["series", "van_loan"])
def test_flow_schemes(scheme, flow_mode, cached, basepoint, leaf_kind):
    B, L, d = 2, 19, 16
    path, clock, A = _random(B, L, d, seed=400, hscale=0.3, ascale=2.0)
    leaf = ops.DenseLeaf(leaf_kind, q=12, M=5, chen_expm=scheme)
    _, fl = ops.dense_local_terms(path.to(DEV), clock.to(DEV), A.to(DEV), 2, 12, flow_mode=flow_mode, leaf=leaf)
    ref = torch.stack([O.flows((clock[b, 1:] - clock[b, :-1]).double(), A.double(), scheme, cached, basepoint)
                       for b in range(B)])
    e = relerr(fl, ref)
    print(f"flows {scheme} {flow_mode} {leaf_kind}: {e:.2e}")
    assert e < 1e-5


# ------------------------------------------------------------------------------------------------ the layer
@pytest.mark.parametrize("readout", ["prefix", "terminal", "mean", "max"])
@pytest.mark.parametrize("mode", MODES)
def test_van_loan_layer_defaults(readout, mode):
    """EWS(A, N) with the reference defaults: leaf van_loan, M = 20, van_loan_expm cayley, chen_expm exact,
    terminal_reduce tree (per-interval flows for the terminal)."""
    B, L, d, N = 2, 150, 16, 3
    path, clock, A = _random(B, L, d, seed=500, hscale=0.02, uniform=mode != "displacement")
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=N, reweighting_mode=mode)
    out = layer(path.to(DEV), clock.to(DEV), readout=readout)
    ref = O.ews(path.double(), clock.double(), A.double(), N, readout, leaf="van_loan", M=20,
                van_loan_expm="cayley", chen_expm="exact", reweighting_mode=mode, terminal_reduce="tree")
    e = relerr(out, ref)
    print(f"vl layer {readout} {mode}: {e:.2e}")
    assert out.shape == ref.shape
    assert e < 1e-5


@pytest.mark.parametrize("chen", ["cayley", "pade", "euler"])
def test_layer_chen_schemes(chen):
    B, L, d, N = 2, 80, 8, 2
    path, clock, A = _random(B, L, d, seed=600, hscale=0.05)
    layer = E.EWS(E.AParamConstant(A.to(DEV)), N=N, M=8, chen_expm=chen, terminal_reduce="assoc")
    out = layer(path.to(DEV), clock.to(DEV), readout="prefix")
    ref = O.ews(path.double(), clock.double(), A.double(), N, "prefix", leaf="van_loan", M=8,
                van_loan_expm="cayley", chen_expm=chen)
    assert relerr(out, ref) < 1e-5
    series = E.EWS(E.AParamConstant(A.to(DEV)), N=N, leaf="series", series_q=14, chen_expm=chen)
    out = series(path.to(DEV), clock.to(DEV), readout="terminal")
    ref = O.ews(path.double(), clock.double(), A.double(), N, "terminal", leaf="series", series_q=14,
                chen_expm=chen, terminal_reduce="tree")
    assert relerr(out, ref) < 1e-5
