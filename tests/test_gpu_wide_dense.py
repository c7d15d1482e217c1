"""GPU parity of dense generators wider than 16 channels (16 < d <= 32, depths 1-2; csrc/ews_wide.hip) against the
float64 oracle and torch float64 autograd through it.

Bars (the reference's metric max|a-b| / max|b| of tests/test_engines.py:31-33, each level
and each gradient on its own scale): forward 1e-5, gradients 1e-4.

Cases: the series leaf and the Van Loan leaf (every scheme of van_loan_expm, every reweighting mode, M from 1 to 8),
flows of every chen_expm scheme per interval and shared, readouts prefix / terminal / mean / max, d = 17, 20, 24 and
32, chunks of 8 intervals (several chunks: the carries and the adjoint's chunk scan) and the default chunk, steps
with |h| ||A|| above 1 (the scaled exponential and its doublings), and the banked SCP1 block
(/root/reference/uea_results/scp1/config.json:28-59: d = 17 skew-symmetric A, depth 2, M = 4, van_loan_expm euler,
chen_expm cayley, displacement_uniform, mean readout) through the layer.
"""

import numpy as np
import pytest
import torch

import ews_mi355x as E
from ews_mi355x import ops
from oracle import ews_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
_FLOW = {"displacement": "per_interval", "displacement_uniform": "cached",
         "displacement_uniform_basepoint": "cached_basepoint"}


def relerr(a, b):
    a = np.asarray(a.detach().cpu().double() if torch.is_tensor(a) else a, np.float64)
    b = np.asarray(b.detach().cpu().double() if torch.is_tensor(b) else b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


def _inputs(B, L, d, seed, hscale=0.05, ascale=1.0, skew=False):
    rng = np.random.default_rng(seed)
    path = np.cumsum(rng.normal(size=(B, L, d)) * 0.3, 1)
    clock = np.cumsum(rng.uniform(0.5, 1.5, size=(B, L)) * hscale, 1)
    G = rng.normal(size=(d, d)) * ascale / np.sqrt(d)
    A = (G - G.T) / 2 if skew else G + 0.5 * ascale * np.eye(d)
    return torch.tensor(path), torch.tensor(clock), torch.tensor(A)


def _leaf(kw, mode):
    return ops.DenseLeaf(kw.get("leaf", "van_loan"), q=kw.get("series_q", 0), M=kw.get("M", 4),
                         van_loan_expm=kw.get("van_loan_expm", "cayley"), reweighting_mode=mode,
                         chen_expm=kw.get("chen_expm", "exact"))


def _check_levels(got, ref, d, N, bar, tag):
    lead = got.shape[-1] - sum(d**k for k in range(1, N + 1))  # the level-0 column
    off = lead
    for k in range(1, N + 1):
        n = d**k
        e = relerr(got[..., off:off + n], ref[..., off:off + n])
        print(f"{tag} level {k}: {e:.2e}")
        assert e < bar, (tag, k, e)
        off += n


def _run(path, clock, A, N, readout, mode, kw, chunk=0, grads=True, seed=7):
    """(GPU output, oracle output[, GPU grads, oracle grads]) for (path, clock, A)."""
    p64, c64, A64 = (x.clone().requires_grad_(grads) for x in (path, clock, A))
    okw = dict(kw)
    okw.setdefault("leaf", "van_loan")
    okw.setdefault("M", 4)
    ref = O.ews(p64, c64, A64, N, readout, reweighting_mode=mode, terminal_reduce="assoc", **okw)
    pg, cg, Ag = (x.float().to(DEV).requires_grad_(grads) for x in (path, clock, A))
    leaf = _leaf(kw, mode)
    out = ops.dense_scan(pg, cg, Ag, N, leaf.q, _FLOW[mode], readout, True, chunk=chunk, leaf=leaf)
    if not grads:
        return out, ref
    gout = torch.tensor(np.random.default_rng(seed).normal(size=ref.shape))
    rg = torch.autograd.grad(ref, (p64, c64, A64), gout)
    gg = torch.autograd.grad(out, (pg, cg, Ag), gout.float().to(DEV))
    return out, ref, gg, rg


def _check_grads(gg, rg, tag, bar=1e-4):
    for name, g, r in zip(("path", "clock", "A"), gg, rg):
        e = relerr(g, r)
        print(f"{tag} grad {name}: {e:.2e}")
        assert e < bar, (tag, name, e)


FWD_CASES = [
    # d, N, L, readout, mode, leaf kw, chunk
    (17, 2, 40, "prefix", "displacement_uniform", dict(van_loan_expm="euler", chen_expm="cayley"), 8),
    (24, 2, 37, "prefix", "displacement", dict(van_loan_expm="cayley"), 8),
    (32, 2, 30, "terminal", "displacement", dict(leaf="series", series_q=6), 8),
    (20, 1, 45, "prefix", "displacement_uniform_basepoint", dict(van_loan_expm="exact", chen_expm="pade"), 8),
    (24, 2, 33, "max", "displacement", dict(van_loan_expm="pade", chen_expm="euler", M=3), 0),
    (32, 2, 70, "prefix", "displacement_uniform", dict(van_loan_expm="exact", M=8), 0),
    (17, 1, 50, "mean", "displacement_uniform", dict(leaf="series", series_q=4, chen_expm="cayley"), 8),
    (18, 2, 26, "prefix", "displacement_uniform_basepoint", dict(van_loan_expm="euler", chen_expm="exact", M=1), 8),
]


@pytest.mark.parametrize("case", FWD_CASES,
                         ids=[f"d{c[0]}-N{c[1]}-{c[3]}-{c[4]}-{i}" for i, c in enumerate(FWD_CASES)])
def test_wide_forward_and_gradients(case):
    d, N, L, readout, mode, kw, chunk = case
    path, clock, A = _inputs(2, L, d, seed=d * 10 + N)
    out, ref, gg, rg = _run(path, clock, A, N, readout, mode, kw, chunk=chunk)
    tag = f"d={d} N={N} {readout} {mode} {kw}"
    _check_levels(out, ref, d, N, 1e-5, tag)
    _check_grads(gg, rg, tag)


@pytest.mark.parametrize("scheme", ["exact", "cayley", "euler", "pade"])
def test_wide_large_steps(scheme):
    """Steps with |h| ||A||_1 well above 1: the exact scheme's scaled exponential takes doublings (forward) and its
    Frechet adjoint a scaled 64 x 64 block; the rational schemes pivot. Per-interval flows and leaf. A is a large
    rotation part plus a unit shift, so the flows rotate and contract and the outputs stay of order one: with
    expanding flows the outputs grow like e^{h L}, and the checker's own float64 gradient (torch's matrix_exp
    backward, which does not rescale the cotangent) loses its accuracy there before this kernel's does."""
    rng = np.random.default_rng(91)
    d, L = 24, 40
    path = torch.tensor(np.cumsum(rng.normal(size=(2, L, d)) * 0.3, 1))
    clock = torch.tensor(np.cumsum(rng.uniform(0.5, 1.5, size=(2, L)) * 0.6, 1))
    G = rng.normal(size=(d, d))
    A = torch.tensor((G - G.T) * (2.0 / np.sqrt(d)) + np.eye(d))
    out, ref, gg, rg = _run(path, clock, A, 2, "terminal", "displacement",
                            dict(van_loan_expm=scheme, chen_expm=scheme, M=2), chunk=16)
    tag = f"large steps {scheme}"
    _check_levels(out, ref, d, 2, 1e-5, tag)
    _check_grads(gg, rg, tag)


def test_wide_scp1_block_through_the_layer():
    """The banked SCP1 block (d = 17 skew-symmetric A, depth 2, M = 4, euler Van Loan steps, cayley flows, uniform
    reweighting, mean readout) through EWS, forward and gradients, at a few hundred steps."""
    path, clock, A = _inputs(3, 300, 17, seed=5, hscale=0.02, skew=True)
    layer = E.EWS(E.AParamGeneral(A.float()), N=2, leaf="van_loan", M=4, van_loan_expm="euler", chen_expm="cayley",
                  reweighting_mode="displacement_uniform").to(DEV)
    pg = path.float().to(DEV).requires_grad_(True)
    cg = clock.float().to(DEV).requires_grad_(True)
    out = layer(pg, cg, readout="mean")
    p64, c64, A64 = (x.clone().requires_grad_(True) for x in (path, clock, A))
    ref = O.ews(p64, c64, A64, 2, "mean", leaf="van_loan", M=4, van_loan_expm="euler", chen_expm="cayley",
                reweighting_mode="displacement_uniform")
    _check_levels(out, ref, 17, 2, 1e-5, "scp1")
    gout = torch.tensor(np.random.default_rng(2).normal(size=ref.shape))
    rg = torch.autograd.grad(ref, (p64, c64, A64), gout)
    out.backward(gout.float().to(DEV))
    gA = [p.grad for p in layer.parameters()][0]
    _check_grads((pg.grad, cg.grad, gA), rg, "scp1")


def test_wide_backward_is_deterministic():
    """Two backward calls give bit-identical gradients (every sum is in a fixed order)."""
    path, clock, A = _inputs(2, 60, 24, seed=13)
    leaf = _leaf(dict(van_loan_expm="exact"), "displacement")
    grads = []
    for _ in range(2):
        p = path.float().to(DEV).requires_grad_(True)
        c = clock.float().to(DEV).requires_grad_(True)
        a = A.float().to(DEV).requires_grad_(True)
        out = ops.dense_scan(p, c, a, 2, 0, "per_interval", "prefix", True, chunk=8, leaf=leaf)
        out.backward(torch.ones_like(out))
        grads.append((p.grad.clone(), c.grad.clone(), a.grad.clone()))
    for name, x, y in zip(("path", "clock", "A"), grads[0], grads[1]):
        assert torch.equal(x, y), f"{name} gradient differs between two identical calls"


KEPT_CASES = [
    # d, readout, mode, leaf kw
    (24, "max", "displacement", dict(van_loan_expm="cayley", M=6)),
    (17, "terminal", "displacement_uniform", dict(van_loan_expm="euler", chen_expm="cayley")),
    (20, "mean", "displacement_uniform_basepoint", dict(leaf="series", series_q=5, chen_expm="pade")),
]


@pytest.mark.parametrize("case", KEPT_CASES, ids=[f"d{c[0]}-{c[1]}-{c[2]}" for c in KEPT_CASES])
def test_wide_kept_backward_equals_recomputing(case):
    """ews_dense_backward_kept starts from what ews_dense_forward_keep left in the workspace (step matrices, local
    terms, chunk summaries and carries, prefix states, the maxima's rows); ews_dense_backward recomputes them. The
    same kernels on the same data: the gradients agree bit for bit, and the kept forward's output with the plain
    forward's and with the forward alone (no gradient: its own workspace, the mean / max from the chunks'
    partials without the prefix states)."""
    d, readout, mode, kw = case
    path, clock, A = _inputs(2, 50, d, seed=d + 3)
    leaf = _leaf(kw, mode)
    gout = None
    res = []
    for keep in (True, False):
        p = path.float().to(DEV).requires_grad_(True)
        c = clock.float().to(DEV).requires_grad_(True)
        a = A.float().to(DEV).requires_grad_(True)
        out = ops.dense_scan(p, c, a, 2, leaf.q, _FLOW[mode], readout, True, chunk=8, leaf=leaf, keep=keep)
        if gout is None:
            gout = torch.randn(out.shape, generator=torch.Generator().manual_seed(5)).to(DEV)
        out.backward(gout)
        res.append((out.detach().clone(), p.grad.clone(), c.grad.clone(), a.grad.clone()))
    for name, x, y in zip(("out", "path", "clock", "A"), res[0], res[1]):
        assert torch.equal(x, y), f"{name}: kept and recomputing backward differ"
    with torch.no_grad():  # the forward alone (its own workspace layout, no prefix states kept)
        out0 = ops.dense_scan(path.float().to(DEV), clock.float().to(DEV), A.float().to(DEV), 2, leaf.q,
                              _FLOW[mode], readout, True, chunk=8, leaf=leaf, keep=False)
    assert torch.equal(out0, res[0][0]), "forward alone and kept forward differ"


@pytest.mark.parametrize("readout", ["prefix", "mean"])
def test_wide_logews(readout):
    """LogEWS over a dense d = 20 generator at depth 2: the wide kernels' rows, then the log and Lyndon compression
    (csrc/ews_log.hip), against the oracle's log_ews_single (ews/layer.py:488-517), forward and gradients."""
    path, clock, A = _inputs(2, 30, 20, seed=44)
    layer = E.LogEWS(E.AParamGeneral(A.float()), N=2, M=4, van_loan_expm="pade", chen_expm="cayley",
                     reweighting_mode="displacement").to(DEV)
    pg = path.float().to(DEV).requires_grad_(True)
    out = layer(pg, clock.float().to(DEV), readout=readout)
    p64 = path.clone().requires_grad_(True)
    ref = torch.stack([O.log_ews_single(p64[b], clock[b], A, 2, readout, leaf="van_loan", M=4,
                                        van_loan_expm="pade", chen_expm="cayley", reweighting_mode="displacement")
                       for b in range(2)])
    e = relerr(out, ref)
    print(f"logews {readout}: forward {e:.2e}")
    assert e < 1e-5
    gout = torch.tensor(np.random.default_rng(3).normal(size=ref.shape))
    (rg,) = torch.autograd.grad(ref, (p64,), gout)
    out.backward(gout.float().to(DEV))
    eg = relerr(pg.grad, rg)
    print(f"logews {readout}: path grad {eg:.2e}")
    assert eg < 1e-4


@pytest.mark.parametrize("scheme", ["exact", "cayley", "pade"])
def test_wide_series_and_fallback_in_one_call(scheme):
    """Per-interval steps on both sides of the series radius in one call (|h| ||A||_1 from about 0.3 to 2.5): the
    matrices inside it come from the powers table, the others from the scaled / inverted forms (k_wmat mode 2), and
    the adjoint splits the same way."""
    rng = np.random.default_rng(17)
    d, L = 20, 50
    path = torch.tensor(np.cumsum(rng.normal(size=(2, L, d)) * 0.3, 1))
    clock = torch.tensor(np.cumsum(rng.uniform(0.05, 0.45, size=(2, L)), 1))
    G = rng.normal(size=(d, d))
    A = torch.tensor((G - G.T) * (0.5 / np.sqrt(d)) + np.eye(d))
    out, ref, gg, rg = _run(path, clock, A, 2, "prefix", "displacement",
                            dict(van_loan_expm=scheme, chen_expm=scheme, M=1), chunk=16)
    tag = f"mixed radius {scheme}"
    _check_levels(out, ref, d, 2, 1e-5, tag)
    _check_grads(gg, rg, tag)


@pytest.mark.parametrize("scheme", ["exact", "cayley", "euler", "pade"])
def test_wide_van_loan_knots_three_ways(scheme):
    """Per-interval Van Loan leaf at M = 20 with |h| ||A||_1 from 0.05 to about 14, so that one call holds the
    three forms of the knots: their own power series (M |c| ||A||_1 inside the scheme's radius, c = h / M), the
    M-step chain over (P, V) from the powers table (|c| ||A||_1 inside it), and the chain over (P, V) from the
    scaled / inverted forms (outside it); the adjoint takes the same three routes."""
    rng = np.random.default_rng(23)
    d, L, M = 20, 48, 20
    G = rng.normal(size=(d, d))
    A = (G - G.T) * (0.5 / np.sqrt(d)) + np.eye(d)
    nrm = np.abs(A).sum(0).max()
    steps = np.exp(rng.uniform(np.log(0.05), np.log(14.0), size=(2, L))) / nrm
    steps[:, 0] = 0.0
    path = torch.tensor(np.cumsum(rng.normal(size=(2, L, d)) * 0.3, 1))
    clock = torch.tensor(np.cumsum(steps, 1))
    out, ref, gg, rg = _run(path, clock, torch.tensor(A), 2, "prefix", "displacement",
                            dict(van_loan_expm=scheme, chen_expm=scheme, M=M), chunk=16)
    tag = f"knots three ways {scheme}"
    _check_levels(out, ref, d, 2, 1e-5, tag)
    _check_grads(gg, rg, tag)


@pytest.mark.parametrize("scheme", ["exact", "cayley", "euler", "pade"])
@pytest.mark.parametrize("mode", ["displacement_uniform", "displacement_uniform_basepoint"])
def test_wide_shared_steps_both_sides_of_the_radius(scheme, mode):
    """Uniform reweighting modes: each sample's shared flow and Van Loan pair come from the powers table when
    |dt| ||A||_1 is inside the series radius (sample 0) and from the scaled / inverted forms otherwise (sample 1,
    flagged per sample), in one call; the adjoint splits the same way."""
    rng = np.random.default_rng(29)
    d, L = 20, 40
    path = torch.tensor(np.cumsum(rng.normal(size=(2, L, d)) * 0.3, 1))
    G = rng.normal(size=(d, d))
    A = (G - G.T) * (0.5 / np.sqrt(d)) + np.eye(d)
    nrm = np.abs(A).sum(0).max()
    steps = np.array([0.05, 2.5]) / nrm  # |dt| ||A||_1: 0.05 and 2.5
    clock = torch.tensor(np.arange(L)[None, :] * steps[:, None])
    out, ref, gg, rg = _run(path, clock, torch.tensor(A), 2, "prefix", mode,
                            dict(van_loan_expm=scheme, chen_expm=scheme, M=3), chunk=8)
    tag = f"shared steps {scheme} {mode}"
    _check_levels(out, ref, d, 2, 1e-5, tag)
    _check_grads(gg, rg, tag)
