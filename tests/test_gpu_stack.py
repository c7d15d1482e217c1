"""Stacked-block parity harness (ews/block.py:473-756, the reference's stack around its layer): the whole model of
``ews_mi355x.block`` (encoder, EWS blocks with their fronts, scans, fused mixer epilogues, norms and channel
stages, head) on the GPU against its float64 restatement (oracle/block_oracle.py, built from the pinned oracle
pieces), forward and the gradient of every parameter and of the input series.

Cases: the shape of BASELINE.json configs[3] (4 token blocks, width 32, real diagonal generators, RMSNorm and GLU
between blocks) and configs[4] (3 series blocks, 12 rotation planes) at reduced B and L, and a mixed stack that
goes through the other block options (dense generator on the Van Loan leaf, output gate, increment paths, basepoint,
binomial prescale, blended clock, slice_post placement, masks, mean-pool head, final norm).

Bars: logits <= 1e-5 and every gradient <= 1e-4, metric max|a-b| / max|b| per tensor (the layer's bars of
BASELINE.json; the stack's float32 norms and linear maps add rounding of the same order as the scan's).
"""

import copy

import numpy as np
import pytest
import torch

import ews_mi355x as E
from oracle import block_oracle as BO

pytestmark = pytest.mark.gpu

DEV = "cuda"
DT = torch.float64


def relerr(a, b):
    a = a.detach().cpu().double()
    b = b.detach().cpu().double()
    return float((a - b).abs().max() / max(float(b.abs().max()), 1e-300))


def _oracle_leaves(model):
    """float64 leaves of every parameter, keyed by name; the generators as float64 copies of their modules
    whose parameters are those leaves."""
    P = {n: p.detach().cpu().double().clone().requires_grad_(True) for n, p in model.named_parameters()}
    fns = []
    for i, blk in enumerate(model.blocks):
        a64 = copy.deepcopy(blk.ewms.A_param).cpu().double()
        for pn, p in a64.named_parameters():
            P[f"blocks.{i}.ewms.A_param.{pn}"] = p
        fns.append(lambda _P, m=a64: m())
    return P, fns


def _compare(model, X, bcfgs, scfg, t=None, mask=None, x_grad=False, seed=0, a_scales=None):
    model = model.to(DEV)
    P, fns = _oracle_leaves(model)
    Xd = X.to(DEV)
    if x_grad:
        Xd = Xd.clone().requires_grad_(True)
    md = None if mask is None else mask.to(DEV)
    out = model(Xd, t=None if t is None else t.to(DEV), mask=md, inference=True)
    Xr = X.double().clone().requires_grad_(True) if x_grad else X
    ref = BO.stack(Xr, P, scfg, bcfgs, fns, t=None if t is None else t.double(), mask=mask, a_scales=a_scales)
    e = relerr(out, ref)
    # with no graph recorded, blocks whose scan allows it run the epilogue inside the scan's output pass
    with torch.no_grad():
        out_ng = model(Xd.detach(), t=None if t is None else t.to(DEV), mask=md, inference=True)
    e_ng = relerr(out_ng, ref)
    print(f"  no-grad route: logits {e_ng:.2e}", flush=True)
    assert e_ng < 1e-5, e_ng
    w = torch.tensor(np.random.default_rng(seed).normal(size=tuple(ref.shape)))
    (out * w.to(DEV, torch.float32)).sum().backward()
    (ref * w).sum().backward()
    errs = {}
    for n, p in model.named_parameters():
        g, gr = p.grad, P[n].grad
        if gr is None or float(gr.abs().max()) == 0.0:
            continue
        errs[n] = relerr(g, gr)
    if x_grad:
        errs["input"] = relerr(Xd.grad, Xr.grad)
    worst = max(errs, key=errs.get)
    print(f"  logits {e:.2e}; worst gradient {worst} {errs[worst]:.2e} ({len(errs)} tensors)", flush=True)
    assert e < 1e-5, e
    assert errs[worst] < 1e-4, (worst, errs[worst])


def test_token_stack_c4_shape():
    """4 token blocks, width 32, real diagonal A = diag(U(0.1, 2)) per block on the series leaf, RMSNorm + GLU."""
    rng = np.random.default_rng(4)
    nb, H, V, B, L = 4, 32, 8, 2, 128
    per = []
    for i in range(nb):
        lam = rng.uniform(0.1, 2.0, size=H)
        per.append(dict(a_param=E.AParamEFM(torch.tensor(np.log(np.expm1(lam)), dtype=torch.float32))))
    kw = dict(m=H, n=2, leaf="series", series_q=12, channel_stage="glu", dropout_rate=0.0)
    model = E.StackedEWS(nb, V, H, V, tokens=True, block_kwargs=kw, per_block_kwargs=per, key=11)
    with torch.no_grad():
        model.embedding.weight.copy_(torch.tensor(rng.normal(0.0, 1.0 / np.sqrt(H), size=(V, H))))
    X = torch.tensor(rng.integers(0, V, size=(B, L)))
    bc = dict(n=2, channel_stage="glu", layer=dict(leaf="series", series_q=12))
    print(f"stack c4 shape: {nb} blocks, H={H}, B={B}, L={L}", flush=True)
    _compare(model, X, [bc] * nb, dict(tokens=True), seed=1)


def test_series_stack_c5_shape():
    """3 series blocks, width 24 (12 damped rotation planes per block, exact plane leaf), MLP channel stage, on
    band-limited signals: sums of 4 sinusoids U(0.5, 3) Hz at 32 Hz plus N(0, 0.05) noise."""
    rng = np.random.default_rng(5)
    nb, H, c, B, L = 3, 24, 6, 1, 1500
    per = []
    for i in range(nb):
        v = torch.tensor(rng.normal(size=H // 2), dtype=torch.float32)
        u = torch.tensor(rng.normal(size=H // 2), dtype=torch.float32)
        per.append(dict(a_param=E.AParamDampedRotation(v, u, H, omega_scale=3.0)))
    kw = dict(m=H, n=2, leaf="plane_closed", channel_stage="mlp", dropout_rate=0.0)
    model = E.StackedEWS(nb, c, H, 1, tokens=False, block_kwargs=kw, per_block_kwargs=per, key=12)
    tt = np.arange(L) / 32.0
    sig = np.zeros((B, L, c))
    for b in range(B):
        for ch in range(c):
            f = rng.uniform(0.5, 3.0, size=4)
            ph = rng.uniform(0, 2 * np.pi, size=4)
            sig[b, :, ch] = np.sin(2 * np.pi * f[:, None] * tt[None] + ph[:, None]).sum(0)
    sig += rng.normal(0.0, 0.05, size=sig.shape)
    X = torch.tensor(sig, dtype=torch.float32)
    bc = dict(n=2, layer=dict(leaf="plane_closed"))
    print(f"stack c5 shape: {nb} blocks, H={H}, B={B}, L={L}", flush=True)
    _compare(model, X, [bc] * nb, dict(tokens=False), x_grad=True, seed=2)


def test_mixed_block_options():
    """Two blocks over the remaining options: block 0 a dense definite_plus_skew generator on the Van Loan leaf
    (M = 4, exact sub-step exponentials), output gate, increment paths, basepoint, binomial prescale, a blended
    variation clock; block 1 slice_post placement, tanh channel stage, static_gain graded norm; masked rows, a
    mean-pool head and a final norm."""
    rng = np.random.default_rng(6)
    H, c, B, L = 12, 5, 3, 40
    clk = dict(mode="blended_variation", alpha=0.4)
    per = [
        dict(m=6, n=2, leaf="van_loan", M=4, van_loan_expm="exact", output_gate=True, path_mode="increment",
             basepoint=True, graded_prescale="binomial", clock=clk, channel_stage="gelu_glu"),
        dict(m=6, n=2, leaf="series", series_q=16, norm_placement="slice_post", channel_stage="tanh",
             graded_norm="static_gain"),
    ]
    model = E.StackedEWS(2, c, H, 4, tokens=False, head_mode="mean_pool", final_norm=True,
                         block_kwargs=dict(dropout_rate=0.0), per_block_kwargs=per, key=13)
    X = torch.tensor(rng.normal(size=(B, L, c)) * 0.5, dtype=torch.float32)
    lengths = [L, L - 7, L - 15]
    mask = torch.tensor([[i < n for i in range(L)] for n in lengths])
    bcs = [
        dict(n=2, layer=dict(leaf="van_loan", M=4, van_loan_expm="exact"), output_gate=True,
             path_mode="increment", basepoint=True, graded_prescale="binomial", clock=clk, channel_stage="gelu_glu"),
        dict(n=2, layer=dict(leaf="series", series_q=16), norm_placement="slice_post", channel_stage="tanh",
             graded_norm="static_gain"),
    ]
    print(f"mixed stack: H={H}, B={B}, L={L}, lengths {lengths}", flush=True)
    _compare(model, X, bcs, dict(tokens=False, head_mode="mean_pool", final_norm=True), mask=mask, x_grad=True,
             seed=3)


def test_token_stack_bounded_rotation_scale():
    """Token blocks on rotation planes: the stack scales each block's generator by 2 pi / dtheta_max, the largest
    per-token clock increment over the embedding table (ews/block.py:626-677), here a token-gated clock on block 0
    (its gate reads the embeddings) and a time clock on block 1 (the row norms); the scale is the checker's own."""
    rng = np.random.default_rng(7)
    nb, H, V, B, L = 2, 16, 6, 2, 60
    gate = dict(mode="token_gated", normalize="constant", norm_constant=2.0, scaling="none")
    per = [dict(a_param=E.AParamBoundedRotation(torch.tensor(rng.normal(size=H // 2), dtype=torch.float32), H,
                                                omega_scale=2.0), clock=gate, path_mode="increment"),
           dict(a_param=E.AParamDampedRotation(torch.tensor(rng.normal(size=H // 2), dtype=torch.float32),
                                               torch.tensor(rng.normal(size=H // 2), dtype=torch.float32), H))]
    kw = dict(m=H, n=2, leaf="plane_closed", channel_stage="glu", dropout_rate=0.0)
    model = E.StackedEWS(nb, V, H, V, tokens=True, block_kwargs=kw, per_block_kwargs=per, key=14)
    with torch.no_grad():
        model.blocks[0].clock.b.fill_(-0.3)  # most tokens open the gate
    X = torch.tensor(rng.integers(0, V, size=(B, L)))
    emb = model.embedding.weight.detach().double()
    c0 = model.blocks[0].clock
    scales = [BO.bounded_a_scale(emb, gate, True, c0.w.detach().double(), c0.b.detach().double()),
              BO.bounded_a_scale(emb, {}, False)]
    got = [float(model.bounded_a_scale(i)) for i in range(nb)]
    assert np.allclose(got, scales, rtol=1e-6), (got, scales)
    bcs = [dict(n=2, channel_stage="glu", layer=dict(leaf="plane_closed"), clock=gate, path_mode="increment"),
           dict(n=2, channel_stage="glu", layer=dict(leaf="plane_closed"))]
    print(f"token rotation stack: a_scale {scales}", flush=True)
    _compare(model, X, bcs, dict(tokens=True), seed=4, a_scales=scales)
