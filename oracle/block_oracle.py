"""CPU float64 restatement of an EWS block and of the stacked model (ews/block.py:36-756), the checker of the
stacked-block parity harness.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports, links or runs this file; ``tests/`` use it to check
``ews_mi355x.block`` end to end. It composes the other oracle restatements (front_oracle: clocks and lift;
ews_oracle: the layer; mixer_oracle: the epilogue) with the block's norms, gate and channel stage, in torch float64
so that gradients come from autograd of the same restatement.

Parameters come in as a dict of float64 leaf tensors keyed by the parameter names of the module under test
(``blocks.0.norm1.weight`` ...), so that one ``backward`` gives every parameter's gradient; the generator of each
block comes in as a callable returning A (float64) from those leaves.
"""

from __future__ import annotations

import math

import torch

from . import ews_oracle as O
from . import front_oracle as FO
from . import mixer_oracle as MO

DT = torch.float64


def rms_norm(x, weight, eps):
    """ews/norms.py:25-27: x * rsqrt(mean(x^2) + eps) * weight."""
    return x * torch.rsqrt(torch.mean(x * x, -1, keepdim=True) + eps) * weight


def layer_norm(x, weight, bias, eps):
    """equinox LayerNorm over the last axis (mean and biased variance), with weight and bias."""
    mu = x.mean(-1, keepdim=True)
    var = ((x - mu) ** 2).mean(-1, keepdim=True)
    return (x - mu) / torch.sqrt(var + eps) * weight + bias


def linear(x, P, name):
    """eqx.nn.Linear applied row-wise: x W^T + b."""
    return x @ P[name + ".weight"].t() + P[name + ".bias"]


def gelu(x):
    """jax.nn.gelu (approximate=True, its default): 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x**3)))


def channel(stage, xhat, P, pre):
    """ews/block.py:361-374."""
    if stage == "mlp":
        return linear(gelu(linear(xhat, P, pre + "ff1")), P, pre + "ff2")
    if stage == "tanh":
        return torch.tanh(linear(xhat, P, pre + "ff1"))
    if stage == "glu":
        h = linear(xhat, P, pre + "ff1")
        a, b = h.chunk(2, -1)
        return a * torch.sigmoid(b)
    h = gelu(xhat)
    return linear(h, P, pre + "ff1") * torch.sigmoid(linear(h, P, pre + "ff2"))


def clock(t, driver, spec, P, pre, mask):
    """The block's clock (ews/block.py:386-389): build_clock_jnp for the parameter-free modes, GatedClock for the
    gated ones (front_oracle)."""
    mode = spec.get("mode", "time")
    if mode in ("token_gated", "clamped_gate"):
        return FO.gated_clock(driver, mode, P[pre + "clock.w"], P[pre + "clock.b"], spec.get("norm_constant"),
                              spec.get("gate_in_scale", 1.0), mask, spec.get("stop_gradient", False))
    return FO.build_clock(t, driver, mode, spec.get("alpha", 1.0), spec.get("scaling", "[0,1]"), mask,
                          spec.get("normalize", "per_sample"), spec.get("norm_constant"),
                          spec.get("time_denominator"), spec.get("variation_eps", 1e-8),
                          spec.get("stop_gradient", False))


def block(x, P, pre, cfg, A_fn, t, mask=None, clock_driver=None, a_scale=1.0):
    """EWSBlock._call_single at inference (no dropout) for a batch (ews/block.py:376-424, 282-306): x (B, L, H).

    cfg: n (depth), norm_placement, second_norm, channel_stage, output_gate, basepoint, path_mode,
    graded_norm, graded_eps, graded_prescale, norm_eps, clock (a dict of ClockSpec fields), preserve (the lift
    keeps its first channel), lift (False: no lift), layer (keyword arguments of ews_oracle.ews: leaf, series_q,
    reweighting_mode, chen_expm, ...)."""
    placement = cfg.get("norm_placement", "pre")
    eps = cfg.get("norm_eps", 1e-6)
    spec = cfg.get("clock", {})
    incr = cfg.get("path_mode", "value") == "increment"
    source = spec.get("source", "block_input")
    driver = x if source == "block_input" else clock_driver
    if incr and driver is not None:
        driver = FO.increment_path(driver, mask)
    theta = clock(t, driver, spec, P, pre, mask)
    branch = rms_norm(x, P[pre + "norm1.weight"], eps) if placement == "pre" else x
    if incr:
        branch_in = FO.increment_path(branch, mask)
    else:
        branch_in = branch
    matrix = P.get(pre + "b_layer.matrix") if cfg.get("lift", True) else None
    # front_oracle.block_front applies the increment representation itself
    p, th = FO.block_front(branch, theta, None, mask, matrix, cfg.get("preserve", False), incr,
                           cfg.get("basepoint", False))
    A = A_fn(P) * a_scale
    n = cfg["n"]
    rows = O.ews(p, th, A, n, "prefix", **cfg.get("layer", {}))
    d = p.shape[-1]
    variant = cfg.get("graded_norm", "live_rms")
    geps = cfg.get("graded_eps", 1e-3)
    geps = [float(geps)] * n if isinstance(geps, (int, float)) else [float(e) for e in geps]
    gains = P.get(pre + "mixer.graded.gains")
    lam = P.get(pre + "mixer.graded.lam")
    r = MO.mixer_epilogue(rows, P[pre + "mixer.c_down.weight"], P[pre + "mixer.c_down.bias"], d, n, variant, geps,
                          gains, lam, cfg.get("basepoint", False), cfg.get("graded_prescale") == "binomial")
    if cfg.get("output_gate", False):
        r = r * torch.sigmoid(linear(branch_in, P, pre + "gate"))
    stage = cfg.get("channel_stage", "mlp")
    if placement == "slice_post":
        y = x + r
        y = y + channel(stage, y, P, pre)
        return layer_norm(y, P[pre + "norm2.weight"], P[pre + "norm2.bias"], eps)
    x = x + r
    if placement == "pre" and cfg.get("second_norm", True):
        xhat = rms_norm(x, P[pre + "norm2.weight"], eps)
    else:
        xhat = x
    return x + channel(stage, xhat, P, pre)


def bounded_a_scale(emb, spec, first, w=None, b=None, input_token_ids=None, pad_id=0):
    """StackedEWS._bounded_a_scale for a rotation-plane block of a token model (ews/block.py:626-687):
    2 pi / dtheta_max, dtheta_max = max over the non-pad (and listed) token ids of the token's clock increment
    (the gate on the embedding row when the block's gate reads the embeddings, else the row's norm), over the
    clock's norm_constant, at least 1e-6 / norm_constant."""
    c = spec.get("norm_constant") or 1.0
    mode, source = spec.get("mode", "time"), spec.get("source", "block_input")
    reads = source == "encoder_output" or (source == "block_input" and first)
    if reads and mode == "token_gated":
        dth = torch.relu(emb @ w - b)
    elif reads and mode == "clamped_gate":
        dth = torch.clamp(emb @ w.t() - b, 0.0, 1.0).sum(-1)
    else:
        dth = torch.sqrt((emb * emb).sum(-1))
    keep = [i for i in range(emb.shape[0]) if i != pad_id and (input_token_ids is None or i in input_token_ids)]
    dmax = max(float(dth[keep].max()), 1e-6) / c
    return 2.0 * math.pi / dmax


def stack(X, P, cfg, block_cfgs, A_fns, t=None, mask=None, raw_driver=None, a_scales=None):
    """StackedEWS.__call__ at inference for a batch (ews/block.py:581-624, 695-756): encoder, blocks, optional
    final norm, head(s). cfg: tokens, head_mode, final_norm, heads (number of heads, 0 for a single head)."""
    if cfg.get("tokens", True):
        h = P["embedding.weight"][X.long()]
    else:
        h = linear(X, P, "embedding")
    L = h.shape[1]
    if t is None:
        t = torch.arange(L, dtype=DT)
    enc = h
    for i, (bc, A_fn) in enumerate(zip(block_cfgs, A_fns)):
        src = bc.get("clock", {}).get("source", "block_input")
        drv = enc if src == "encoder_output" else (raw_driver if src == "raw_input" else None)
        h = block(h, P, f"blocks.{i}.", bc, A_fn, t, mask, drv, 1.0 if a_scales is None else a_scales[i])
    if cfg.get("final_norm", False):
        h = rms_norm(h, P["final_norm.weight"], 1e-6)

    def head(name):
        if cfg.get("head_mode", "seq2seq") == "seq2seq":
            return linear(h, P, name)
        if mask is not None:
            w = mask.to(DT)[..., None]
            pooled = (h * w).sum(-2) / torch.clamp(w.sum(-2), min=1.0)
        else:
            pooled = h.mean(-2)
        return linear(pooled, P, name)

    nh = cfg.get("heads", 0)
    if nh:
        return tuple(head(f"head.{k}") for k in range(nh))
    return head("head")
