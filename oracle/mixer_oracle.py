"""CPU float64 restatement of the mixer epilogue of an EWS block: levels -> binomial prescale -> GradedRMSNorm ->
c_down.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports, links or runs this file; ``tests/`` use it as the
checker of the fused HIP epilogue. Written with torch float64 tensors so that gradients come from autograd of the
same restatement. Every function cites the reference file:line it restates.
"""

from __future__ import annotations

import math

import torch

DT = torch.float64


def level_slices(d, N):
    """ews/norms.py:30-45: (start, end) of each level in the level-0-free layout [lvl1 | ... | lvlN]."""
    out, s = [], 0
    for k in range(1, N + 1):
        out.append((s, s + d**k))
        s += d**k
    return out


def levels_from_flat(flat, basepoint):
    """ews/block.py:302-305: drop the level-0 column of the scan's flat prefix rows; without a basepoint a zero
    row goes in front (the state before the first interval). flat (..., R, 1 + D) -> (..., R [+ 1], D)."""
    lv = flat[..., 1:]
    if basepoint:
        return lv
    z = torch.zeros(lv.shape[:-2] + (1, lv.shape[-1]), dtype=lv.dtype)
    return torch.cat([z, lv], -2)


def binomial_prescale(levels, d, N):
    """ews/block.py:336-357: level k of row t times 1 / C(t_len, k), t_len = max(t + 1, k), via log-gamma."""
    L = levels.shape[-2]
    cols = []
    for k, (s, e) in enumerate(level_slices(d, N), start=1):
        f = []
        for t in range(L):
            tk = max(t + 1.0, float(k))
            f.append(math.exp(-(math.lgamma(tk + 1.0) - math.lgamma(tk - k + 1.0) - math.lgamma(k + 1.0))))
        cols.append(torch.tensor(f, dtype=DT)[:, None].expand(L, e - s))
    return levels * torch.cat(cols, 1)


def graded_rms_norm(x, d, N, variant, eps, gains=None, lam=None):
    """ews/norms.py:115-134. live_rms: g_k block / (RMS + eps_k) with the zero-safe RMS (value and gradient 0
    at ms == 0); static_gain: g_k block; dilation: lam^k block."""
    blocks = []
    for k, (s, e) in enumerate(level_slices(d, N)):
        blk = x[..., s:e]
        if variant == "live_rms":
            ms = torch.mean(blk * blk, dim=-1, keepdim=True)
            safe = torch.where(ms > 0, ms, torch.ones_like(ms))
            rms = torch.where(ms > 0, torch.sqrt(safe), torch.zeros_like(ms))
            blocks.append(gains[k] * blk / (rms + eps[k]))
        elif variant == "static_gain":
            blocks.append(blk * gains[k])
        else:
            blocks.append(blk * lam ** (k + 1))
    return torch.cat(blocks, -1)


def per_level_rms(x, d, N):
    """ews/norms.py:102-113."""
    return torch.stack([torch.sqrt(torch.mean(x[..., s:e] ** 2, dim=-1)) for s, e in level_slices(d, N)], -1)


def mixer_epilogue(flat, weight, bias, d, N, variant, eps, gains=None, lam=None, basepoint=False, prescale=False):
    """ews/block.py:405-406 after _mixer_levels (:282-306) and _prescale (:336-357): per sample,
    ``jax.vmap(c_down)(graded(_prescale(levels)))`` with c_down = eqx.nn.Linear (weight (hidden, D), bias)."""
    lv = levels_from_flat(flat, basepoint)
    if prescale:
        lv = binomial_prescale(lv, d, N)
    y = graded_rms_norm(lv, d, N, variant, eps, gains, lam)
    return y @ weight.t() + bias
