"""CPU float64 restatement of the front of an EWS block: the clock theta(t, driver, mask), the increment path, the
lift B, the forward fill past the end of the mask and the basepoint row.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports, links or runs this file; ``tests/`` use it as the
checker of the HIP clock and lift kernels. Written with torch float64 tensors, batched over a leading sample axis,
so that gradients come from autograd of the same restatement. Every function cites the reference file:line it
restates.
"""

from __future__ import annotations

import torch

DT = torch.float64


def scale_component(c, scaling):
    """ews/clocks.py:129-147 (_scale_clock_component_jnp), over the last axis: the per-sample affine map of a monotone
    component onto [0, 1] or [-1, 1] through its first and last values (+1e-12), 'steps' = the sample index."""
    if scaling == "none":
        return c
    if scaling == "steps":
        return torch.arange(c.shape[-1], dtype=c.dtype).expand(c.shape)
    z = (c - c[..., :1]) / ((c[..., -1:] - c[..., :1]) + 1e-12)
    if scaling == "[0,1]":
        return z
    if scaling == "[-1,1]":
        return 2.0 * z - 1.0
    raise ValueError(scaling)


def range_map(z, scaling):
    """ews/clocks.py:150-161 (_range_map_jnp)."""
    if scaling in ("none", "[0,1]"):
        return z
    if scaling == "[-1,1]":
        return 2.0 * z - 1.0
    raise ValueError(scaling)


def _pairs(mask):
    """Increment s (between rows s - 1 and s) counts when both ends are real (ews/clocks.py:252-254)."""
    return (mask[:, 1:] & mask[:, :-1]).to(DT)


def _freeze(theta, mask):
    """ews/clocks.py:262-264: theta held at row n = sum(mask) - 1 past the end. jnp.take with n = -1 (no real row)
    reads the last row, as negative indices count from the end."""
    if mask is None:
        return theta
    n = mask.to(torch.int64).sum(-1, keepdim=True) - 1
    L = theta.shape[-1]
    idx = torch.where(n >= 0, n, n + L)
    frozen = torch.gather(theta, -1, idx)
    return torch.where(torch.arange(L)[None, :] <= n, theta, frozen)


def _cumsum0(incr):
    return torch.cat([torch.zeros(incr.shape[:-1] + (1,), dtype=incr.dtype), torch.cumsum(incr, -1)], -1)


def build_clock(t, driver, mode, alpha, scaling, mask=None, normalize="per_sample", norm_constant=None,
                time_denominator=None, variation_eps=1e-8, stop_gradient=False):
    """ews/clocks.py:164-267 (build_clock_jnp), batched: t (L,), driver (B, L, c), mask (B, L) bool -> (B, L).
    theta = alpha * t_s + (1 - alpha) * V_s (blended modes) or t_s ("time")."""
    B = driver.shape[0] if driver is not None else (mask.shape[0] if mask is not None else 1)
    t = t.to(DT)
    L = t.shape[0]
    if time_denominator is None:
        t_s = scale_component(t, scaling)
    else:
        t_s = range_map((t - t[0]) / float(time_denominator), scaling)
    t_s = t_s.expand(B, L)
    if mode == "time":
        theta = t_s
    else:
        dx = driver[:, 1:] - driver[:, :-1]
        sq = (dx * dx).sum(-1)
        incr = torch.sqrt(sq + variation_eps) if mode == "blended_variation" else sq
        if mask is not None:
            incr = incr * _pairs(mask)
        V = _cumsum0(incr)
        if normalize == "per_sample":
            V_s = scale_component(V, scaling)
        else:
            V_s = range_map(V / float(norm_constant), scaling)
        theta = alpha * t_s + (1.0 - alpha) * V_s
    theta = _freeze(theta, mask)
    return theta.detach() if stop_gradient else theta


def gated_clock(driver, mode, w, b, norm_constant, in_scale=1.0, mask=None, stop_gradient=False):
    """ews/clocks.py:443-466 (GatedClock.__call__): the driver scaled before the difference, increments
    relu(w . dx - b) (token_gated, w (c,), b scalar) or sum_k clip(w_k . dx - b_k, 0, 1) (clamped_gate, w (K, c),
    b (K,)), cumulated and divided by norm_constant."""
    s = driver * in_scale
    dx = s[:, 1:] - s[:, :-1]
    if mode == "clamped_gate":
        incr = torch.clamp(dx @ w.t() - b, 0.0, 1.0).sum(-1)
    else:
        incr = torch.relu(dx @ w - b)
    if mask is not None:
        incr = incr * _pairs(mask)
    theta = _cumsum0(incr) / float(norm_constant if norm_constant is not None else 1.0)
    theta = _freeze(theta, mask)
    return theta.detach() if stop_gradient else theta


def learned_alpha(alpha_raw, parametrisation):
    """ews/clocks.py:502-506 (LearnableBlendedClock.alpha). jnp.clip is minimum(maximum(x, 0), 1), whose
    derivative is 1/2 at a bound (ties split evenly, as torch.maximum / torch.minimum also do)."""
    if parametrisation == "sigmoid":
        return torch.sigmoid(alpha_raw)
    zero = torch.zeros((), dtype=alpha_raw.dtype)
    return torch.minimum(torch.maximum(alpha_raw, zero), zero + 1.0)


def increment_path(p, mask):
    """ews/paths.py:126-131 (to_increment_path_jnp): pads zeroed, then the cumulative sum over rows."""
    if mask is not None:
        p = p * mask[..., None].to(p.dtype)
    return torch.cumsum(p, -2)


def lift(u, matrix, preserve_first_channel):
    """ews/params.py:1181-1191 (B.__call__): u @ B^T, or the first channel kept and B on the rest."""
    if matrix is None:
        return u
    if preserve_first_channel:
        return torch.cat([u[..., :1], u[..., 1:] @ matrix.t()], -1)
    return u @ matrix.t()


def forward_fill(arr, mask):
    """ews/block.py:29-33 (_forward_fill), batched: rows past n = sum(mask) - 1 take row n (the last row when no
    row is real, as jnp.take counts negative indices from the end)."""
    if mask is None:
        return arr
    L = arr.shape[-2]
    n = mask.to(torch.int64).sum(-1) - 1
    idx = torch.minimum(torch.arange(L)[None, :], n[:, None])
    idx = torch.where(idx >= 0, idx, idx + L)
    return torch.gather(arr, -2, idx[..., None].expand(arr.shape))


def block_front(branch, theta, theta_app, mask, matrix, preserve_first_channel, increment, basepoint):
    """ews/block.py:284-301 (_mixer_levels up to the EWS call) with the increment representation of
    ews/block.py:393-395: u = [theta_app | branch], p = B(u), forward fill, basepoint row. Returns (p_in, theta_in),
    the path and clock the block hands to its EWS layer."""
    if increment:
        branch = increment_path(branch, mask)
    u = branch if theta_app is None else torch.cat([theta_app[..., None].to(branch.dtype), branch], -1)
    p = lift(u, matrix, preserve_first_channel)
    p = forward_fill(p, mask)
    if basepoint:
        p = torch.cat([torch.zeros_like(p[:, :1]), p], 1)
        theta = torch.cat([theta[:, :1], theta], 1)
    return p, theta
