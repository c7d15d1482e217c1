"""EWS blocks and the stacked model (ews/block.py:36-756): the residual scaffold the reference wraps around its EWS
layer, assembled from this package's device pieces.

Per block (norm_placement "pre", ews/block.py:376-424):

    theta, p = BlockFront(RMSNorm1(x), driver)     the clock and the lift, one kernel sequence (csrc/ews_front.hip)
    S        = EWS prefix rows of (p, theta)       the scan kernels
    r        = c_down(GradedRMSNorm(S))            the fused mixer epilogue (csrc/ews_mixer.hip)
    x        = x + Dropout(r [* sigmoid(gate(branch))])
    x        = x + Dropout(channel_stage(RMSNorm2(x)))

The norms, the gate and the channel stage (plain linear maps and pointwise functions around the scan) are torch
operations. Field names follow the reference (``norm1``, ``ewms``, ``graded``, ``c_down``, ``gate``, ``norm2``,
``ff1``, ``ff2``, ``clock``, ``append_clock``, ``b_layer``), so a checkpoint converted key by key loads into the
same places. Two differences from the reference's constructor: the generator is passed as a module (``a_param``,
any parametrisation of ``ews_mi355x.params``; default the reference's definite_plus_skew with entries N(0, 0.005))
instead of an ``a_config`` dict, and ``key`` is an int seed or a ``torch.Generator`` (initial values are drawn from
the same distributions as the reference's, not the same numbers). Dropout draws from torch's generator.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from .front import B, BlockFront, ClockSpec, make_clock
from .layer import EWS
from .mixer import MixerEpilogue
from .params import AParamBoundedRotation, AParamDampedRotation, AParamDefinitePlusSkew, is_rotation_planes

BOUNDED_PAD_ID = 0  # the token id the bounded-rotation scale ignores (ews/block.py:26)


def _generator(key):
    if isinstance(key, torch.Generator):
        return key
    return torch.Generator().manual_seed(0 if key is None else int(key))


def _spec(clock) -> Optional[ClockSpec]:
    if clock is None or isinstance(clock, ClockSpec):
        return clock
    return ClockSpec.from_config(clock)


def _linear(fan_in, fan_out, gen, dtype):
    """A Linear map with the reference's initialisation (weights and bias U(-1/sqrt(in), 1/sqrt(in)))."""
    lin = nn.Linear(fan_in, fan_out, dtype=dtype)
    lim = 1.0 / math.sqrt(fan_in)
    with torch.no_grad():
        lin.weight.copy_((torch.rand((fan_out, fan_in), generator=gen, dtype=torch.float64) * 2 - 1) * lim)
        lin.bias.copy_((torch.rand((fan_out,), generator=gen, dtype=torch.float64) * 2 - 1) * lim)
    return lin


class RMSNorm(nn.Module):
    """ews/norms.py:13-27: x * rsqrt(mean(x^2) + eps) * weight over the last axis, weight initialised to ones."""

    def __init__(self, dim: int, eps: float = 1e-6, dtype: torch.dtype = torch.float32):
        super().__init__()
        self.eps = float(eps)
        self.weight = nn.Parameter(torch.ones((int(dim),), dtype=dtype))

    def forward(self, x):
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + self.eps) * self.weight


def increment_path(p, mask):
    """ews/paths.py:126-131: rows are per-step increments, the path is their cumulative sum; pads are zeroed
    first. p (B, L, c), mask (B, L) or None."""
    if mask is not None:
        p = p * mask[..., None].to(p.dtype)
    return torch.cumsum(p, dim=-2)


class EWSBlock(nn.Module):
    """A residual layer around an EWS mixer (ews/block.py:36-470). Arguments as the reference's, with ``a_param``
    (a generator parametrisation module) in place of ``a_config`` and ``b_matrix`` / ``lift`` in place of
    ``b_config``: ``b_matrix`` (out, in) sets the lift matrix, ``lift=False`` drops the lift (p = u).

    Input (L, hidden_dim) or (B, L, hidden_dim) on the HIP device; the output has the same shape."""

    def __init__(self, hidden_dim: int, m: int = 8, n: int = 1, *, a_param: Optional[nn.Module] = None,
                 b_matrix: Optional[torch.Tensor] = None, lift: bool = True, M: int = 4,
                 reweighting_mode: str = "displacement", terminal_reduce: str = "tree", van_loan_expm: str = "exact",
                 chen_expm: str = "exact", leaf: str = "van_loan", series_q: Optional[int] = None,
                 combine: str = "assoc", combine_chunk: int = 1024, combine_tile: int = 4,
                 jordan_flows: bool = False, basepoint: bool = False, clock=None, append_clock=None,
                 norm_placement: str = "pre", second_norm: bool = True, graded_norm: str = "live_rms",
                 graded_eps: Union[float, Sequence[float]] = 1e-3, channel_stage: str = "mlp",
                 graded_prescale: Optional[str] = None, path_mode: str = "value", ff_mult: int = 4,
                 output_gate: bool = False, dropout_rate: float = 0.01, norm_eps: float = 1e-6,
                 dtype: torch.dtype = torch.float32, key=None):
        super().__init__()
        if norm_placement not in {"pre", "slice_post", "none"}:
            raise ValueError("norm_placement must be one of {'pre', 'slice_post', 'none'}.")
        if channel_stage not in {"mlp", "tanh", "glu", "gelu_glu"}:
            raise ValueError("channel_stage must be one of {'mlp', 'tanh', 'glu', 'gelu_glu'}.")
        if graded_prescale not in {None, "binomial"}:
            raise ValueError("graded_prescale must be None or 'binomial'.")
        if path_mode not in {"value", "increment"}:
            raise ValueError("path_mode must be 'value' or 'increment'.")
        clock_spec = (_spec(clock) or ClockSpec()).validate()
        append_spec = None if append_clock is None else _spec(append_clock).validate()
        self.hidden_dim, self.m, self.n = int(hidden_dim), int(m), int(n)
        self.basepoint = bool(basepoint)
        self.norm_placement = norm_placement
        self.second_norm = bool(second_norm)
        self.channel_stage = channel_stage
        self.output_gate = bool(output_gate)
        self.dropout_rate = float(dropout_rate)
        self.path_mode = path_mode
        self.graded_prescale = graded_prescale
        self.dtype = dtype
        gen = _generator(key)
        H = self.hidden_dim
        append_on = append_spec is not None
        d_in = H + int(append_on)
        # the lift: out_dim m (+1 with an appended clock channel, which it preserves) (ews/block.py:176-195)
        if not lift:
            self.b_layer = None
            w = d_in
        else:
            if b_matrix is None:
                shape = (self.m, d_in - 1) if append_on else (self.m, d_in)
                b_matrix = torch.randn(shape, generator=gen, dtype=torch.float64) / math.sqrt(float(H))
            self.b_layer = B(torch.as_tensor(b_matrix, dtype=dtype), preserve_first_channel=append_on)
            w = b_matrix.shape[0] + int(append_on)
        self.w_eff = int(w)
        self.D = sum(self.w_eff**k for k in range(1, self.n + 1))
        if a_param is None:  # the reference block's default: definite_plus_skew, entries N(0, 0.005)
            sd = math.sqrt(0.005)
            nl, nu = w * (w + 1) // 2, w * (w - 1) // 2
            a_param = AParamDefinitePlusSkew(
                (sd * torch.randn((nl,), generator=gen, dtype=torch.float64)).to(dtype),
                (sd * torch.randn((nu,), generator=gen, dtype=torch.float64)).to(dtype), w)
        if int(a_param.dim) != self.w_eff:
            raise ValueError(f"a_param has width {a_param.dim}, the lift produces {self.w_eff} channels")
        self.ewms = EWS(a_param, N=self.n, M=int(M), dtype=dtype, reweighting_mode=reweighting_mode,
                        terminal_reduce=terminal_reduce, van_loan_expm=van_loan_expm, chen_expm=chen_expm,
                        leaf=leaf, series_q=series_q, combine=combine, combine_chunk=combine_chunk,
                        combine_tile=combine_tile, jordan_flows=jordan_flows)
        self.mixer = MixerEpilogue(self.w_eff, self.n, H, graded_variant=graded_norm, graded_eps=graded_eps,
                                   graded_prescale=graded_prescale, basepoint=self.basepoint, dtype=dtype)
        mixer_c = _linear(self.D, H, gen, dtype)
        with torch.no_grad():
            self.mixer.c_down.weight.copy_(mixer_c.weight)
            self.mixer.c_down.bias.copy_(mixer_c.bias)
        self.gate = _linear(H, H, gen, dtype) if self.output_gate else None
        # calls that record no graph run the epilogue inside the scan's output pass where the scan allows it
        # (EWS.mixed_prefix); False keeps the scan -> epilogue composition for every call
        self.fused_epilogue = True
        if norm_placement == "pre":
            self.norm1 = RMSNorm(H, norm_eps, dtype)
            self.norm2 = RMSNorm(H, norm_eps, dtype) if self.second_norm else None
        elif norm_placement == "slice_post":
            self.norm1 = None
            self.norm2 = nn.LayerNorm(H, eps=norm_eps, dtype=dtype)
        else:
            self.norm1 = self.norm2 = None
        if channel_stage == "mlp":
            if ff_mult < 1:
                raise ValueError("ff_mult must be at least 1.")
            self.ff1, self.ff2 = _linear(H, ff_mult * H, gen, dtype), _linear(ff_mult * H, H, gen, dtype)
        elif channel_stage == "tanh":
            self.ff1, self.ff2 = _linear(H, H, gen, dtype), None
        elif channel_stage == "glu":
            self.ff1, self.ff2 = _linear(H, 2 * H, gen, dtype), None
        else:  # gelu_glu
            self.ff1, self.ff2 = _linear(H, H, gen, dtype), _linear(H, H, gen, dtype)
        self.clock = make_clock(clock_spec, H, key=int(torch.randint(0, 2**31 - 1, (1,), generator=gen)), dtype=dtype)
        self.append_clock = (None if append_spec is None else
                             make_clock(append_spec, H, key=int(torch.randint(0, 2**31 - 1, (1,), generator=gen)),
                                        dtype=dtype))
        self.front = BlockFront(self.clock, self.b_layer, self.append_clock, path_mode, self.basepoint)

    # the reference's field names for the mixer's parts
    @property
    def graded(self):
        return self.mixer.graded

    @property
    def c_down(self):
        return self.mixer.c_down

    def _resolve_driver(self, x, clock_driver):
        """ews/block.py:269-280."""
        if self.clock.spec.source == "block_input":
            return x
        if clock_driver is None and self.clock.spec.mode != "time":
            raise ValueError(f"clock_driver is required for clock source '{self.clock.spec.source}'.")
        return clock_driver

    def _channel(self, xhat):
        """ews/block.py:361-374 (jax.nn.gelu is the tanh approximation)."""
        if self.channel_stage == "mlp":
            return self.ff2(F.gelu(self.ff1(xhat), approximate="tanh"))
        if self.channel_stage == "tanh":
            return torch.tanh(self.ff1(xhat))
        if self.channel_stage == "glu":
            a, b = self.ff1(xhat).chunk(2, dim=-1)
            return a * torch.sigmoid(b)
        h = F.gelu(xhat, approximate="tanh")
        return self.ff1(h) * torch.sigmoid(self.ff2(h))

    def _drop(self, x, inference):
        if inference or self.dropout_rate == 0.0:
            return x
        return F.dropout(x, self.dropout_rate, training=True)

    def mixer_levels(self, x, *, t=None, mask=None, clock_driver=None, a_scale=1.0):
        """The flat prefix rows the block's scan produces (level 0 included), (B, R, 1 + D): the pre-epilogue
        features of ews/block.py:308-334 before the level-0 column is dropped."""
        driver = self._resolve_driver(x, clock_driver)
        branch_in = self.norm1(x) if self.norm_placement == "pre" else x
        path, theta = self.front(branch_in, driver, t=t, mask=mask)
        return self.ewms(path, theta, readout="prefix", output_format="flat", a_scale=a_scale)

    def forward(self, x, *, t=None, mask=None, clock_driver=None, inference: bool = False, a_scale=1.0):
        """ews/block.py:376-470: x (L, H) or (B, L, H); t (L,); mask (L,) or (B, L); clock_driver as x's
        batch."""
        if x.dim() == 2:
            out = self.forward(x[None], t=t, mask=None if mask is None else mask.reshape(1, -1),
                               clock_driver=None if clock_driver is None else clock_driver[None],
                               inference=inference, a_scale=a_scale)
            return out[0]
        if x.dim() != 3:
            raise ValueError(f"x must be 2D or 3D, got shape {tuple(x.shape)}")
        if mask is not None and mask.dim() == 1:
            mask = mask[None].expand(x.shape[0], -1)
        driver = self._resolve_driver(x, clock_driver)
        branch_in = self.norm1(x) if self.norm_placement == "pre" else x
        path, theta = self.front(branch_in, driver, t=t, mask=mask)
        r = None
        if self.fused_epilogue and not (torch.is_grad_enabled() and _needs_grad(path, theta, self)):
            # no graph recorded: the scan's output pass runs the epilogue itself (no D-wide rows in memory); a
            # training step composes the scan and the epilogue, whose backward does not regenerate the rows
            r = self.ewms.mixed_prefix(path, theta, self.mixer, a_scale=a_scale)
        if r is None:
            rows = self.ewms(path, theta, readout="prefix", output_format="flat", a_scale=a_scale)
            r = self.mixer(rows)
        if self.gate is not None:
            g_in = increment_path(branch_in, mask) if self.path_mode == "increment" else branch_in
            r = r * torch.sigmoid(self.gate(g_in))
        if self.norm_placement == "slice_post":
            y = x + r
            y = y + self._channel(y)
            return self._drop(self.norm2(y), inference)
        x = x + self._drop(r, inference)
        xhat = self.norm2(x) if (self.norm_placement == "pre" and self.norm2 is not None) else x
        return x + self._drop(self._channel(xhat), inference)


def _needs_grad(path, theta, module):
    return path.requires_grad or theta.requires_grad or any(p.requires_grad for p in module.parameters())


class StackedEWS(nn.Module):
    """An encoder, ``num_blocks`` EWSBlocks and a head (ews/block.py:473-756). The encoder is an Embedding for
    tokens (``tokens=True``) or a Linear map for series; the head acts per position ("seq2seq") or on a masked mean
    ("mean_pool"); ``label_dim`` may be a tuple for several heads. Blocks whose clock source is "encoder_output"
    read the encoder output, "raw_input" blocks the ``raw_driver`` argument."""

    def __init__(self, num_blocks: int, data_dim: int, hidden_dim: int, label_dim: Union[int, Tuple[int, ...]], *,
                 tokens: bool = True, head_mode: str = "seq2seq", final_norm: bool = False,
                 cosine_head_tau: Optional[float] = None, input_token_ids: Optional[Sequence[int]] = None,
                 block_kwargs: Optional[dict] = None, per_block_kwargs: Optional[Sequence[dict]] = None,
                 dtype: torch.dtype = torch.float32, key=None):
        super().__init__()
        if num_blocks < 1:
            raise ValueError("num_blocks must be at least 1.")
        if head_mode not in {"seq2seq", "mean_pool"}:
            raise ValueError("head_mode must be one of {'seq2seq', 'mean_pool'}.")
        if per_block_kwargs is not None and len(per_block_kwargs) != num_blocks:
            raise ValueError("per_block_kwargs must have length num_blocks.")
        self.tokens = bool(tokens)
        self.head_mode = head_mode
        self.cosine_head_tau = None if cosine_head_tau is None else float(cosine_head_tau)
        self.input_token_ids = None if input_token_ids is None else tuple(int(i) for i in input_token_ids)
        self.num_blocks, self.data_dim, self.hidden_dim = int(num_blocks), int(data_dim), int(hidden_dim)
        self.dtype = dtype
        gen = _generator(key)
        if self.tokens:
            self.embedding = nn.Embedding(self.data_dim, self.hidden_dim, dtype=dtype)
            with torch.no_grad():
                self.embedding.weight.copy_(torch.randn((self.data_dim, self.hidden_dim), generator=gen,
                                                        dtype=torch.float64))
        else:
            self.embedding = _linear(self.data_dim, self.hidden_dim, gen, dtype)
        base = dict(block_kwargs or {})
        blocks = []
        for i in range(self.num_blocks):
            kw = dict(base)
            if per_block_kwargs is not None:
                kw.update(per_block_kwargs[i])
            kw.setdefault("key", int(torch.randint(0, 2**31 - 1, (1,), generator=gen)))
            blocks.append(EWSBlock(self.hidden_dim, dtype=dtype, **kw))
        self.blocks = nn.ModuleList(blocks)
        if isinstance(label_dim, int):
            self.label_dim = int(label_dim)
            self.head = _linear(self.hidden_dim, self.label_dim, gen, dtype)
        elif isinstance(label_dim, tuple):
            self.label_dim = tuple(int(x) for x in label_dim)
            self.head = nn.ModuleList([_linear(self.hidden_dim, ld, gen, dtype) for ld in self.label_dim])
        else:
            raise TypeError("label_dim must be int or tuple of int")
        self.final_norm = RMSNorm(self.hidden_dim, dtype=dtype) if final_norm else None

    def _mask_phantom(self, vals):
        """ews/block.py:679-687: -inf at the pad id and at ids outside input_token_ids."""
        vals = vals.clone()
        vals[BOUNDED_PAD_ID] = -math.inf
        if self.input_token_ids is not None:
            keep = torch.zeros_like(vals, dtype=torch.bool)
            keep[list(self.input_token_ids)] = True
            vals = torch.where(keep, vals, torch.full_like(vals, -math.inf))
        return vals

    def bounded_a_scale(self, i: int):
        """ews/block.py:626-677: 2 pi / dtheta_max for a rotation-plane block of a token model (dtheta_max the
        largest per-token clock increment over the embedding table, pad excluded, no gradient); 1.0 otherwise."""
        block = self.blocks[i]
        # the gate keys on the class as the reference's does, by the five rotation-plane class names it lists
        # (AParamBounded/Clamped/Damped/ReluDamped/UnboundedRotation): a parametrisation of any of them, this
        # module's or a caller's own, gets the bounded scale, never a silent 1.0
        if not (self.tokens and is_rotation_planes(block.ewms.A_param)):
            return 1.0
        spec = block.clock.spec
        c = spec.norm_constant or 1.0
        E = self.embedding.weight
        reads = spec.source == "encoder_output" or (spec.source == "block_input" and i == 0)
        with torch.no_grad():
            if reads and spec.mode == "token_gated":
                dth = torch.relu(E @ block.clock.w - block.clock.b)
            elif reads and spec.mode == "clamped_gate":
                dth = torch.clamp(E @ block.clock.w.t() - block.clock.b, 0.0, 1.0).sum(-1)
            else:
                dth = torch.linalg.norm(E, dim=1)
            dth = self._mask_phantom(dth)
            dmax = torch.clamp(dth.max(), min=1e-6) / c
        return 2.0 * math.pi / dmax

    def hidden(self, X, *, t=None, mask=None, raw_driver=None, inference: bool = False):
        """ews/block.py:581-624 for a batch: encoder and blocks, no head -> (B, L, hidden_dim)."""
        h = self.embedding(X.long()) if self.tokens else self.embedding(X)
        enc = h
        for i, block in enumerate(self.blocks):
            driver = None
            if block.clock.spec.source == "encoder_output":
                driver = enc
            elif block.clock.spec.source == "raw_input":
                driver = raw_driver
            h = block(h, t=t, mask=mask, clock_driver=driver, inference=inference, a_scale=self.bounded_a_scale(i))
        if self.final_norm is not None:
            h = self.final_norm(h)
        return h

    def _cosine_logits(self, head, h):
        W = head.weight
        W_hat = W / (torch.linalg.norm(W, dim=1, keepdim=True) + 1e-8)
        h_hat = h / (torch.linalg.norm(h, dim=-1, keepdim=True) + 1e-8)
        return (h_hat @ W_hat.t()) / self.cosine_head_tau

    def _apply_head(self, head, h, mask):
        """ews/block.py:695-707."""
        if self.head_mode == "seq2seq":
            return self._cosine_logits(head, h) if self.cosine_head_tau is not None else head(h)
        if mask is not None:
            w = mask.to(h.dtype)[..., None]
            pooled = (h * w).sum(-2) / torch.clamp(w.sum(-2), min=1.0)
        else:
            pooled = h.mean(-2)
        return self._cosine_logits(head, pooled) if self.cosine_head_tau is not None else head(pooled)

    def forward(self, X, *, t=None, mask=None, raw_driver=None, inference: bool = False):
        """ews/block.py:709-756: tokens (L,) / (B, L) or series (L, c) / (B, L, c)."""
        single = X.dim() == (1 if self.tokens else 2)
        if single:
            out = self.forward(X[None], t=t, mask=None if mask is None else mask.reshape(1, -1),
                               raw_driver=None if raw_driver is None else raw_driver[None], inference=inference)
            return tuple(o[0] for o in out) if isinstance(out, tuple) else out[0]
        if mask is not None and mask.dim() == 1:
            mask = mask[None].expand(X.shape[0], -1)
        h = self.hidden(X, t=t, mask=mask, raw_driver=raw_driver, inference=inference)
        if isinstance(self.head, nn.ModuleList):
            return tuple(self._apply_head(hd, h, mask) for hd in self.head)
        return self._apply_head(self.head, h, mask)
