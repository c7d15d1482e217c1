"""Front of an EWS block on the HIP device: the clocks of ews/clocks.py, the lift B of ews/params.py and the path
the block hands to its EWS layer (ews/block.py:284-301, 380-395).

The classes mirror the reference's: ``ClockSpec`` (same fields, config keys, checks and error messages),
``FixedClock`` / ``GatedClock`` / ``LearnableBlendedClock`` behind ``make_clock``, the lift ``B`` and a
``BlockFront`` that turns a block's inputs into (path, theta) for ``EWS``. Every clock and the lift run as HIP
kernels (csrc/ews_front.hip), forward and backward, batched over samples: inputs are (batch, seq_len, channels)
tensors, a single (seq_len, channels) sample is accepted as a batch of one. There is no CPU path.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional, Tuple, Union

import torch
import torch.nn as nn

from . import _native as nat
from .ops import ClockFn, LiftFn

CLOCK_MODES = (
    "time",
    "blended_variation",
    "blended_quad_variation",
    "token_gated",
    "clamped_gate",
    "blended_learn",
)
FIXED_MODES = ("time", "blended_variation", "blended_quad_variation")
GATED_MODES = ("token_gated", "clamped_gate")
LEARNED_MODES = ("blended_learn",)
_CLOCK_SCALINGS = {"none", "[0,1]", "[-1,1]", "steps"}
_CLOCK_NORMALIZE = {"per_sample", "constant"}
_ALPHA_PARAMETRISATIONS = {"clip", "sigmoid"}
CLOCK_SOURCES = ("block_input", "encoder_output", "raw_input")


@dataclass(frozen=True)
class ClockSpec:
    """Configuration of one clock (ews/clocks.py:51-124): the field names are the config keys of `clock`."""

    mode: str = "time"
    alpha: float = 1.0
    scaling: str = "[0,1]"
    normalize: str = "per_sample"
    norm_constant: Optional[float] = None
    time_denominator: Optional[float] = None
    variation_eps: float = 1e-8
    stop_gradient: bool = False
    gate_init_scale: Optional[float] = None
    gate_init_bias: Union[float, Tuple[float, ...]] = -2.0
    gate_K: int = 4
    gate_in_scale: float = 1.0
    learn: bool = True
    alpha_parametrisation: str = "clip"
    source: str = "block_input"

    @classmethod
    def from_config(cls, cfg: Optional[dict], **overrides) -> "ClockSpec":
        d = dict(cfg or {})
        d.update(overrides)
        if isinstance(d.get("gate_init_bias"), list):
            d["gate_init_bias"] = tuple(float(x) for x in d["gate_init_bias"])
        unknown = set(d) - set(cls.__dataclass_fields__)
        if unknown:
            raise ValueError(f"unknown clock keys: {sorted(unknown)}")
        return cls(**d)

    def validate(self) -> "ClockSpec":
        if self.mode not in CLOCK_MODES:
            raise ValueError(f"clock mode must be one of {CLOCK_MODES}, got {self.mode!r}")
        if self.scaling not in _CLOCK_SCALINGS:
            raise ValueError("clock scaling must be one of {'none', '[0,1]', '[-1,1]'}.")
        if self.scaling == "steps" and self.mode != "time":
            raise ValueError("clock scaling 'steps' (theta_i = i) is defined for mode 'time' only.")
        if self.normalize not in _CLOCK_NORMALIZE:
            raise ValueError("clock normalize must be one of {'per_sample', 'constant'}.")
        if self.source not in CLOCK_SOURCES:
            raise ValueError(f"clock source must be one of {CLOCK_SOURCES}, got {self.source!r}")
        if self.mode != "time" and not 0.0 <= float(self.alpha) <= 1.0:
            raise ValueError("alpha must be in [0, 1] for blended clock modes.")
        if self.alpha_parametrisation not in _ALPHA_PARAMETRISATIONS:
            raise ValueError(
                f"clock alpha_parametrisation must be one of {sorted(_ALPHA_PARAMETRISATIONS)}, "
                f"got {self.alpha_parametrisation!r}"
            )
        if self.mode in GATED_MODES:
            if not float(self.gate_in_scale) > 0.0:
                raise ValueError(f"clock gate_in_scale must be positive, got {self.gate_in_scale!r}")
            if self.normalize != "constant" or self.norm_constant is None:
                raise ValueError(
                    f"clock mode {self.mode!r} requires normalize='constant' with an explicit norm_constant."
                )
            if self.scaling != "none":
                raise ValueError(f"clock mode {self.mode!r} requires scaling='none'.")
        return self

    @property
    def has_parameters(self) -> bool:
        return self.mode in GATED_MODES or self.mode in LEARNED_MODES


def _check_builder_args(spec: ClockSpec):
    """The extra checks of build_clock_jnp (ews/clocks.py:202-241) for the parameter-free and learned modes."""
    if spec.scaling == "steps" and (spec.mode != "time" or spec.time_denominator is not None):
        raise ValueError("scaling 'steps' is defined for mode 'time' without a time_denominator.")
    if spec.mode != "time" and spec.normalize == "constant" and spec.norm_constant is None:
        raise ValueError("norm_constant is required when normalize='constant'.")


def _batched(driver, mask):
    """A single sample, (L, c) driver and (L,) mask, as a batch of one; returns (driver, mask, squeeze)."""
    squeeze = (driver is not None and driver.dim() == 2) or (driver is None and mask is not None and mask.dim() == 1)
    if squeeze:
        driver = driver[None] if driver is not None else None
        mask = mask[None] if mask is not None and mask.dim() == 1 else mask
    return driver, mask, squeeze


class _JaxClip01(torch.autograd.Function):
    """clip(x, 0, 1) with the derivative of jnp.clip = minimum(maximum(x, 0), 1): 1 inside, 1/2 at a bound (a
    tie of the max or min splits its derivative evenly), 0 outside."""

    @staticmethod
    def forward(ctx, x):
        ctx.save_for_backward(x)
        return x.clamp(0.0, 1.0)

    @staticmethod
    def backward(ctx, g):
        (x,) = ctx.saved_tensors
        w = torch.where((x > 0.0) & (x < 1.0), torch.ones_like(x), torch.zeros_like(x))
        w = torch.where((x == 0.0) | (x == 1.0), torch.full_like(x, 0.5), w)
        return g * w


class Clock(nn.Module):
    """Common interface (ews/clocks.py:370-390): theta = clock(t, driver, mask)."""

    def __init__(self, spec: ClockSpec):
        super().__init__()
        self.spec = spec.validate()

    @property
    def is_static(self) -> bool:
        return not self.spec.has_parameters

    def _params(self, device):
        return None

    def _desc(self, B, L, c, has_mask, increment_driver, basepoint):
        s = self.spec
        mode = nat.CLOCK_MODES[s.mode]
        gated = s.mode in GATED_MODES
        K = (self.w.shape[0] if self.w.dim() == 2 else 1) if gated else 0
        normalize = 1 if (gated or s.normalize == "constant") else 0
        return nat.ClockDesc(
            B, L, c, mode, nat.CLOCK_SCALINGS[s.scaling], normalize, K, int(has_mask), int(increment_driver),
            int(s.time_denominator is not None), int(basepoint), int(s.mode in LEARNED_MODES),
            float(s.alpha), float(s.norm_constant if s.norm_constant is not None else 1.0),
            float(s.time_denominator if s.time_denominator is not None else 1.0), float(s.variation_eps),
            float(getattr(self, "in_scale", 1.0)))

    def forward(self, t, driver, mask=None, *, increment_driver=False, basepoint=False, batch=None):
        """theta of every sample: driver (B, L, c) or (L, c), mask (B, L) or (L,) prefix-structured, t (L,) the
        time base shared by the batch (None: the sample grid). ``increment_driver``: the driver rows are
        increments whose masked cumulative sum is the clock's driver (path_mode "increment");
        ``basepoint``: theta gets a leading copy of its first row; ``batch``: the batch size of a time clock
        given neither driver nor mask."""
        s = self.spec
        if s.mode != "time" and driver is None:
            raise ValueError(
                f"{s.mode} clock requires a driver." if s.mode in GATED_MODES
                else "driver is required for blended clock modes.")
        driver, mask, squeeze = _batched(driver, mask)
        if driver is not None:
            B, L, c = driver.shape
            dev = driver.device
        elif mask is not None:
            B, L = mask.shape
            c, dev = 0, mask.device
        else:
            B, L, c = int(batch or 1), t.shape[0], 0
            dev = t.device
        if t is None:
            t = torch.arange(L, dtype=torch.float32, device=dev)
        t = t.to(device=dev, dtype=torch.float32).contiguous()
        if t.dim() != 1 or t.shape[0] != L:
            raise ValueError("times must be 1D (seq_len,) aligned with the driver.")
        if s.mode == "time":
            drv = None
        else:
            drv = driver
        desc = self._desc(B, L, c, mask is not None, increment_driver, basepoint)
        params = self._params(dev)
        if s.stop_gradient:
            with torch.no_grad():
                theta = ClockFn.apply(drv.detach() if drv is not None else None,
                                      params.detach() if params is not None else None, t, mask, desc)
        else:
            theta = ClockFn.apply(drv, params, t, mask, desc)
        return theta[0] if squeeze else theta

    def per_token_increment(self, embeds):
        raise NotImplementedError


class FixedClock(Clock):
    """time / blended_variation / blended_quad_variation: no parameters (ews/clocks.py:393-433)."""

    def __init__(self, spec: ClockSpec):
        super().__init__(spec)
        _check_builder_args(self.spec)

    def per_token_increment(self, embeds):
        """ews/clocks.py:415-430: the clock increment of each vocabulary token (V, d) -> (V,)."""
        s = self.spec
        if s.normalize != "constant" or s.norm_constant is None:
            raise ValueError("per-token clock increments need normalize='constant'.")
        if s.mode == "time":
            if s.time_denominator is None:
                raise ValueError("time clock needs time_denominator for per-token increments.")
            return torch.full((embeds.shape[0],), 1.0 / float(s.time_denominator), dtype=embeds.dtype,
                              device=embeds.device)
        if float(s.alpha) != 0.0:
            raise ValueError("per-token increments of a blended clock need alpha = 0.")
        sq = torch.sum(embeds ** 2, dim=1)
        if s.mode == "blended_variation":
            return torch.sqrt(sq + s.variation_eps) / s.norm_constant
        return sq / s.norm_constant


class GatedClock(Clock):
    """token_gated / clamped_gate: learnable thresholds on the driver increments (ews/clocks.py:436-476).
    ``key``: an int seed or a torch.Generator for the weight initialisation."""

    def __init__(self, spec: ClockSpec, dim: int, key, dtype=torch.float32):
        super().__init__(spec)
        self.in_scale = float(spec.gate_in_scale)
        gs = float(dim) ** -0.5 if spec.gate_init_scale is None else float(spec.gate_init_scale)
        gen = key if isinstance(key, torch.Generator) else torch.Generator().manual_seed(int(key))
        if spec.mode == "token_gated":
            w = gs * torch.randn((int(dim),), generator=gen, dtype=torch.float64)
            b = torch.tensor(float(spec.gate_init_bias), dtype=torch.float64)
        else:
            if isinstance(spec.gate_init_bias, (list, tuple)):
                b = torch.tensor([float(x) for x in spec.gate_init_bias], dtype=torch.float64)
            else:
                b = torch.full((int(spec.gate_K),), float(spec.gate_init_bias), dtype=torch.float64)
            w = gs * torch.randn((int(b.shape[0]), int(dim)), generator=gen, dtype=torch.float64)
        self.w = nn.Parameter(w.to(dtype), requires_grad=bool(spec.learn))
        self.b = nn.Parameter(b.to(dtype), requires_grad=bool(spec.learn))

    def _params(self, device):
        return torch.cat([self.w.reshape(-1), self.b.reshape(-1)]).to(device=device, dtype=torch.float32)

    def per_token_increment(self, embeds):
        """ews/clocks.py:468-473."""
        c = self.spec.norm_constant
        embeds = embeds * self.in_scale
        if self.spec.mode == "token_gated":
            return torch.relu(embeds @ self.w - self.b) / c
        return torch.clamp(embeds @ self.w.t() - self.b, 0.0, 1.0).sum(-1) / c


class LearnableBlendedClock(Clock):
    """blended_learn: blended_variation with a trainable alpha, held in [0, 1] by a clip or a sigmoid
    (ews/clocks.py:479-525)."""

    _EPS = 1e-4

    def __init__(self, spec: ClockSpec, dtype=torch.float32):
        super().__init__(spec)
        _check_builder_args(self.spec)
        a0 = float(spec.alpha)
        if self.spec.alpha_parametrisation == "sigmoid":
            a0 = min(max(a0, self._EPS), 1.0 - self._EPS)
            a0 = math.log(a0 / (1.0 - a0))
        self.alpha_raw = nn.Parameter(torch.tensor(a0, dtype=dtype), requires_grad=bool(spec.learn))

    @property
    def alpha(self):
        if self.spec.alpha_parametrisation == "sigmoid":
            return torch.sigmoid(self.alpha_raw)
        return _JaxClip01.apply(self.alpha_raw)

    def _params(self, device):
        return self.alpha.reshape(1).to(device=device, dtype=torch.float32)

    def per_token_increment(self, embeds):
        raise NotImplementedError(
            "blended_learn has a trainable alpha, so a token's clock increment is not a constant of the "
            "token: no token cache."
        )


def make_clock(spec: ClockSpec, dim: int, key=None, dtype=torch.float32) -> Clock:
    """ews/clocks.py:528-537: the clock module for `spec`; `key` (seed or generator) only for the gated modes."""
    spec = spec.validate()
    if spec.mode in LEARNED_MODES:
        return LearnableBlendedClock(spec, dtype)
    if spec.has_parameters:
        if key is None:
            raise ValueError(f"clock mode {spec.mode!r} has parameters and needs a key.")
        return GatedClock(spec, dim, key, dtype)
    return FixedClock(spec)


class B(nn.Module):
    """Learnable linear path transformation (ews/params.py:1165-1191): the first channel kept and B on the rest
    (preserve_first_channel=True), or B on every channel."""

    def __init__(self, matrix, preserve_first_channel: bool = True):
        super().__init__()
        self.matrix = nn.Parameter(torch.as_tensor(matrix, dtype=torch.float32).clone())
        self.preserve_first_channel = bool(preserve_first_channel)

    def forward(self, path):
        squeeze = path.dim() == 2
        if squeeze:
            path = path[None]
        if self.preserve_first_channel and path.shape[-1] < 2:
            raise ValueError("preserve_first_channel=True requires path with at least 2 channels")
        p = lift_path(path, None, self, None, increment=False, basepoint=False)
        return p[0] if squeeze else p


def lift_path(branch, theta_app, b_layer, mask, increment=False, basepoint=False):
    """The path of ews/block.py:284-301: u = [theta_app | branch] (branch as its masked cumulative sum under
    path_mode "increment"), p = B(u), forward-filled past the end of the mask, a zero row in front with a
    basepoint. branch (B, L, H), theta_app (B, L) or None, mask (B, L) or None -> (B, L + basepoint, w)."""
    Bn, L, H = branch.shape
    app = theta_app is not None
    Hin = H + int(app)
    if b_layer is None:
        mode, w, matrix = nat.LIFT_NONE, Hin, None
    else:
        matrix = b_layer.matrix
        if b_layer.preserve_first_channel:
            mode, w = nat.LIFT_PRESERVE, matrix.shape[0] + 1
            if tuple(matrix.shape) != (w - 1, Hin - 1):
                raise ValueError(f"B matrix {tuple(matrix.shape)} does not act on {Hin - 1} channels")
        else:
            mode, w = nat.LIFT_FULL, matrix.shape[0]
            if matrix.shape[1] != Hin:
                raise ValueError(f"B matrix {tuple(matrix.shape)} does not act on {Hin} channels")
    desc = nat.LiftDesc(Bn, L, H, int(app), w, mode, int(bool(increment)), int(mask is not None),
                        int(bool(basepoint)))
    return LiftFn.apply(branch, theta_app, matrix, mask, desc)


class BlockFront(nn.Module):
    """The front of EWSBlock (ews/block.py:380-395, 284-301): from the branch input and the clock driver, the
    (path, theta) pair the block hands to its EWS layer, each on the device in one kernel sequence.

    clock, append_clock: ``Clock`` modules (append_clock may be None); b_layer: ``B`` or None; path_mode "value"
    or "increment"; basepoint as the block's."""

    def __init__(self, clock: Clock, b_layer: Optional[B] = None, append_clock: Optional[Clock] = None,
                 path_mode: str = "value", basepoint: bool = False):
        super().__init__()
        if path_mode not in {"value", "increment"}:
            raise ValueError("path_mode must be 'value' or 'increment'.")
        self.clock = clock
        self.append_clock = append_clock
        self.b_layer = b_layer
        self.path_mode = path_mode
        self.basepoint = bool(basepoint)

    def forward(self, branch, driver=None, *, t=None, mask=None):
        """branch (B, L, H) (the block's RMSNorm1(x), or x), driver (B, L, c) (the clock's signal), t (L,),
        mask (B, L) -> path (B, L + basepoint, w), theta (B, L + basepoint)."""
        incr = self.path_mode == "increment"
        if mask is not None and mask.dim() == 1:
            mask = mask[None].expand(branch.shape[0], -1)
        if t is None:
            t = torch.arange(branch.shape[1], dtype=torch.float32, device=branch.device)
        kw = dict(increment_driver=incr and driver is not None, batch=branch.shape[0])
        theta = self.clock(t, driver, mask, basepoint=self.basepoint, **kw)
        theta_app = None
        if self.append_clock is not None:
            theta_app = self.append_clock(t, driver, mask, **kw)
        path = lift_path(branch, theta_app, self.b_layer, mask, increment=incr, basepoint=self.basepoint)
        return path, theta
