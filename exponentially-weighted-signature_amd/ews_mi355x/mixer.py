"""Mixer epilogue of an EWS block (ews/block.py:282-306, 336-357, 405-408; ews/norms.py:19-134): after the scan,
drop the level-0 column, put a zero row in front (unless basepoint), optionally prescale level k of row t by
1 / C(t + 1, k), normalise each level (GradedRMSNorm) and apply c_down. ``MixerEpilogue`` runs the whole chain
as one fused HIP kernel (forward and backward); ``GradedRMSNorm`` keeps the reference's module (fields, checks,
``per_level_rms``) for the parameters and for standalone use on a flat graded tensor."""

from __future__ import annotations

from typing import Optional, Sequence, Tuple, Union

import torch

from . import ops


def graded_level_slices(d: int, n: int) -> Tuple[Tuple[int, int], ...]:
    """(start, end) of each level block in a level-0-free flat feature [lvl1 | lvl2 | ... | lvlN]
    (ews/norms.py:30-45)."""
    out, start = [], 0
    for k in range(1, n + 1):
        out.append((start, start + d**k))
        start += d**k
    return tuple(out)


class GradedRMSNorm(torch.nn.Module):
    """Per-level normalisation of a flat graded feature (ews/norms.py:47-134):
    live_rms ``g_k x_k / (RMS_k + eps_k)``, static_gain ``g_k x_k``, dilation ``lam**k x_k``; an all-zero level
    maps to zero with a finite gradient. Fields and errors as the reference's."""

    def __init__(self, d: int, N: int, variant: str = "live_rms", eps: Union[float, Sequence[float]] = 1e-3,
                 dtype: torch.dtype = torch.float32):
        super().__init__()
        if variant not in {"live_rms", "static_gain", "dilation"}:
            raise ValueError("variant must be one of {'live_rms', 'static_gain', 'dilation'}.")
        self.d = int(d)
        self.N = int(N)
        self.variant = variant
        self.level_slices = graded_level_slices(self.d, self.N)
        if isinstance(eps, (int, float)):
            eps_t = tuple(float(eps) for _ in range(self.N))
        else:
            eps_t = tuple(float(e) for e in eps)
            if len(eps_t) != self.N:
                raise ValueError("eps must be a scalar or a sequence of length N.")
        self.eps = eps_t
        if variant == "dilation":
            self.gains = None
            self.lam = torch.nn.Parameter(torch.ones((), dtype=dtype))
        else:
            self.gains = torch.nn.Parameter(torch.ones((self.N,), dtype=dtype))
            self.lam = None

    def per_level_rms(self, x: torch.Tensor) -> torch.Tensor:
        """Positionwise RMS of each level block -> (..., N)."""
        return torch.stack([torch.sqrt(torch.mean(x[..., s:e] ** 2, dim=-1)) for s, e in self.level_slices], -1)

    def gain_tensor(self) -> torch.Tensor:
        """The kernel's gains argument: (N,) gains, or lam as a 1-element vector."""
        return self.lam.reshape(1) if self.variant == "dilation" else self.gains

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape[-1] != self.level_slices[-1][1]:
            raise ValueError(f"last axis must be D = {self.level_slices[-1][1]} (level-0-free layout), got "
                             f"{x.shape[-1]}")
        blocks = []
        for k, (s, e) in enumerate(self.level_slices):
            blk = x[..., s:e]
            if self.variant == "live_rms":
                ms = torch.mean(blk * blk, dim=-1, keepdim=True)
                rms = torch.where(ms > 0, torch.sqrt(torch.where(ms > 0, ms, torch.ones_like(ms))),
                                  torch.zeros_like(ms))
                blocks.append(self.gains[k] * blk / (rms + self.eps[k]))
            elif self.variant == "static_gain":
                blocks.append(blk * self.gains[k])
            else:
                blocks.append(blk * self.lam ** (k + 1))
        return torch.cat(blocks, -1)


class MixerEpilogue(torch.nn.Module):
    """``jax.vmap(c_down)(graded(_prescale(levels)))`` of EWSBlock (ews/block.py:405-406) on the flat prefix rows
    of the EWS scan: ``graded`` and ``c_down`` carry the reference block's field names. Input (R, 1 + D) or
    (B, R, 1 + D) float32 on the HIP device; output (R + 1, hidden) rows (R without the leading zero row when
    ``basepoint``). ``graded_prescale="binomial"`` divides level k of levels row t by C(max(t + 1, k), k)."""

    def __init__(self, d: int, N: int, hidden_dim: int, graded_variant: str = "live_rms",
                 graded_eps: Union[float, Sequence[float]] = 1e-3, graded_prescale: Optional[str] = None,
                 basepoint: bool = False, dtype: torch.dtype = torch.float32):
        super().__init__()
        if graded_prescale not in {None, "binomial"}:
            raise ValueError("graded_prescale must be None or 'binomial'.")
        self.d, self.N, self.hidden_dim = int(d), int(N), int(hidden_dim)
        self.D = sum(self.d**k for k in range(1, self.N + 1))
        self.graded_prescale = graded_prescale
        self.basepoint = bool(basepoint)
        self.graded = GradedRMSNorm(self.d, self.N, graded_variant, graded_eps, dtype)
        self.c_down = torch.nn.Linear(self.D, self.hidden_dim, dtype=dtype)

    def forward(self, flat: torch.Tensor) -> torch.Tensor:
        single = flat.dim() == 2
        rows = flat[None] if single else flat
        if rows.shape[-1] != self.D + 1:
            raise ValueError(f"flat rows must carry the level-0 column: last axis {self.D + 1}, got "
                             f"{rows.shape[-1]}")
        r = ops.mixer_epilogue(rows, self.c_down.weight, self.c_down.bias, self.graded.gain_tensor(), self.d,
                               self.N, self.graded.variant, self.graded.eps, prepend=not self.basepoint,
                               prescale=self.graded_prescale == "binomial", level0=True)
        return r[0] if single else r
