"""Generator parametrisations the layer needs to recognise: the materialised A (d, d) plus its static structure.

The reference keeps 18 families (ews/params.py:61-80); the scan only ever sees the materialised matrix and
the structure its class implies (ews/core/kernels/combine.py:37-63). This module provides the families whose
structure selects a kernel here, with the reference's class and field names so code written against the
reference constructs them the same way:

    AParamConstant / AParamGeneral    dense A                       (ews/params.py:268-277)
    AParamEFM                         positive diagonal              (ews/params.py:280-301)
    AParamBlockDiag                   free diagonal blocks
    AParamBoundedRotation             planes [[0, -b], [b, 0]]       (ews/params.py:538-566)
    AParamDampedRotation              planes [[a, -b], [b, a]]       (ews/params.py:569-606)
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

ROTATION_CLASSES = (
    "AParamBoundedRotation",
    "AParamDampedRotation",
    "AParamReluDampedRotation",
    "AParamClampedRotation",
    "AParamUnboundedRotation",
)


class AParamConstant(torch.nn.Module):
    """A fixed (non-trainable) generator."""

    def __init__(self, A: torch.Tensor):
        super().__init__()
        self.register_buffer("A", A)
        self.dim = int(A.shape[0])

    def forward(self):
        return self.A


class AParamGeneral(torch.nn.Module):
    def __init__(self, matrix: torch.Tensor):
        super().__init__()
        self.matrix = torch.nn.Parameter(matrix)
        self.dim = int(matrix.shape[0])

    def forward(self):
        return self.matrix


class AParamEFM(torch.nn.Module):
    """Positive diagonal: softplus(theta) or theta**2 per channel."""

    def __init__(self, theta: torch.Tensor, positivity: str = "softplus"):
        super().__init__()
        if positivity not in ("softplus", "square"):
            raise ValueError(f"efm positivity must be one of ('softplus', 'square'), got {positivity!r}")
        self.theta = torch.nn.Parameter(theta)
        self.positivity = positivity
        self.dim = int(theta.shape[0])

    def diagonal(self):
        return self.theta**2 if self.positivity == "square" else F.softplus(self.theta)

    def forward(self):
        return torch.diag(self.diagonal())


class AParamBlockDiag(torch.nn.Module):
    def __init__(self, blocks, sizes):
        super().__init__()
        self.blocks = torch.nn.ParameterList([torch.nn.Parameter(b) for b in blocks])
        self.sizes = [int(s) for s in sizes]
        self.dim = int(sum(self.sizes))

    def forward(self):
        return torch.block_diag(*self.blocks)


class AParamBoundedRotation(torch.nn.Module):
    """Planes [[0, -omega_j], [omega_j, 0]], omega_j = omega_scale * sigmoid(u_j)."""

    def __init__(self, u: torch.Tensor, dim: int, omega_scale: float = 1.0):
        super().__init__()
        if int(dim) % 2:
            raise ValueError("bounded_rotation requires even A width (2 rows per plane)")
        self.u = torch.nn.Parameter(u)
        self.dim = int(dim)
        self.omega_scale = float(omega_scale)

    def plane_params(self):
        """(P, 2) rows (d_j, w_j) of the canonical plane form [[d, w], [-w, d]]."""
        om = self.omega_scale * torch.sigmoid(self.u)
        return torch.stack([torch.zeros_like(om), -om], -1)

    def forward(self):
        return _planes_to_dense(self.plane_params())


class AParamDampedRotation(torch.nn.Module):
    """Planes [[a_j, -b_j], [b_j, a_j]], a_j = softplus(v_j), b_j = omega_scale * sigmoid(u_j)."""

    def __init__(self, v: torch.Tensor, u: torch.Tensor, dim: int, omega_scale: float = 1.0):
        super().__init__()
        if int(dim) % 2:
            raise ValueError("damped_rotation requires even A width (2 rows per plane)")
        self.v = torch.nn.Parameter(v)
        self.u = torch.nn.Parameter(u)
        self.dim = int(dim)
        self.omega_scale = float(omega_scale)

    def plane_params(self):
        a = F.softplus(self.v)
        b = self.omega_scale * torch.sigmoid(self.u)
        return torch.stack([a, -b], -1)

    def forward(self):
        return _planes_to_dense(self.plane_params())


def _planes_to_dense(dw):
    """(P, 2) rows (d_j, w_j) -> block-diagonal (2P, 2P) with blocks [[d, w], [-w, d]]."""
    P = dw.shape[0]
    A = torch.zeros((2 * P, 2 * P), dtype=dw.dtype, device=dw.device)
    i = torch.arange(P, device=dw.device)
    A = A.index_put((2 * i, 2 * i), dw[:, 0])
    A = A.index_put((2 * i + 1, 2 * i + 1), dw[:, 0])
    A = A.index_put((2 * i, 2 * i + 1), dw[:, 1])
    A = A.index_put((2 * i + 1, 2 * i), -dw[:, 1])
    return A


def block_sizes_of(a_param):
    """Diagonal-block sizes of a parametrisation, from its class (ews/core/kernels/combine.py:37-58)."""
    if isinstance(a_param, AParamBlockDiag):
        return tuple(a_param.sizes)
    if type(a_param).__name__ in ROTATION_CLASSES:
        d = int(a_param.dim)
        return None if d % 2 else (2,) * (d // 2)
    return None


def is_rotation_planes(a_param):
    """combine.py:61-63."""
    return type(a_param).__name__ in ROTATION_CLASSES


def diagonal_structure(a_param):
    """Which diagonal kernel a parametrisation can use: "planes", "real_diag" or None."""
    if is_rotation_planes(a_param):
        return "planes"
    if isinstance(a_param, AParamEFM):
        return "real_diag"
    if isinstance(a_param, AParamBlockDiag) and all(s == 1 for s in a_param.sizes):
        return "real_diag"
    return None
