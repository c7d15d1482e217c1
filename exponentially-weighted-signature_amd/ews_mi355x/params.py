"""Generator parametrisations the layer needs to recognise: the materialised A (d, d) plus its static structure.

The reference keeps 18 families (ews/params.py:61-80); the scan only ever sees the materialised matrix and
the structure its class implies (ews/core/kernels/combine.py:37-63). This module provides the families whose
structure selects a kernel here, with the reference's class and field names so code written against the
reference constructs them the same way:

    AParamConstant / AParamGeneral    dense A                       (ews/params.py:268-277)
    AParamDefinitePlusSkew            L L^T + eps I + (U - U^T)      (ews/params.py:372-391; EWSBlock's default)
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


class AParamDefinitePlusSkew(torch.nn.Module):
    """A = L L^T + epsilon I + (U - U^T): ``lower`` fills the lower triangle of L (diagonal included, row-major
    order of the lower-triangle indices), ``upper`` the strict upper triangle of U (ews/params.py:152-163,
    372-391)."""

    def __init__(self, lower: torch.Tensor, upper: torch.Tensor, dim: int, epsilon: float = 0.0):
        super().__init__()
        n = int(dim)
        if lower.numel() != n * (n + 1) // 2 or upper.numel() != n * (n - 1) // 2:
            raise ValueError(f"definite_plus_skew at dim {n} takes {n * (n + 1) // 2} lower and "
                             f"{n * (n - 1) // 2} upper entries")
        self.lower = torch.nn.Parameter(lower)
        self.upper = torch.nn.Parameter(upper)
        self.dim = n
        self.epsilon = float(epsilon)

    def forward(self):
        n = self.dim
        il = torch.tril_indices(n, n, 0, device=self.lower.device)
        iu = torch.triu_indices(n, n, 1, device=self.upper.device)
        Lm = torch.zeros((n, n), dtype=self.lower.dtype, device=self.lower.device).index_put(
            (il[0], il[1]), self.lower)
        Um = torch.zeros((n, n), dtype=self.upper.dtype, device=self.upper.device).index_put(
            (iu[0], iu[1]), self.upper)
        pd = Lm @ Lm.t()
        if self.epsilon > 0.0:
            pd = pd + self.epsilon * torch.eye(n, dtype=pd.dtype, device=pd.device)
        return pd + (Um - Um.t())


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
        A = torch.diag(self.diagonal())
        A._ews_chain = ("real", 1)  # the structure by construction (read without a device-to-host copy)
        return A


class AParamBlockDiag(torch.nn.Module):
    def __init__(self, blocks, sizes):
        super().__init__()
        self.blocks = torch.nn.ParameterList([torch.nn.Parameter(b) for b in blocks])
        self.sizes = [int(s) for s in sizes]
        self.dim = int(sum(self.sizes))

    def forward(self):
        return torch.block_diag(*self.blocks)


class AParamJordanRepeated(torch.nn.Module):
    """Block-diagonal A of Jordan blocks (ews/params.py:412-460): a real block of size n is lambda = softplus(v) on
    the diagonal with ones directly above (:177-187); a complex block of size 2k is R = [[a, -b], [b, a]],
    a = softplus(v), in every diagonal slot with the 2x2 identity above (:190-204). block_params: per block a
    tensor [v] (real) or [v, b] (complex)."""

    def __init__(self, block_sizes, block_kinds, block_params):
        super().__init__()
        self.block_sizes = tuple(int(x) for x in block_sizes)
        self.block_kinds = tuple(str(x) for x in block_kinds)
        for size, kind in zip(self.block_sizes, self.block_kinds):
            if kind not in ("real", "complex"):
                raise ValueError(f"Unknown Jordan block kind '{kind}'")
            if kind == "real" and size < 2:
                raise ValueError(
                    "a real Jordan block needs size >= 2 for the eigenvalue to repeat; "
                    "size 1 is a plain diagonal entry"
                )
            if kind == "complex" and (size % 2 != 0 or size < 4):
                raise ValueError(
                    f"a complex Jordan block needs an even size >= 4, got {size}: a conjugate pair "
                    "already occupies a 2x2 real block, so size 2 is one pair with nothing to chain "
                    "to -- that is `unconstrained_rotation`, not a Jordan block"
                )
        self.block_params = torch.nn.ParameterList([torch.nn.Parameter(torch.as_tensor(p)) for p in block_params])
        self.dim = int(sum(self.block_sizes))
        self._index = {}  # uniform chains: entry indices of A by device

    def _uniform_index(self, device):
        """Index tensors of A's entries for uniform chains (every block the same kind and size): the eigenvalue
        slots, the -b / +b slots of complex blocks, and the constant couplings (ones)."""
        key = str(device)
        if key not in self._index:
            kind, size = self.block_kinds[0], self.block_sizes[0]
            lam_r, lam_c, nb_r, nb_c, pb_r, pb_c, one_r, one_c = [], [], [], [], [], [], [], []
            for j in range(len(self.block_sizes)):
                f = j * size
                if kind == "real":
                    lam_r += [f + i for i in range(size)]
                    lam_c += [f + i for i in range(size)]
                    one_r += [f + i for i in range(size - 1)]
                    one_c += [f + i + 1 for i in range(size - 1)]
                else:
                    for m in range(size // 2):
                        r = f + 2 * m
                        lam_r += [r, r + 1]
                        lam_c += [r, r + 1]
                        nb_r.append(r)
                        nb_c.append(r + 1)
                        pb_r.append(r + 1)
                        pb_c.append(r)
                        if m + 1 < size // 2:
                            one_r += [r, r + 1]
                            one_c += [r + 2, r + 3]
            mk = lambda x: torch.tensor(x, dtype=torch.long, device=device)  # noqa: E731
            self._index[key] = tuple(mk(x) for x in (lam_r, lam_c, nb_r, nb_c, pb_r, pb_c, one_r, one_c))
        return self._index[key]

    def _forward_uniform(self):
        """The same A for uniform chains from a handful of batched operations (one stack of the block parameters,
        one softplus, one scatter), instead of a few per block."""
        kind, size = self.block_kinds[0], self.block_sizes[0]
        P = torch.stack(list(self.block_params))
        lam_r, lam_c, nb_r, nb_c, pb_r, pb_c, one_r, one_c = self._uniform_index(P.device)
        a = F.softplus(P[:, 0]).repeat_interleave(size)  # eigenvalue slots per block (2 per complex coordinate)
        rows, cols, vals = [lam_r], [lam_c], [a]
        if kind == "complex":
            b = P[:, 1].repeat_interleave(size // 2)
            rows += [nb_r, pb_r]
            cols += [nb_c, pb_c]
            vals += [-b, b]
        if one_r.numel():
            rows.append(one_r)
            cols.append(one_c)
            vals.append(torch.ones(one_r.numel(), dtype=P.dtype, device=P.device))
        A = torch.zeros(self.dim, self.dim, dtype=P.dtype, device=P.device)
        return A.index_put((torch.cat(rows), torch.cat(cols)), torch.cat(vals))

    def forward(self):
        if len(set(self.block_sizes)) == 1 and len(set(self.block_kinds)) == 1 and all(
                p.shape == self.block_params[0].shape for p in self.block_params):
            return self._forward_uniform()
        blocks = []
        for size, kind, p in zip(self.block_sizes, self.block_kinds, self.block_params):
            kw = dict(dtype=p.dtype, device=p.device)
            if kind == "real":
                lam = F.softplus(p[0])
                blk = torch.diag(lam.expand(size)) + torch.diag(torch.ones(size - 1, **kw), 1)
            else:
                a, b = F.softplus(p[0]), p[1]
                R = torch.stack([torch.stack([a, -b]), torch.stack([b, a])])
                k = size // 2
                blk = torch.kron(torch.eye(k, **kw), R) + torch.kron(torch.diag(torch.ones(k - 1, **kw), 1),
                                                                     torch.eye(2, **kw))
            blocks.append(blk)
        return torch.block_diag(*blocks)


JORDAN_REAL_SIZES, JORDAN_COMPLEX_SIZES = (2, 3, 4), (4, 6, 8)


def jordan_chains_of(a_param):
    """ews/core/kernels/jordan_engine.py:30-43: (kind, size) when A is AParamJordanRepeated with uniform chains of a
    supported size (real 2-4, complex 4 / 6 / 8), else None."""
    if not isinstance(a_param, AParamJordanRepeated) or not a_param.block_sizes:
        return None
    sizes, kinds = set(a_param.block_sizes), set(a_param.block_kinds)
    if len(sizes) != 1 or len(kinds) != 1:
        return None
    kind, size = kinds.pop(), int(sizes.pop())
    if size not in (JORDAN_REAL_SIZES if kind == "real" else JORDAN_COMPLEX_SIZES):
        return None
    return kind, size


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
    A._ews_chain = ("complex", 2)  # rotation planes by construction (read without a device-to-host copy)
    return A


def block_sizes_of(a_param):
    """Diagonal-block sizes of a parametrisation, from its class (ews/core/kernels/combine.py:37-58)."""
    if isinstance(a_param, AParamBlockDiag):
        return tuple(a_param.sizes)
    if isinstance(a_param, AParamJordanRepeated):
        return tuple(a_param.block_sizes)
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
