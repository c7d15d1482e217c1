"""The EWS layer and its log-signature variant: the reference's layer API (ews/layer.py) over the HIP library.

``EWS`` / ``LogEWS`` keep the reference's constructor arguments, field names, ``__call__`` signature, shapes,
readouts and error behaviour (ews/layer.py:43-556). Everything between the call and the readout runs in
``libews_mi355x.so`` on the GPU; inputs on the CPU raise instead of falling back.

Engines by generator structure (the structure comes from the parametrisation's class, as in
ews/core/kernels/combine.py:37-63):

    rotation planes, leaf "plane_closed"             fused closed-form leaf + Chen scan (exact, as the reference)
    rotation planes / real diagonal,
        leaf "block_series" or "series"              the same fused kernels with the leaf's order-q series: every
                                                     coefficient is the degree-<= q Taylor polynomial of the closed
                                                     form ("series" at every level, "block_series" at level 2 with
                                                     an exact level 1); exact flows (chen_expm "exact")
    any generator (dense A: d <= 16 at depths    dense kernels (d <= 32: padded 32 x 32 step matrices and
    1-3, 16 < d <= 32 at depths 1-2)              states, matrix functions per interval or per sample)
        leaf "series"                                dense kernels: series leaf of order series_q
        leaf "van_loan" (the reference default)      dense kernels: Van Loan leaf with M knots per interval under
                                                     van_loan_expm and reweighting_mode
        (also planes / diagonals at depth 3, or      flows M_t of chen_expm evaluated in the kernels, MFMA Chen
        with chen_expm other than "exact")           mode products
    Jordan chains, leaf "jordan_closed(_tables)";    the chains' closed-form local terms at any step (float64
    planes, "plane_closed" with approximate flows    tables on the device), flows of chen_expm (exact for
                                                     jordan_flows), the dense combine (d <= 16, at most 8 chains)
    block-diagonal A, leaf "block_series"            dense kernels: the exact level 1 phi(-h A) v at any step
                                                     (scaled Taylor and doublings), the order-series_q series at
                                                     level 2, flows of chen_expm
    anything else                                    NotImplementedError
"""

from __future__ import annotations

from typing import Optional

import torch

from . import ops
from .params import AParamConstant, block_sizes_of, diagonal_structure, is_rotation_planes, jordan_chains_of

LEAF_KINDS = ("van_loan", "series", "plane_closed", "block_series", "jordan_closed", "jordan_closed_tables")
COMBINE_KINDS = ("assoc", "lean", "block_kernel", "dense_kernel")
JORDAN_LEAVES = ("jordan_closed", "jordan_closed_tables")


def _normalize_expm_method(method: str) -> str:
    """ews/layer.py:34-40."""
    method = method.lower()
    if method in {"pade_lite", "pade-lite"}:
        return "pade"
    if method not in {"exact", "euler", "cayley", "pade"}:
        raise ValueError("expm method must be one of 'exact', 'euler', 'cayley', 'pade'")
    return method


class EWS(torch.nn.Module):
    """EWS layer (ews/layer.py:43-307): (path, clock) -> exponentially weighted signature features."""

    def __init__(
        self,
        A,
        N: int,
        M: int = 20,
        dtype: torch.dtype = torch.float32,
        reweighting_mode: str = "displacement",
        terminal_reduce: str = "tree",
        van_loan_expm: str = "cayley",
        chen_expm: str = "exact",
        leaf: str = "van_loan",
        series_q: Optional[int] = None,
        combine: str = "assoc",
        combine_chunk: int = 1024,
        combine_tile: int = 4,
        jordan_flows: bool = False,
    ):
        super().__init__()
        if isinstance(A, torch.Tensor):
            A_param = AParamConstant(A.to(dtype))
        else:
            A_param = A
        self.A_param = A_param
        self.d = int(A_param.dim) if hasattr(A_param, "dim") else int(A_param().shape[0])
        self.N = N
        self.M = M
        self.dtype = dtype
        self.reweighting_mode = reweighting_mode
        if terminal_reduce not in {"tree", "assoc"}:
            raise ValueError("terminal_reduce must be 'tree' or 'assoc'")
        self.terminal_reduce = terminal_reduce
        self.van_loan_expm = _normalize_expm_method(van_loan_expm)
        self.chen_expm = _normalize_expm_method(chen_expm)
        if leaf not in LEAF_KINDS:
            raise ValueError(f"leaf must be one of {LEAF_KINDS}, got {leaf!r}")
        if leaf == "series" and series_q is None:
            raise ValueError("leaf='series' requires series_q (see ews.core.leaf.check_series_q)")
        self.leaf = leaf
        self.series_q = None if series_q is None else int(series_q)
        if combine not in COMBINE_KINDS:
            raise ValueError(f"combine must be one of {COMBINE_KINDS}, got {combine!r}")
        self.combine = combine
        self.combine_chunk = int(combine_chunk)
        self.combine_tile = int(combine_tile)
        self.block_sizes = block_sizes_of(A_param)
        if combine == "block_kernel" and self.block_sizes is None:
            raise ValueError(
                "combine='block_kernel' needs a block-diagonal A parametrisation "
                "(rotation planes, AParamUnconstrainedRotation, AParamJordanRepeated or AParamBlockDiag)"
            )
        self.jordan_flows = bool(jordan_flows)
        if self.jordan_flows and (combine != "block_kernel" or jordan_chains_of(A_param) is None):
            raise ValueError("jordan_flows needs combine='block_kernel' and a jordan_repeated A with uniform chains")
        if leaf == "block_series" and self.block_sizes is None:
            raise ValueError("leaf='block_series' needs a block-diagonal A parametrisation")
        if leaf == "plane_closed" and not is_rotation_planes(A_param):
            raise ValueError(
                "leaf='plane_closed' needs a rotation-plane A parametrisation "
                "(bounded/damped/relu_damped/clamped/unbounded rotation)"
            )
        if leaf == "block_series" and N == 2 and series_q is None:
            raise ValueError("leaf='block_series' at depth 2 requires series_q")
        if leaf in JORDAN_LEAVES and jordan_chains_of(A_param) is None:
            raise ValueError(
                f"leaf={leaf!r} needs a jordan_repeated A with uniform chains (every block the same kind and size: "
                "real 2-4 or complex 4, 6, 8)"
            )
        self.structure = diagonal_structure(A_param)

    # ------------------------------------------------------------------------------------------ engine
    def _flow_mode(self, readout):
        if self.leaf == "van_loan" and self.reweighting_mode not in (
            "displacement", "displacement_uniform", "displacement_uniform_basepoint"
        ):
            raise ValueError(
                "reweighting_mode must be 'displacement', 'displacement_uniform', or "
                f"'displacement_uniform_basepoint', got {self.reweighting_mode}"
            )
        # the assoc combine's tree terminal always takes per-interval flows (ews/core/chen_scan.py:286-298)
        if readout == "terminal" and self.combine == "assoc" and self.terminal_reduce == "tree":
            return "per_interval"
        if self.reweighting_mode == "displacement_uniform":
            return "cached"
        if self.reweighting_mode == "displacement_uniform_basepoint":
            return "cached_basepoint"
        return "per_interval"

    def _diag_params(self, A):
        """Kernel parameters read off the materialised A as ews/core/leaf.py:130-131 reads them."""
        if self.structure == "planes":
            ii = torch.arange(0, self.d, 2, device=A.device)
            return torch.stack([A[ii, ii], A[ii, ii + 1]], -1).contiguous()
        return torch.diagonal(A).contiguous()

    def _chain_form(self):
        """(kind, size, series_q, leaf step mode) when the depth-1 chain kernels take this layer, else None: a
        generator of uniform Jordan chains (any number) under exact flows (jordan_flows or chen_expm "exact"),
        and rotation planes / real diagonals wider than the dense kernels with the van_loan leaf. The leaf's level
        1 is then phi(-hA) v exactly (jordan_closed, block_series, plane_closed, van_loan with an exact
        van_loan_expm) or its order-q truncation (series)."""
        if self.N != 1 or not (self.jordan_flows or self.chen_expm == "exact"):
            return None
        chains = jordan_chains_of(self.A_param)
        if chains is None:
            if self.structure is None or self.leaf != "van_loan" or self.d <= 16:
                return None
            chains = ("complex", 2) if self.structure == "planes" else ("real", 1)
        if self.leaf == "van_loan":
            if self.van_loan_expm != "exact":
                return None
            step = {"displacement": "per_interval", "displacement_uniform": "cached",
                    "displacement_uniform_basepoint": "cached_basepoint"}.get(self.reweighting_mode)
            return None if step is None else (chains[0], chains[1], 0, step)
        if self.leaf == "series":
            if not 1 <= int(self.series_q or 0) <= 48:
                return None
            return (chains[0], chains[1], int(self.series_q), "per_interval")
        if self.leaf in JORDAN_LEAVES or self.leaf in ("block_series", "plane_closed"):
            return (chains[0], chains[1], 0, "per_interval")
        return None

    def _engine_check(self):
        if self._chain_form() is not None:
            return "chain"
        if self.leaf in JORDAN_LEAVES or (self.leaf == "block_series" and self.structure is None):
            if self.N > 2:
                raise NotImplementedError(f"leaf={self.leaf!r}: closed-form local terms exist for depths 1 and 2")
            if self.d > 16:
                raise NotImplementedError(f"leaf={self.leaf!r} runs on the dense kernels here: d <= 16")
            return "dense"
        diag_ok = self.structure is not None and self.leaf in ("plane_closed", "block_series", "series") and self.N <= 2
        if diag_ok and self.chen_expm == "exact":
            if self.structure == "planes" and self.d % 2:
                raise ValueError("leaf='plane_closed' needs an even dimension (2x2 planes)")
            return "diag"
        if self.leaf in ("series", "van_loan"):
            if self.N > 3 or self.d > 32 or (self.d > 16 and self.N > 2):
                raise NotImplementedError(
                    f"leaf={self.leaf!r}: the dense-generator kernels cover depths 1-3 at d <= 16 and depths 1-2 at "
                    "d <= 32")
            return "dense"
        if diag_ok and self.d <= 16:
            return "dense"  # closed-form leaf with approximate flows: exact integrals on the dense kernels
        if diag_ok:
            raise NotImplementedError(
                f"leaf={self.leaf!r}: the closed-form kernels take exact flows exp(-h A) (chen_expm='exact'), "
                f"got chen_expm={self.chen_expm!r}"
            )
        if self.structure is not None and self.N > 2:
            raise NotImplementedError(
                f"leaf={self.leaf!r}: closed-form local terms exist for depths 1 and 2 (use leaf='series' at depth 3)"
            )
        raise NotImplementedError(
            f"no MI355X kernel for leaf={self.leaf!r} with a dense generator in this build: use leaf='series' "
            "(any generator, depths 1-3) or a rotation-plane / diagonal parametrisation with leaf='plane_closed'"
        )

    def _keep_dense(self):
        """The dense forward keeps its backward workspace only in training mode with grad mode on (and unless
        EWS_DENSE_KEEP=0): an evaluation pass that still records a graph does not hold it."""
        return None if self.training else False

    def _run(self, path, clock, readout, level0, a_scale):
        engine = self._engine_check()
        if self.dtype != torch.float32:
            raise TypeError("the MI355X kernels compute in float32 (dtype=torch.float32)")
        A = self.A_param().to(torch.float32) * torch.as_tensor(a_scale, dtype=torch.float32, device=path.device)
        if engine == "chain":
            kind, size, q, step = self._chain_form()
            kr = readout if readout in ("prefix", "terminal") else "prefix"
            out = ops.chain_scan(path.to(torch.float32), clock.to(torch.float32), A.to(path.device).contiguous(),
                                 kind, size, self._flow_mode(readout), step, kr, level0, q)
            if readout == "mean":
                return out.mean(1)
            if readout == "max":
                return out.max(1).values
            return out
        if engine == "dense":
            chen = "exact" if self.jordan_flows else self.chen_expm  # closed-form chain flows are exact
            if self.leaf in JORDAN_LEAVES or (self.leaf == "plane_closed" and self.structure == "planes"):
                # the chains' closed-form local terms at any step (a rotation plane is a complex chain of one
                # coordinate), the flows of chen_expm, the dense combine
                kind, size = jordan_chains_of(self.A_param) if self.leaf in JORDAN_LEAVES else ("complex", 2)
                return ops.jordan_scan(path.to(torch.float32), clock.to(torch.float32),
                                       A.to(path.device).contiguous(), self.N, kind, size, self._flow_mode(readout),
                                       readout, level0, chen_expm=chen)
            if self.leaf == "block_series":
                # the block-series leaf (general blocks, or planes / diagonals under approximate flows): the exact
                # level 1 G v at any step and the blockwise order-series_q series at level 2, as the reference
                # computes them (ews/core/leaf.py:138-175, blockdiag_engine.py:88-155)
                leaf = ops.DenseLeaf("block_series", q=self.series_q or 0, chen_expm=chen)
                return ops.dense_scan(path.to(torch.float32), clock.to(torch.float32),
                                      A.to(path.device).contiguous(), self.N, leaf.q, self._flow_mode(readout),
                                      readout, level0, leaf=leaf, keep=self._keep_dense())
            if self.leaf == "van_loan":
                leaf = ops.DenseLeaf("van_loan", M=self.M, van_loan_expm=self.van_loan_expm,
                                     reweighting_mode=self.reweighting_mode, chen_expm=chen)
            else:
                leaf = ops.DenseLeaf("series", q=self.series_q, chen_expm=chen)
            return ops.dense_scan(path.to(torch.float32), clock.to(torch.float32), A.to(path.device).contiguous(),
                                  self.N, leaf.q, self._flow_mode(readout), readout, level0, leaf=leaf,
                                  keep=self._keep_dense())
        params = self._diag_params(A.to(path.device))
        if path.dtype != torch.bfloat16:
            path = path.to(torch.float32)
        clock = clock.to(torch.float32)
        leaf = self.leaf if self.leaf in ("series", "block_series") else "plane_closed"
        return ops.diag_scan(path, clock, params, self.N, self.structure, self._flow_mode(readout), readout,
                             level0, chunk=0, leaf=leaf, series_q=self.series_q or 0)

    def _log_prefix_fused(self, path, clock):
        """LogEWS prefix rows computed inside the scan (rotation planes or a real diagonal, depth 2, the diagonal
        leaves with exact flows): the compressed log of every prefix row (ews/layer.py:488-517), written by the
        scan's output pass without the flat rows ever reaching memory. None when the configuration takes the
        rows-then-log route (the dense kernels)."""
        if self.structure is None or self.N != 2 or path.dim() != 3:
            return None
        if self._engine_check() != "diag":
            return None
        if self.dtype != torch.float32:
            raise TypeError("the MI355X kernels compute in float32 (dtype=torch.float32)")
        A = self.A_param().to(torch.float32)
        params = self._diag_params(A.to(path.device))
        if path.dtype != torch.bfloat16:
            path = path.to(torch.float32)
        leaf = self.leaf if self.leaf in ("series", "block_series") else "plane_closed"
        return ops.diag_scan(path, clock.to(torch.float32), params, self.N, self.structure,
                             self._flow_mode("prefix"), "log_prefix", False, chunk=0, leaf=leaf,
                             series_q=self.series_q or 0)

    def mixed_prefix(self, path, clock, mixer, a_scale=1.0):
        """The prefix rows (level 0 included) straight into ``mixer`` (a MixerEpilogue over this layer's width and
        depth) inside the scan's output pass (ops.scan_mixer): the D-wide rows never reach memory. Applies to rotation
        planes / real diagonals with exact flows that run on the chunk kernels, depth 1-2 and c_down at most 64 wide;
        None elsewhere (the caller composes the scan and the mixer)."""
        if self.structure is None or self.N not in (1, 2) or path.dim() != 3 or self.dtype != torch.float32:
            return None
        if mixer.d != self.d or mixer.N != self.N or mixer.hidden_dim > 64 or self._engine_check() != "diag":
            return None
        self._check_batch(path, clock)
        A = self.A_param().to(torch.float32) * torch.as_tensor(a_scale, dtype=torch.float32, device=path.device)
        params = self._diag_params(A.to(path.device))
        if path.dtype != torch.bfloat16:
            path = path.to(torch.float32)
        leaf = self.leaf if self.leaf in ("series", "block_series") else "plane_closed"
        return ops.scan_mixer(path, clock.to(torch.float32), params, mixer.c_down.weight, mixer.c_down.bias,
                              mixer.graded.gain_tensor(), self.N, self.structure, self._flow_mode("prefix"), leaf,
                              self.series_q or 0, mixer.graded.variant, mixer.graded.eps, not mixer.basepoint,
                              mixer.graded_prescale == "binomial")

    def _levels(self, packed, lead):
        out, s = [], 0
        for k in range(1, self.N + 1):
            n = self.d**k
            out.append(packed[..., s : s + n].reshape(lead + (self.d,) * k))
            s += n
        return out

    # ------------------------------------------------------------------------------------------ call
    def forward(
        self,
        path: torch.Tensor,
        clock: torch.Tensor,
        return_terminal: bool = True,
        output_format: str = "flat",
        readout: Optional[str] = None,
        a_scale=1.0,
    ):
        """path (L, d) or (B, L, d); clock (L,) or (B, L). Readouts as ews/layer.py:267-302."""
        if readout is None:
            readout = "terminal" if return_terminal else "prefix"
        if readout not in {"terminal", "prefix", "mean", "max"}:
            raise ValueError("readout must be 'terminal', 'prefix', 'mean', or 'max'")
        if path.dim() == 2:
            if clock.dim() != 1 or clock.shape[0] != path.shape[0]:
                raise ValueError("clock must be 1D and aligned with path length")
            out = self.forward(path[None], clock[None], output_format=output_format, readout=readout,
                               a_scale=a_scale)
            return [o[0] for o in out] if isinstance(out, list) else out[0]
        self._check_batch(path, clock)
        if output_format == "list":
            if readout in ("mean", "max"):
                raise ValueError(f"readout='{readout}' requires output_format='flat'")
            packed = self._run(path, clock, readout, False, a_scale)
            return self._levels(packed, tuple(packed.shape[:-1]))
        return self._run(path, clock, readout, True, a_scale)

    @staticmethod
    def _check_batch(path, clock):
        if path.dim() != 3:
            raise ValueError(f"Path must be 2D or 3D, got shape {tuple(path.shape)}")
        if clock.dim() != 2:
            raise ValueError("clock must be 2D for batched paths")
        if clock.shape[1] != path.shape[1] or clock.shape[0] != path.shape[0]:
            raise ValueError("clock must be 1D and aligned with path length")

    @property
    def signature_dim(self) -> int:
        return sum(self.d**k for k in range(1, self.N + 1))


# ---------------------------------------------------------------------------------------------- log-signature
def lyndon_words(N, d):
    """Lyndon words of lengths 1..N over {0..d-1}, each length in lexicographic order (Duval)."""
    words = [[] for _ in range(N)]
    w = [-1]
    while w:
        w[-1] += 1
        words[len(w) - 1].append(tuple(w))
        m = len(w)
        while len(w) < N:
            w.append(w[len(w) - m])
        while w and w[-1] == d - 1:
            w.pop()
    return [sorted(ws) for ws in words]


def log_level_sizes(d: int, N: int):
    """[W_d(1), .., W_d(N)] (ews/layer.py:417-420)."""
    return [len(w) for w in lyndon_words(N, d)]


def log_signature_dim(d: int, N: int) -> int:
    """ews/layer.py:423-425."""
    return int(sum(log_level_sizes(d, N)))


def log_level_slices(d: int, N: int):
    """ews/layer.py:428-437."""
    slices, start = [], 0
    for size in log_level_sizes(d, N):
        slices.append((start, start + size))
        start += size
    return tuple(slices)


class LogEWS(torch.nn.Module):
    """log(EWS) in the compressed Lyndon basis (ews/layer.py:440-556)."""

    def __init__(self, A, N: int, M: int = 20, dtype=torch.float32, reweighting_mode="displacement",
                 terminal_reduce="tree", van_loan_expm="cayley", chen_expm="exact", leaf="van_loan",
                 series_q=None, combine="assoc", combine_chunk=1024, combine_tile=4, jordan_flows=False):
        super().__init__()
        self.ewms = EWS(A, N=N, M=M, dtype=dtype, reweighting_mode=reweighting_mode,
                        terminal_reduce=terminal_reduce, van_loan_expm=van_loan_expm, chen_expm=chen_expm,
                        leaf=leaf, series_q=series_q, combine=combine, combine_chunk=combine_chunk,
                        combine_tile=combine_tile, jordan_flows=jordan_flows)
        self.d = self.ewms.d
        self.N = self.ewms.N

    def forward(self, path, clock, return_terminal=True, output_format="flat", readout=None):
        """log-then-pool (ews/layer.py:488-517): the EWS rows, then ews_log_forward (log, Lyndon coefficients,
        readout) on the GPU."""
        if readout is None:
            readout = "terminal" if return_terminal else "prefix"
        if readout not in {"terminal", "prefix", "mean", "max"}:
            raise ValueError("readout must be 'terminal', 'prefix', 'mean', or 'max'")
        if path.dim() not in (2, 3):
            raise ValueError(f"Path must be 2D or 3D, got shape {tuple(path.shape)}")
        if path.dim() == 3 and clock.dim() != 2:
            raise ValueError("clock must be 2D for batched paths")
        if output_format == "list" and readout in ("mean", "max"):
            raise ValueError(f"readout='{readout}' requires output_format='flat'")
        single = path.dim() == 2
        if single:
            path, clock = path[None], clock[None]
        feat = None
        if readout == "prefix":
            self.ewms._check_batch(path, clock)
            feat = self.ewms._log_prefix_fused(path, clock)  # the log rows written by the scan itself
        if feat is None:
            if readout == "terminal":
                rows = self.ewms(path, clock, readout="terminal", output_format="flat")[:, None, :]
            else:
                rows = self.ewms(path, clock, readout="prefix", output_format="flat")
            feat = ops.log_rows(rows, self.d, self.N, True, readout)
        if single:
            feat = feat[0]
        if output_format == "list":
            return self._split(feat)
        return feat

    def _split(self, feat):
        return [feat[..., s:e] for s, e in log_level_slices(self.d, self.N)]

    @property
    def log_signature_dim(self) -> int:
        return log_signature_dim(self.d, self.N)


class BToSignature(torch.nn.Module):
    """Optional lift B + EWS (ews/layer.py:310-341)."""

    def __init__(self, b, ewms: EWS):
        super().__init__()
        self.b = b
        self.ewms = ewms

    def forward(self, path, clock, return_terminal=True, output_format="flat", readout=None):
        if self.b is not None:
            path = self.b(path)
        return self.ewms(path, clock, return_terminal=return_terminal, output_format=output_format,
                         readout=readout)
