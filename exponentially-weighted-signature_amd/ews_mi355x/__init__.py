"""MI355X-native EWS: the reference's EWS / LogEWS layer API over hand-written HIP kernels for gfx950."""

from ._native import LIB_PATH, NativeLibraryError, load  # noqa: F401
from .layer import (  # noqa: F401
    COMBINE_KINDS,
    EWS,
    LEAF_KINDS,
    BToSignature,
    LogEWS,
    log_level_sizes,
    log_level_slices,
    log_signature_dim,
    lyndon_words,
)
from .front import (  # noqa: F401
    B,
    BlockFront,
    Clock,
    ClockSpec,
    FixedClock,
    GatedClock,
    LearnableBlendedClock,
    lift_path,
    make_clock,
)
from .mixer import GradedRMSNorm, MixerEpilogue, graded_level_slices  # noqa: F401
from .block import EWSBlock, RMSNorm, StackedEWS  # noqa: F401
from .ops import diag_scan, mixer_epilogue  # noqa: F401
from .token_scan import build_token_cache, token_cached_prefix_scan  # noqa: F401
from .params import (  # noqa: F401
    AParamBlockDiag,
    AParamBoundedRotation,
    AParamConstant,
    AParamDefinitePlusSkew,
    AParamDampedRotation,
    AParamEFM,
    AParamGeneral,
    AParamJordanRepeated,
    block_sizes_of,
    is_rotation_planes,
    jordan_chains_of,
)

__version__ = "0.1.0"
