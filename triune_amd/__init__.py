"""triune_amd -- MI355X (gfx950) implementation of the reference's gated-linear-attention path.

Host code in Python over a C-ABI library of hand-written HIP kernels (libtriune_hip.so, see
include/triune_hip.h).  Operator surface mirrors triune.ops.gla / triune.kernels.fast_gla.
"""

from .fast_gla import (
    FusedRecurrentScan,
    TriuneHipError,
    fast_chunk_gated_deltanet,
    fast_chunk_gla,
    fast_chunk_gla_varlen,
    fast_recurrent_gated_deltanet,
    gla_decode_step,
)
from .gla import gated_deltanet, gla
from .gla_prep import (fused_qkv_g_prep_chunk_gla, fused_qkv_g_prep_inplace, fused_qkvg_decode_step,
                       fused_qkvg_decode_step_pool)

__all__ = [
    "FusedRecurrentScan",
    "TriuneHipError",
    "fast_chunk_gated_deltanet",
    "fast_chunk_gla",
    "fast_chunk_gla_varlen",
    "fast_recurrent_gated_deltanet",
    "fused_qkv_g_prep_chunk_gla",
    "fused_qkv_g_prep_inplace",
    "fused_qkvg_decode_step",
    "fused_qkvg_decode_step_pool",
    "gated_deltanet",
    "gla",
    "gla_decode_step",
]
