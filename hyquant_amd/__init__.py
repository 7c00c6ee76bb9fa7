"""MI355X-native (gfx950) implementation of HyQuant's hybrid-precision
attention hot path: per-token KV quantisation (2/4/8 bits), the fused
four-segment split-K decode, the vertical-line selector, the freeze / flush
of the decode cache and the hybrid INT8-QK prefill, exposed through the C ABI
of libhyq.so (include/hyq.h)."""

from .decode_d_stage import (  # noqa: F401
    GROUP_SIZE,
    decode_bf16_full,
    dequantize_per_token,
    fused_d_stage_decode,
    fused_d_stage_decode_batched,
    fused_d_stage_decode_splitk,
    quantize_per_token,
)
from .sage_unified import (  # noqa: F401
    sage_unified_attention,
    sage_vertical_attention_v2,
    sage_vertical_attention_v2_fp8,
)
from .vertical import compute_vertical_indices  # noqa: F401
from .d_stage_cache import (  # noqa: F401
    d_stage_decode_attention,
    fused_decode_attention_k4v4,
    legacy_dequantize,
    splitk_decode_attention_k4v4,
    splitk_decode_attention_k4v4_mma,
)
from .cache_io import load_cache, save_cache  # noqa: F401

__all__ = [
    "GROUP_SIZE",
    "quantize_per_token",
    "dequantize_per_token",
    "fused_d_stage_decode",
    "fused_d_stage_decode_splitk",
    "fused_d_stage_decode_batched",
    "decode_bf16_full",
    "compute_vertical_indices",
    "sage_vertical_attention_v2",
    "sage_unified_attention",
    "sage_vertical_attention_v2_fp8",
    "save_cache",
    "load_cache",
    "legacy_dequantize",
    "fused_decode_attention_k4v4",
    "splitk_decode_attention_k4v4",
    "splitk_decode_attention_k4v4_mma",
    "d_stage_decode_attention",
]
