"""MI355X-native (gfx950) implementation of HyQuant's hybrid-precision
attention hot path: int4 K4V4 decode cache quantisation, the fused
four-segment split-K decode kernel and the vertical-line selector, exposed
through the C ABI of libhyq.so (include/hyq.h)."""

from .decode_d_stage import (  # noqa: F401
    GROUP_SIZE,
    decode_bf16_full,
    dequantize_per_token,
    fused_d_stage_decode,
    fused_d_stage_decode_splitk,
    quantize_per_token,
)
from .vertical import compute_vertical_indices  # noqa: F401

__all__ = [
    "GROUP_SIZE",
    "quantize_per_token",
    "dequantize_per_token",
    "fused_d_stage_decode",
    "fused_d_stage_decode_splitk",
    "decode_bf16_full",
    "compute_vertical_indices",
]
