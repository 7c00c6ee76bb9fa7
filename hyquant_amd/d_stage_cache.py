"""The legacy decode format of the reference's `src/ops/d_stage_cache.py`.

Drop-in for its entry points:

- `fused_decode_attention_k4v4` (:504), `splitk_decode_attention_k4v4`
  (:825) and `splitk_decode_attention_k4v4_mma` (:1247) read a quantised
  prefix in the legacy format: uint8 offset-encoded codes (int4: even
  channel in the HIGH nibble, value u - 8; int2: channel 4k+i in bits
  (7-2i, 6-2i), value u - 1.5) with one fp16 scale per (128-token group,
  channel), `[BH_KV, G, D]`.  Nothing in the reference writes this format
  (the D-stage cache stores per-token scales), so these entry points exist
  for callers that build it themselves.
- `d_stage_decode_attention` / `decode_4seg_attention` (:212, :274): the
  per-token format, dequantised to the model dtype first, with one KV head
  per query head and a `[B, H, W, D]` window.

`hyq_decode_legacy` reads the legacy prefix directly (K and V of 4 or 2
bits, as the reference's MMA variant takes them, :977-1092): each tile's
codes and group scales are dequantised in registers to the bf16 values of
`legacy_dequantize`, and the prefix and the three bf16 segments go through
one softmax.  For the per-token format the prefix is dequantised to the
model dtype first (`hyq_dequant`), as the reference's legacy path A does
(:1-8).  The operand roundings are those of the reference's MMA variant: K
and V of the prefix rounded to bf16, P rounded to bf16 for the P.V product,
fp32 accumulation.
`split_size` / `block_kv` are the reference's tuning knobs and do not change
the result; they are accepted and ignored.  The model dtype must be bf16.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib
from .decode_d_stage import (GROUP_SIZE, _decode, _inner_contig, _packed_dim, _require_gpu, _stream,
                             _workspace, dequantize_per_token)

__all__ = [
    "legacy_dequantize",
    "fused_decode_attention_k4v4",
    "splitk_decode_attention_k4v4",
    "splitk_decode_attention_k4v4_mma",
    "d_stage_decode_attention",
    "decode_4seg_attention",
]


def legacy_dequantize(packed: torch.Tensor, scale: torch.Tensor, D: int, nbits: int,
                      out: Optional[torch.Tensor] = None, group: int = GROUP_SIZE) -> torch.Tensor:
    """Legacy-format prefix -> bf16 values: packed uint8 [BH, N, D*nbits/8],
    scale fp16 [BH, ceil(N/group), D] -> bf16 [BH, N, D] =
    bf16((code value) * scale[token // group][channel])
    (src/ops/d_stage_cache.py:1019-1045, :1063-1092).  `out` may be a view
    (for example the first N rows of a larger buffer)."""
    if nbits not in (2, 4):
        raise ValueError(f"legacy format bits must be 2 or 4, got {nbits}")
    _require_gpu(packed, "packed")
    if packed.dim() != 3 or scale.dim() != 3:
        raise ValueError("legacy_dequantize expects packed [BH, N, D_packed] and scale [BH, G, D]")
    BH, N, DP = packed.shape
    if DP != _packed_dim(D, nbits):
        raise ValueError(f"packed rows hold {DP} bytes, expected {_packed_dim(D, nbits)} for D={D}, {nbits} bits")
    if packed.dtype not in (torch.uint8, torch.int8) or scale.dtype != torch.float16:
        raise ValueError("legacy_dequantize expects uint8 packed codes and fp16 scales")
    if scale.shape[0] != BH or scale.shape[2] != D or scale.shape[1] * group < N:
        raise ValueError(f"scale must be [BH, >= ceil(N/{group}), D], got {tuple(scale.shape)}")
    if out is None:
        out = torch.empty(BH, N, D, dtype=torch.bfloat16, device=packed.device)
    elif out.dtype != torch.bfloat16 or tuple(out.shape) != (BH, N, D):
        raise ValueError(f"out must be bf16 [{BH}, {N}, {D}]")
    if BH * N == 0:
        return out
    if packed.stride(-1) != 1:
        packed = packed.contiguous()
    if scale.stride(-1) != 1 or scale.data_ptr() % 16 or any(s % 8 for s in scale.stride()[:2]):
        scale = scale.contiguous()
    st = _lib.lib().hyq_legacy_dequant(packed.data_ptr(), BH, N, D, packed.stride(0), packed.stride(1), nbits,
                                       scale.data_ptr(), scale.stride(0), scale.stride(1), group,
                                       out.data_ptr(), out.stride(0), out.stride(1), _stream(packed.device))
    _lib.check(st, "legacy_dequantize")
    return out


def _nonempty(t: Optional[torch.Tensor]) -> bool:
    return t is not None and t.numel() > 0 and t.shape[1] > 0


def _bf16_rows(BH: int, D: int, like: torch.Tensor) -> torch.Tensor:
    return torch.empty(BH, 0, D, dtype=torch.bfloat16, device=like.device)


def _legacy_decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging, v_staging,
                   k_window, v_window, kv_repeat, k_bits, v_bits, sm_scale, what):
    _require_gpu(q, "q")
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"{what}: q must be [B, H_Q, 1, D], got {tuple(q.shape)}")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"{what}: the legacy decode format takes bf16 models, got {q.dtype}")
    B, H_Q, _, D = q.shape
    assert D % 2 == 0
    if H_Q % kv_repeat:
        raise ValueError(f"{what}: H_Q ({H_Q}) is not a multiple of kv_repeat ({kv_repeat})")
    BH_KV = B * (H_Q // kv_repeat)
    N_q = k_quant_packed.shape[1] if k_quant_packed.numel() > 0 else 0
    if N_q > 0:
        assert k_quant_packed.shape[0] == BH_KV, f"K_packed[0]={k_quant_packed.shape[0]} vs BH_KV={BH_KV} mismatch"
    return _legacy_direct(q, k_quant_packed, v_quant_packed, k_scale, v_scale, N_q, BH_KV,
                          [(k_topk, v_topk), (k_staging, v_staging), (k_window, v_window)],
                          kv_repeat, k_bits, v_bits, sm_scale, what)


def _legacy_direct(q, kp, vp, ks, vs, N_q, BH_KV, segs, kv_repeat, k_bits, v_bits, sm_scale, what):
    """hyq_decode_legacy reads the legacy codes (K and V of 4 or 2 bits) and
    their group scales directly (dequantised in registers to the bf16 values
    of legacy_dequantize) together with the three bf16 segments, one
    softmax."""
    B, H_Q, _, D = q.shape
    L = _lib.lib()
    qf = _inner_contig(q.reshape(B * H_Q, D))
    out = torch.empty(B * H_Q, D, dtype=torch.bfloat16, device=q.device)
    if k_bits not in (2, 4) or v_bits not in (2, 4):
        raise ValueError(f"{what}: k_bits and v_bits must be 2 or 4, got {k_bits}, {v_bits}")
    p = _lib.LegacyParams()
    p.k_bits, p.v_bits = k_bits, v_bits
    p.q, p.q_stride = qf.data_ptr(), qf.stride(0)
    p.out, p.out_stride = out.data_ptr(), out.stride(0)
    keep = [qf]
    if N_q > 0:
        if kp.dtype not in (torch.uint8, torch.int8) or vp.dtype not in (torch.uint8, torch.int8):
            raise ValueError(f"{what}: the packed prefix must be uint8 codes")
        if ks.dtype != torch.float16 or vs.dtype != torch.float16:
            raise ValueError(f"{what}: the prefix scales must be fp16")
        if kp.shape[2] != D * k_bits // 8 or vp.shape[2] != D * v_bits // 8 or vp.shape[:2] != kp.shape[:2]:
            raise ValueError(f"{what}: packed K and V must be [BH_KV, N_q, D * bits / 8] "
                             f"({D * k_bits // 8} and {D * v_bits // 8} bytes)")
        groups = -(-N_q // GROUP_SIZE)
        for name, sc in (("k_scale", ks), ("v_scale", vs)):
            if sc.dim() != 3 or sc.shape[0] != BH_KV or sc.shape[2] != D or sc.shape[1] < groups:
                raise ValueError(f"{what}: {name} must be [{BH_KV}, >= {groups}, {D}], got {tuple(sc.shape)}")
        kp, vp, ks, vs = (_inner_contig(t) for t in (kp, vp, ks, vs))
        keep += [kp, vp, ks, vs]
        p.k_codes, p.kc_stride_bh, p.kc_stride_n = kp.data_ptr(), kp.stride(0), kp.stride(1)
        p.v_codes, p.vc_stride_bh, p.vc_stride_n = vp.data_ptr(), vp.stride(0), vp.stride(1)
        p.k_scale, p.ks_stride_bh, p.ks_stride_g = ks.data_ptr(), ks.stride(0), ks.stride(1)
        p.v_scale, p.vs_stride_bh, p.vs_stride_g = vs.data_ptr(), vs.stride(0), vs.stride(1)
        p.n, p.group = N_q, GROUP_SIZE
    for i, (sk, sv) in enumerate(segs):
        if not _nonempty(sk):
            continue
        if sk.dtype != torch.bfloat16 or sv.dtype != torch.bfloat16 or sk.shape != sv.shape:
            raise ValueError(f"{what}: segment {i} must be bf16 K and V of one shape")
        if sk.shape[0] != BH_KV or sk.shape[2] != D:
            raise ValueError(f"{what}: segment {i} must be [{BH_KV}, n, {D}], got {tuple(sk.shape)}")
        sk, sv = _inner_contig(sk), _inner_contig(sv)
        keep += [sk, sv]
        p.seg_k[i], p.seg_k_stride_bh[i] = sk.data_ptr(), sk.stride(0)
        p.seg_v[i], p.seg_v_stride_bh[i] = sv.data_ptr(), sv.stride(0)
        p.seg_n[i] = sk.shape[1]
    p.bh_kv, p.kv_repeat, p.head_dim = BH_KV, kv_repeat, D
    p.sm_scale = D ** -0.5 if sm_scale is None else float(sm_scale)
    stream = _stream(q.device)
    need = L.hyq_decode_legacy_workspace_size(ctypes.byref(p))
    ws = _workspace(q.device, stream, max(need, 1))
    st = L.hyq_decode_legacy(ctypes.byref(p), ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, what)
    return out.view(B, H_Q, 1, D)


def fused_decode_attention_k4v4(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk,
                                k_staging, v_staging, k_window, v_window, *, kv_repeat: int,
                                sm_scale: Optional[float] = None) -> torch.Tensor:
    """Legacy-format K int4 + V int4 decode (src/ops/d_stage_cache.py:504-591):
    q [B, H_Q, 1, D] bf16, k/v_quant_packed uint8 [BH_KV, N_q, D/2],
    k/v_scale fp16 [BH_KV, G, D], top-k / staging / window bf16 [BH_KV, n, D].
    Returns [B, H_Q, 1, D]."""
    return _legacy_decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging,
                          v_staging, k_window, v_window, kv_repeat, 4, 4, sm_scale, "fused_decode_attention_k4v4")


def splitk_decode_attention_k4v4(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk,
                                 k_staging, v_staging, k_window, v_window, *, kv_repeat: int,
                                 sm_scale: Optional[float] = None, split_size: int = 1024,
                                 block_kv: int = 128) -> torch.Tensor:
    """Split-K variant of fused_decode_attention_k4v4
    (src/ops/d_stage_cache.py:825-951); same operands and result."""
    return _legacy_decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging,
                          v_staging, k_window, v_window, kv_repeat, 4, 4, sm_scale, "splitk_decode_attention_k4v4")


def splitk_decode_attention_k4v4_mma(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk,
                                     k_staging, v_staging, k_window, v_window, *, kv_repeat: int,
                                     k_bits: int = 4, v_bits: int = 4, sm_scale: Optional[float] = None,
                                     split_size: int = 1024, block_kv: int = 128) -> torch.Tensor:
    """GQA-grouped split-K variant with 4- or 2-bit K and V codes
    (src/ops/d_stage_cache.py:1247-1366): packed rows of D/2 (int4) or D/4
    (int2) bytes."""
    assert k_bits in (2, 4), f"k_bits must be 2 or 4, got {k_bits}"
    assert v_bits in (2, 4), f"v_bits must be 2 or 4, got {v_bits}"
    return _legacy_decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging,
                          v_staging, k_window, v_window, kv_repeat, k_bits, v_bits, sm_scale,
                          "splitk_decode_attention_k4v4_mma")


def d_stage_decode_attention(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk,
                             k_staging, v_staging, k_window, v_window, *, v_bits: int = 4,
                             sm_scale: Optional[float] = None) -> torch.Tensor:
    """The reference's legacy path A (src/ops/d_stage_cache.py:212-271): the
    per-token int4 K prefix (and 4- or 2-bit V prefix) of
    quantize_per_token, dequantised to fp16 and cast to the model dtype, then
    four bf16 segments under one softmax.  One KV head per query head:
    q [B, H, 1, D]; prefix / top-k / staging [B*H, n, D]; window [B, H, W, D].
    Returns [B, H, 1, D]."""
    _require_gpu(q, "q")
    if q.dim() != 4 or q.shape[2] != 1:
        raise ValueError(f"d_stage_decode_attention: q must be [B, H, 1, D], got {tuple(q.shape)}")
    if q.dtype != torch.bfloat16:
        raise ValueError(f"d_stage_decode_attention: bf16 models only, got {q.dtype}")
    B, H, _, D = q.shape
    BH = B * H
    N_q = k_quant_packed.shape[1] if k_quant_packed.numel() > 0 else 0
    T = k_topk.shape[1] if _nonempty(k_topk) else 0
    kf = torch.empty(BH, N_q + T, D, dtype=torch.bfloat16, device=q.device)
    vf = torch.empty_like(kf)
    if N_q > 0:
        # dequantize_k_int4_channel(...).to(q.dtype): fp16 values rounded to bf16
        kf[:, :N_q].copy_(dequantize_per_token(k_quant_packed, k_scale, D, 4))
        vf[:, :N_q].copy_(dequantize_per_token(v_quant_packed, v_scale, D, v_bits))
    if T > 0:
        kf[:, N_q:].copy_(k_topk)
        vf[:, N_q:].copy_(v_topk)
    e = _bf16_rows(BH, D, q)
    ks = k_staging if _nonempty(k_staging) else e
    vs = v_staging if _nonempty(v_staging) else e
    kw = k_window.reshape(BH, k_window.shape[2], D)
    vw = v_window.reshape(BH, v_window.shape[2], D)
    none8 = torch.empty(BH, 0, D // 2, dtype=torch.int8, device=q.device)
    none16 = torch.empty(BH, 0, dtype=torch.float16, device=q.device)
    out = _decode(q.reshape(BH, D), none8, none8, none16, none16, kf, vf, ks, vs, kw, vw,
                  4, 4, 1, sm_scale, 0, None, None)
    return out.view(B, H, 1, D)


decode_4seg_attention = d_stage_decode_attention
