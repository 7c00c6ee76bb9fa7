"""Hybrid-precision prefill attention on MI355X: drop-in for
`sage_vertical_attention_v2` (src/ops/sage_unified.py:550-622), the index part
of `reorder_kv_for_vertical` (:499-547) and the vendored `per_block_int8`
(src/ops/vendor/sageattention/triton/quant_per_block.py:49-101).

Every call runs the HIP kernels of libhyq.so on the current HIP stream of
the input's device; there is no CPU or Triton path.  q, k and v are bf16 or
fp16 (one dtype); an fp16 model takes the reference's fp16 branch
(src/ops/sage_unified.py:565-580): the K mean, k - km and the scaled Q are
rounded once to fp16, and the output is fp16.
"""

from __future__ import annotations

import ctypes
import threading
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib
from .decode_d_stage import _require_gpu, _stream

_LOG2_E = 1.44269504          # src/ops/sage_unified.py:22
BLOCK_M = 128                 # query rows per block (src/ops/sage_unified.py:597)
BLOCK_N = 64                  # keys per tile / rest-K scale block
PV_MODES = {"fp16": 0, "fp8": 1}

_ws_lock = threading.Lock()
_ws_cache: dict = {}


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Prefill scratch (per-head fp16 / int8 copies of K and V), cached per
    (device, stream) and grown on demand; calls on one stream are ordered."""
    key = (device.index, stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            _ws_cache.pop(key, None)
            buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
        return buf


def _rows16(t: torch.Tensor) -> torch.Tensor:
    """Channels contiguous and every row 16-byte aligned, else a contiguous copy."""
    es = t.element_size()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all((s * es) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


def _qk_scale(sm_scale: float) -> float:
    """fp32(sm_scale * 1.44269504), the constant the reference hands to its kernels."""
    return float(np.float32(sm_scale * _LOG2_E))


# ---------------------------------------------------------------------------
# per-block int8 quantisation
# ---------------------------------------------------------------------------


def _per_block(x: torch.Tensor, layout: str, sm: float, blk: int, km: Optional[torch.Tensor]):
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError("per_block_int8 expects bf16 or fp16 inputs")
    if layout == "HND":
        b, h, n, d = x.shape
        xs = (x.stride(0), x.stride(1), x.stride(2))
    elif layout == "NHD":
        b, n, h, d = x.shape
        xs = (x.stride(0), x.stride(2), x.stride(1))
    else:
        raise ValueError(f"Unknown tensor layout: {layout}")
    out = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    os_ = (out.stride(0), out.stride(1), out.stride(2)) if layout == "HND" else \
        (out.stride(0), out.stride(2), out.stride(1))
    scale = torch.empty((b, h, (n + blk - 1) // blk), dtype=torch.float32, device=x.device)
    kmp, kms = None, (0, 0)
    if km is not None:
        km = km.to(torch.bfloat16)
        km = km if km.stride(-1) == 1 else km.contiguous()
        kmp = km.data_ptr()
        kms = (km.stride(0), km.stride(1)) if layout == "HND" else (km.stride(0), km.stride(2))
    L = _lib.lib()
    st = L.hyq_per_block_int8(x.data_ptr(), int(x.dtype == torch.float16), *xs, b, h, n, d, float(sm), blk,
                              kmp, *kms, out.data_ptr(), *os_, scale.data_ptr(), scale.stride(0), scale.stride(1),
                              _stream(x.device))
    _lib.check(st, "per_block_int8")
    return out, scale


def per_block_int8(q: torch.Tensor, k: torch.Tensor, km: Optional[torch.Tensor] = None, BLKQ: int = 128,
                   BLKK: int = 64, sm_scale: Optional[float] = None, tensor_layout: str = "HND"):
    """Q int8 per BLKQ rows with sm_scale*log2e folded in, K (minus km) int8
    per BLKK rows; returns (q_int8, q_scale, k_int8, k_scale) as the
    reference (quant_per_block.py:49-101)."""
    _require_gpu(q, "q")
    q = _rows16(q)
    k = _rows16(k)
    head_dim = q.shape[-1]
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    q_int8, q_scale = _per_block(q, tensor_layout, _qk_scale(sm_scale), BLKQ, None)
    k_int8, k_scale = _per_block(k, tensor_layout, 1.0, BLKK, km)
    return q_int8, q_scale, k_int8, k_scale


# ---------------------------------------------------------------------------
# rest / vertical lists
# ---------------------------------------------------------------------------


def vertical_lists(vertical_indices: torch.Tensor, seq_len: int, window_size: int) -> dict:
    """Index part of reorder_kv_for_vertical: per (b, h) the clamped vertical
    indices sorted ascending (`vert` [B*H, T]), the other prefix positions
    ascending (`rest` [B*H, P], first `rcount` valid) and per 128-row query
    block the counts below the window start (`nr`, `nv` [B*H, ceil(N/128)])."""
    _require_gpu(vertical_indices, "vertical_indices")
    B, H, T = vertical_indices.shape
    vidx = vertical_indices.to(torch.int64)
    P = max(0, seq_len - window_size)
    nblk = (seq_len + BLOCK_M - 1) // BLOCK_M
    dev = vidx.device
    out = dict(vert=torch.empty(B * H, T if P else 0, dtype=torch.int32, device=dev),
               rest=torch.empty(B * H, P, dtype=torch.int32, device=dev),
               rcount=torch.empty(B * H, dtype=torch.int32, device=dev),
               nr=torch.empty(B * H, nblk, dtype=torch.int32, device=dev),
               nv=torch.empty(B * H, nblk, dtype=torch.int32, device=dev))
    if P == 0:
        out["rcount"].zero_()
    L = _lib.lib()
    stream = _stream(dev)
    need = L.hyq_prefill_lists_workspace_size(B, H, seq_len, T, window_size)
    ws = _workspace(dev, stream, need) if need else None
    st = L.hyq_prefill_lists(vidx.data_ptr(), vidx.stride(0), vidx.stride(1), vidx.stride(2), B, H,
                             seq_len, T, window_size, out["vert"].data_ptr(), out["rest"].data_ptr(),
                             out["rcount"].data_ptr(), out["nr"].data_ptr(), out["nv"].data_ptr(),
                             None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), stream)
    _lib.check(st, "vertical_lists")
    return out


def reorder_kv_for_vertical(k: torch.Tensor, v: torch.Tensor, vertical_indices: torch.Tensor, window_size: int):
    """Drop-in of reorder_kv_for_vertical (src/ops/sage_unified.py:499-547):
    k, v [BH, N, D] -> (k_rest, v_rest, k_vert, v_vert, n_rest_valid [BH, N],
    n_vert_valid [BH, N], R, V).  Rows whose rest list is shorter than R are
    padded with their last rest row (the reference pads with vertical rows)."""
    BH, N, D = k.shape
    P = max(0, N - window_size)
    if P == 0:
        empty_kv = torch.zeros(BH, 0, D, device=k.device, dtype=k.dtype)
        empty_n = torch.zeros(BH, N, device=k.device, dtype=torch.int32)
        return empty_kv, empty_kv, empty_kv, empty_kv, empty_n, empty_n, 0, 0
    B, H, VLEN = vertical_indices.shape
    lists = vertical_lists(vertical_indices, N, window_size)
    R = int(lists["rcount"].max().item())
    pos = torch.arange(R, device=k.device, dtype=torch.int64)
    last = (lists["rcount"].to(torch.int64) - 1).clamp(min=0)
    ridx = lists["rest"][:, :R].to(torch.int64)
    ridx = torch.where(pos[None, :] < lists["rcount"][:, None], ridx, ridx.gather(1, last[:, None]))
    vidx = lists["vert"].to(torch.int64)
    g = lambda t, i: t.gather(1, i.unsqueeze(-1).expand(-1, -1, D))
    blk = torch.arange(N, device=k.device) // BLOCK_M
    n_rest = lists["nr"][:, blk].contiguous()
    n_vert = lists["nv"][:, blk].contiguous()
    return (g(k, ridx).contiguous(), g(v, ridx).contiguous(), g(k, vidx).contiguous(), g(v, vidx).contiguous(),
            n_rest, n_vert, R, VLEN)


# ---------------------------------------------------------------------------
# hybrid prefill
# ---------------------------------------------------------------------------


def _prefill(entry: str, name: str, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             vertical_indices: Optional[torch.Tensor], window_size: int, sm_scale: Optional[float],
             smooth_k: bool, pv_mode: str) -> torch.Tensor:
    _require_gpu(q, "q")
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"{name} expects q, k, v of one dtype, bf16 or fp16; got {q.dtype}, {k.dtype}, {v.dtype}")
    if pv_mode not in PV_MODES:
        raise ValueError(f"pv_mode must be one of {tuple(PV_MODES)}")
    B, H_q, N, D = q.shape
    _, H_kv, Nk, _ = k.shape
    if Nk != N or v.shape != k.shape or H_q % H_kv:
        raise ValueError(f"{name}: expected k/v [B, H_q / g, N, D] matching q")
    if window_size < 0:
        raise ValueError(f"{name}: window_size must be >= 0")
    if sm_scale is None:
        sm_scale = D ** -0.5
    q, k, v = _rows16(q), _rows16(k), _rows16(v)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    mode = PV_MODES[pv_mode]
    T = 0 if vertical_indices is None else vertical_indices.shape[2]
    L = _lib.lib()
    nbytes = L.hyq_prefill_workspace_size(B, H_q, H_kv, N, T, window_size, mode)
    stream = _stream(q.device)
    ws = _workspace(q.device, stream, nbytes)
    p = _lib.PrefillParams()
    p.q, (p.q_stride_b, p.q_stride_h, p.q_stride_n) = q.data_ptr(), q.stride()[:3]
    p.k, (p.k_stride_b, p.k_stride_h, p.k_stride_n) = k.data_ptr(), k.stride()[:3]
    p.v, (p.v_stride_b, p.v_stride_h, p.v_stride_n) = v.data_ptr(), v.stride()[:3]
    if vertical_indices is not None:
        p.vidx, (p.vi_stride_b, p.vi_stride_h, p.vi_stride_t) = vertical_indices.data_ptr(), vertical_indices.stride()
    p.out, (p.o_stride_b, p.o_stride_h, p.o_stride_n) = out.data_ptr(), out.stride()[:3]
    p.batch, p.hq, p.hkv, p.head_dim = B, H_q, H_kv, D
    p.n, p.t = N, T
    p.window, p.smooth_k, p.pv_mode = window_size, int(bool(smooth_k)), mode
    p.sm_scale = float(sm_scale)
    p.dtype_fp16 = int(q.dtype == torch.float16)
    st = getattr(L, entry)(ctypes.byref(p), ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, name)
    return out


def sage_vertical_attention_v2(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, vertical_indices: torch.Tensor,
                               *, window_size: int = 256, sm_scale: Optional[float] = None, smooth_k: bool = True,
                               pv_mode: str = "fp16") -> torch.Tensor:
    """Hybrid prefill (int8 QK on rest tiles, fp16 QK on vertical / window
    tiles, one online softmax, fp16 P.V).  q [B, H_q, N, D], k/v
    [B, H_kv, N, D] bf16 or fp16 (GQA-native), vertical_indices [B, H_q, T]
    -> [B, H_q, N, D] of q.dtype.  pv_mode "fp8" runs P.V on the rest tiles in OCP e4m3
    with per-channel V scales."""
    _require_gpu(q, "q")
    if vertical_indices.dim() != 3 or vertical_indices.shape[:2] != q.shape[:2]:
        raise ValueError("vertical_indices must be [B, H_q, T]")
    return _prefill("hyq_prefill_hybrid", "sage_vertical_attention_v2", q, k, v, vertical_indices.to(torch.int64),
                    window_size, sm_scale, smooth_k, pv_mode)


def sage_unified_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, window_size: int = 0,
                           sm_scale: Optional[float] = None, smooth_k: bool = True) -> torch.Tensor:
    """Window-only INT8-QK / fp16-PV prefill, the sage_w (window_size > 0) and
    sage_w0 (window_size = 0) modes (src/ops/sage_unified.py:234-313, kernel
    :112-231).  window_size > 0: int8 keys below the 64-aligned window start
    of each 128-row query block, fp16 causal window above it; window_size = 0:
    every key up to the diagonal in int8.  q [B, H_q, N, D], k/v
    [B, H_kv, N, D] bf16 or fp16 -> [B, H_q, N, D] of q.dtype."""
    return _prefill("hyq_prefill_unified", "sage_unified_attention", q, k, v, None, window_size, sm_scale,
                    smooth_k, "fp16")


# The FP8-QK variant (src/ops/sage_unified_fp8.py) needs no optional dtype
# support here: the e4m3 codes are produced and consumed by libhyq.so.
FP8_SUPPORTED = True


def sage_vertical_attention_v2_fp8(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                                   vertical_indices: torch.Tensor, *, window_size: int = 256,
                                   sm_scale: Optional[float] = None, smooth_k: bool = True) -> torch.Tensor:
    """FP8-QK hybrid prefill (src/ops/sage_unified_fp8.py:312-398): the
    partition of sage_vertical_attention_v2 with the rest keys scored in OCP
    e4m3 (Q per 128-row block, rest K per 64-entry block, scale amax / 448),
    fp16 vertical and window tiles and fp16 P.V."""
    _require_gpu(q, "q")
    if vertical_indices.dim() != 3 or vertical_indices.shape[:2] != q.shape[:2]:
        raise ValueError("vertical_indices must be [B, H_q, T]")
    return _prefill("hyq_prefill_hybrid_fp8qk", "sage_vertical_attention_v2_fp8", q, k, v,
                    vertical_indices.to(torch.int64), window_size, sm_scale, smooth_k, "fp16")
