"""CPU oracle for HyQuant's hybrid-precision attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the `hyquant_amd` product path may import,
call or link this module: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker.

Every function restates the reference's algorithm from its source (cited as
`path:line` relative to the HyQuant repository root) in numpy / torch-CPU code
written for this repository.  Arrays holding "bf16" data are float32 arrays
whose values are exactly representable in bfloat16.

Parity pins (the tests under tests/ that check this oracle independently of
its own formulas):
  quantize_per_token / pack / unpack  -> hand-computed known answers, nibble
      layout vectors, round-half-even ties, subnormal and overflow scales,
      round-trip and |x - deq(x)| <= scale/2 invariants.
  compute_vertical_indices            -> brute-force full sort on tiny inputs,
      planted-line known answer, rho=1 selects everything, tie rule vectors,
      exact-dot cross-check against Python integer/fraction arithmetic.
  freeze                              -> partition invariants (topk U compact =
      prefix, disjoint, compact ascending), window = last W, brute force.
  decode_fp64                         -> closed forms: N_q = 0 reduces to plain
      softmax attention (checked against torch fp64 SDPA), segment permutation
      invariance, GQA equals explicit head expansion, single-token softmax = v.
  decode_bf16_eager                   -> same inputs agree with decode_fp64 to
      bf16 precision.
  e4m3_round                          -> torch.float8_e4m3fn on every in-range
      grid point and tie, hand known answers (ties to even, subnormals,
      saturation at 448).
  hybrid_prefill_fp64(pv_mode='fp8')  -> with V, P exactly representable in
      e4m3 (powers of two) it equals the fp16 mode; per-channel V scale
      invariance; fp8 error against exact attention within the e4m3 bound.
  legacy_unpack / legacy_values       -> hand-decoded bytes (nibble and crumb
      order, offsets 8 and 1.5), every byte value against per-bit Python
      arithmetic, group boundaries of the [G, D] scales.
  legacy_decode_fp64                  -> with unit scales and no bf16 segments
      it equals decode_fp64 over the same values re-expressed per token.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

GROUP_SIZE = 128          # staging ring size; src/ops/decode_d_stage.py:19
LOG2E = 1.44269504        # src/ops/decode_d_stage.py:17

# ---------------------------------------------------------------------------
# bfloat16 helpers (exact bit manipulation, round-to-nearest-even)
# ---------------------------------------------------------------------------


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 -> bfloat16 bits with round-to-nearest-even (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint32)
    nan = np.isnan(x)
    if nan.any():
        rounded = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> nearest bfloat16 value (returned as float32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(x, dtype=np.float32)))


def f64_to_f32_round_odd(x: np.ndarray) -> np.ndarray:
    """float64 -> float32 with round-to-odd (sticky), so a following RNE to a
    narrower format equals one correct rounding of the float64 value."""
    x = np.asarray(x, dtype=np.float64)
    f = x.astype(np.float32)
    fd = f.astype(np.float64)
    # step toward zero where RNE rounded away from zero
    over = np.abs(fd) > np.abs(x)
    f = np.where(over, np.nextafter(f, np.float32(0)), f)
    inexact = f.astype(np.float64) != x
    bits = f.view(np.uint32).copy()
    bits[inexact] |= np.uint32(1)
    return bits.view(np.float32)


def bf16_round_f64(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest bfloat16 (single correct RNE rounding)."""
    return bf16_round(f64_to_f32_round_odd(x))


# ---------------------------------------------------------------------------
# a1/a2: per-token symmetric quantisation, int4 packing
# src/ops/decode_d_stage.py:50-77 (quantize_per_token), :80-101 (dequantize),
# :104-111 (_pack_int4), :114-123 (_unpack_int4), :126-149 (int2)
# ---------------------------------------------------------------------------


def quantize_codes(x: np.ndarray, nbits: int) -> Tuple[np.ndarray, np.ndarray]:
    """x [..., D] (bf16 values) -> (codes int8 [..., D], scale float16 [...]).

    scale = fp16(max(amax, 1e-5) / q_max) computed in fp32, codes =
    clamp(round_half_even(x / fp32(scale)), q_min, q_max)
    (src/ops/decode_d_stage.py:61-68).
    """
    if nbits not in (2, 4, 8):
        raise ValueError(f"nbits must be 2, 4, or 8, got {nbits}")
    q_max = 2 ** (nbits - 1) - 1
    q_min = -(2 ** (nbits - 1))
    xf = np.asarray(x, dtype=np.float32)
    amax = np.abs(xf).max(axis=-1)
    amax = np.maximum(amax, np.float32(1e-5))
    with np.errstate(over="ignore"):
        scale = (amax / np.float32(q_max)).astype(np.float32).astype(np.float16)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(xf / scale.astype(np.float32)[..., None])
    codes = np.clip(r, q_min, q_max).astype(np.int8)
    return codes, scale


def pack_int4(codes: np.ndarray) -> np.ndarray:
    """[..., D] int8 in [-8,7] -> [..., D/2] int8: even channel in the low
    nibble, odd channel in the high nibble (src/ops/decode_d_stage.py:104-111)."""
    u = codes.astype(np.int16) & 0x0F
    return (u[..., 0::2] | (u[..., 1::2] << 4)).astype(np.uint8).view(np.int8)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """Inverse of pack_int4 with sign extension (src/ops/decode_d_stage.py:114-123)."""
    x = packed.view(np.uint8).astype(np.int32)
    lo = ((x & 0x0F) ^ 8) - 8
    hi = (((x >> 4) & 0x0F) ^ 8) - 8
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.int8)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out


def pack_int2(codes: np.ndarray) -> np.ndarray:
    """Channels 4i..4i+3 in bits [1:0],[3:2],[5:4],[7:6] (src/ops/decode_d_stage.py:126-133)."""
    u = codes.astype(np.int16) & 0x03
    return (u[..., 0::4] | (u[..., 1::4] << 2) | (u[..., 2::4] << 4) | (u[..., 3::4] << 6)).astype(np.uint8).view(np.int8)


def unpack_int2(packed: np.ndarray) -> np.ndarray:
    x = packed.view(np.uint8).astype(np.int32)
    out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 4,), dtype=np.int8)
    for j in range(4):
        out[..., j::4] = (((x >> (2 * j)) & 0x03) ^ 2) - 2
    return out


def quantize_per_token(x: np.ndarray, nbits: int) -> Tuple[np.ndarray, np.ndarray]:
    """[BH, N, D] -> (packed int8 [BH, N, D*nbits/8], scale fp16 [BH, N])."""
    codes, scale = quantize_codes(x, nbits)
    if nbits == 8:
        return codes, scale
    if nbits == 4:
        return pack_int4(codes), scale
    return pack_int2(codes), scale


def unpack_codes(packed: np.ndarray, nbits: int) -> np.ndarray:
    if nbits == 8:
        return packed.astype(np.int8)
    if nbits == 4:
        return unpack_int4(packed)
    if nbits == 2:
        return unpack_int2(packed)
    raise ValueError(f"nbits must be 2, 4, or 8, got {nbits}")


def dequantize_per_token(packed: np.ndarray, scale: np.ndarray, nbits: int) -> np.ndarray:
    """fp16(code * scale) as the reference's eager path does
    (src/ops/decode_d_stage.py:80-101); returned as float32 holding fp16 values."""
    q = unpack_codes(packed, nbits).astype(np.float32)
    return (q * scale.astype(np.float32)[..., None]).astype(np.float16).astype(np.float32)


# ---------------------------------------------------------------------------
# a4: vertical-line selector, src/patch/_common.py:144-190
# ---------------------------------------------------------------------------


def top_k_count(prefix_len: int, top_ratio: float) -> int:
    """top_k = min(max(1, ceil(P * rho)), P) (src/patch/_common.py:187-188)."""
    t = max(1, int(math.ceil(prefix_len * top_ratio)))
    return min(t, prefix_len)


def f16_round_f64(x: np.ndarray) -> np.ndarray:
    """float64 -> nearest fp16 value (single correct RNE rounding), as float32."""
    return f64_to_f32_round_odd(x).astype(np.float16).astype(np.float32)


def mean_f16(x: np.ndarray, axis: int) -> np.ndarray:
    """fp16 mean, as mean_bf16 with one RNE rounding to fp16."""
    n = x.shape[axis]
    s = np.asarray(x, dtype=np.float64).sum(axis=axis)
    return f16_round_f64(s / np.float64(n))


def mean_bf16(x: np.ndarray, axis: int) -> np.ndarray:
    """bf16 mean: exact float64 sum, one float64 division, one RNE rounding to
    bf16.  Equals torch's fp32-accumulated bf16 mean except where the fp32 sum
    is inexact right at a bf16 rounding boundary."""
    n = x.shape[axis]
    s = np.asarray(x, dtype=np.float64).sum(axis=axis)
    return bf16_round_f64(s / np.float64(n))


def mean_half(x: np.ndarray, axis: int, fp16: bool = False) -> np.ndarray:
    """The model dtype's mean: mean_f16 for an fp16 model, else mean_bf16."""
    return mean_f16(x, axis) if fp16 else mean_bf16(x, axis)


def dot_bf16_exact(qm: np.ndarray, k: np.ndarray, fp16: bool = False) -> np.ndarray:
    """scores[..., p] = bf16(sum_d qm[..., d] * k[..., p, d]) with the sum taken
    sequentially in d order in float64 (products of bf16 values are exact in
    float64; the running sum is exact unless the products span > 2^37 in
    magnitude).  fp16=True (fp16 operands, products exact in float64 too):
    the sum is rounded to fp16 instead.  qm [..., D], k [..., P, D] -> [..., P]."""
    qm64 = np.asarray(qm, dtype=np.float64)
    k64 = np.asarray(k, dtype=np.float64)
    acc = np.zeros(k64.shape[:-1], dtype=np.float64)
    for d in range(k64.shape[-1]):
        acc = acc + qm64[..., d, None] * k64[..., d]
    return f16_round_f64(acc) if fp16 else bf16_round_f64(acc)


def orderable_bf16_key(scores_bf16: np.ndarray, fp16: bool = False) -> np.ndarray:
    """Monotone uint16 key of a bf16 value (fp16 when fp16=True: the same
    sign / biased-exponent layout); -0 and +0 get the same key (torch
    compares them equal)."""
    if fp16:
        b = np.asarray(scores_bf16, np.float32).astype(np.float16).view(np.uint16).astype(np.uint32)
    else:
        b = f32_to_bf16_bits(scores_bf16).astype(np.uint32)
    b = np.where(b == 0x8000, 0, b)
    neg = (b & 0x8000) != 0
    return np.where(neg, (~b) & 0xFFFF, b | 0x8000).astype(np.uint32)


def topk_desc_index_asc(scores_bf16: np.ndarray, k: int, fp16: bool = False) -> np.ndarray:
    """Top-k along the last axis ordered by score descending, ties broken by
    lower index first (the deterministic rule this build adopts for
    torch.topk(sorted=True), src/patch/_common.py:189)."""
    key = orderable_bf16_key(scores_bf16, fp16).astype(np.int64)
    P = scores_bf16.shape[-1]
    idx = np.broadcast_to(np.arange(P, dtype=np.int64), key.shape)
    combo = key * (1 << 32) + (0xFFFFFFFF - idx)
    order = np.argsort(-combo, axis=-1, kind="stable")[..., :k]
    return order.astype(np.int64)


def compute_vertical_indices(query_states: np.ndarray, key_states: np.ndarray,
                             window_size: int, top_ratio: float,
                             kv_repeat: int = 1, fp16: bool = False) -> np.ndarray:
    """src/patch/_common.py:144-190.

    query_states [B, H_Q, Q, D] (bf16 values), key_states [B, H, K, D] with
    H == H_Q or H == H_Q / kv_repeat.  fp16=True: fp16 values, the mean and
    the scores in fp16 (the model dtype).  Returns int64 [B, H_Q, top_k].
    """
    B, HQ, QL, D = query_states.shape
    KL = key_states.shape[2]
    P = max(0, KL - window_size)
    if P == 0:
        return np.zeros((B, HQ, 0), dtype=np.int64)
    tail = min(window_size, QL)
    qm = mean_half(query_states[:, :, QL - tail:, :], 2, fp16)          # [B, HQ, D]
    HK = key_states.shape[1]
    if kv_repeat <= 1 or HK == HQ:
        kp = key_states[:, :, :P, :]
        scores = dot_bf16_exact(qm, kp, fp16)                             # [B, HQ, P]
    else:
        assert HQ == HK * kv_repeat
        kp = np.repeat(key_states[:, :, :P, :], kv_repeat, axis=1)        # head h -> h // R
        scores = dot_bf16_exact(qm, kp, fp16)
    k = top_k_count(P, top_ratio)
    return topk_desc_index_asc(scores, k, fp16)


def vertical_scores(query_states, key_states, window_size, kv_repeat=1, fp16=False):
    """The bf16 (fp16) score matrix the selector ranks (for tests)."""
    B, HQ, QL, D = query_states.shape
    KL = key_states.shape[2]
    P = max(0, KL - window_size)
    tail = min(window_size, QL)
    qm = mean_half(query_states[:, :, QL - tail:, :], 2, fp16)
    HK = key_states.shape[1]
    kp = key_states[:, :, :P, :]
    if HK != HQ:
        kp = np.repeat(kp, HQ // HK, axis=1)
    return dot_bf16_exact(qm, kp, fp16)


# ---------------------------------------------------------------------------
# a5/a3: cache reorganisation (freeze) and staging ring
# src/ops/d_stage_kv_cache.py:82-100 (prefill), :106-189 (freeze),
# :195-217 (append_staging / flush)
# ---------------------------------------------------------------------------


@dataclass
class DecodeState:
    """The four decode segments at KV-head granularity (BH = B * H_KV)."""
    k_packed: np.ndarray           # int8 [BH, Nq, D/2]
    v_packed: np.ndarray
    k_scale: np.ndarray            # fp16 [BH, Nq]
    v_scale: np.ndarray
    k_topk: np.ndarray             # bf16 values [BH, T, D]
    v_topk: np.ndarray
    k_window: np.ndarray           # [BH, W, D]
    v_window: np.ndarray
    k_ring: np.ndarray             # [BH, 128, D]
    v_ring: np.ndarray
    ring_ptr: int = 0
    k_bits: int = 4
    v_bits: int = 4
    topk_idx: Optional[np.ndarray] = None      # [B, H_KV, T] positions in the prefix
    compact_idx: Optional[np.ndarray] = None   # [B, H_KV, Nq_initial]

    @property
    def k_staging(self):
        return self.k_ring[:, :self.ring_ptr]

    @property
    def v_staging(self):
        return self.v_ring[:, :self.ring_ptr]


def group_mean_query(query_tail: np.ndarray, h_kv: int, fp16: bool = False) -> np.ndarray:
    """[B, H_Q, W, D] -> bf16 (fp16) mean over each KV group (src/ops/d_stage_kv_cache.py:131-133)."""
    B, HQ, W, D = query_tail.shape
    R = HQ // h_kv
    return mean_half(query_tail.reshape(B, h_kv, R, W, D), 2, fp16)


def freeze(keys: np.ndarray, values: np.ndarray, query_tail: Optional[np.ndarray],
           window_size: int, top_ratio: float, kv_repeat: int,
           k_bits: int = 4, v_bits: int = 4, use_vert: bool = True, fp16: bool = False) -> DecodeState:
    """Prefill -> decode reorganisation (src/ops/d_stage_kv_cache.py:106-189).

    keys/values [B, H_KV, N, D]; query_tail [B, H_Q, W', D] (the last
    min(window_size, Q) prefill queries, :97-100).  fp16=True: an fp16
    model's values; the selector's means and scores are fp16 (quantisation
    is the same formula on the fp16 values).
    """
    B, HKV, N, D = keys.shape
    BH = B * HKV
    W = min(window_size, N)
    P = N - W
    k_window = keys[:, :, N - W:, :].reshape(BH, W, D).copy()
    v_window = values[:, :, N - W:, :].reshape(BH, W, D).copy()
    topk_idx = np.zeros((B, HKV, 0), dtype=np.int64)
    if P > 0:
        kp = keys[:, :, :P, :]
        vp = values[:, :, :P, :]
        if use_vert and query_tail is not None and kv_repeat >= 1:
            q_kv = group_mean_query(query_tail, HKV, fp16)                 # [B, HKV, W', D]
            # the selector again subtracts window_size from the already
            # window-free prefix (F3: vertical lines come from [0, N - 2W))
            topk_idx = compute_vertical_indices(q_kv, kp, window_size, top_ratio, fp16=fp16)
        T = topk_idx.shape[-1]
        sel = np.zeros((B, HKV, P), dtype=bool)
        bi, hi = np.meshgrid(np.arange(B), np.arange(HKV), indexing="ij")
        for t in range(T):
            sel[bi, hi, topk_idx[:, :, t]] = True
        compact = np.stack([np.stack([np.nonzero(~sel[b, h])[0] for h in range(HKV)]) for b in range(B)])
        k_topk = np.take_along_axis(kp, topk_idx[..., None], axis=2).reshape(BH, T, D)
        v_topk = np.take_along_axis(vp, topk_idx[..., None], axis=2).reshape(BH, T, D)
        kc = np.take_along_axis(kp, compact[..., None], axis=2).reshape(BH, P - T, D)
        vc = np.take_along_axis(vp, compact[..., None], axis=2).reshape(BH, P - T, D)
        k_packed, k_scale = quantize_per_token(kc, k_bits)
        v_packed, v_scale = quantize_per_token(vc, v_bits)
    else:
        compact = np.zeros((B, HKV, 0), dtype=np.int64)
        k_topk = np.zeros((BH, 0, D), np.float32)
        v_topk = np.zeros((BH, 0, D), np.float32)
        k_packed = np.zeros((BH, 0, D * k_bits // 8), np.int8)
        v_packed = np.zeros((BH, 0, D * v_bits // 8), np.int8)
        k_scale = np.zeros((BH, 0), np.float16)
        v_scale = np.zeros((BH, 0), np.float16)
    return DecodeState(k_packed, v_packed, k_scale, v_scale, k_topk, v_topk,
                       k_window, v_window,
                       np.zeros((BH, GROUP_SIZE, D), np.float32),
                       np.zeros((BH, GROUP_SIZE, D), np.float32),
                       0, k_bits, v_bits, topk_idx, compact)


def append_staging(st: DecodeState, k_new: np.ndarray, v_new: np.ndarray) -> None:
    """k_new/v_new [B, H_KV, S, D]: write into the ring, flushing (quantise +
    append to the prefix) whenever 128 slots fill (src/ops/d_stage_kv_cache.py:195-217)."""
    B, HKV, S, D = k_new.shape
    k = k_new.reshape(B * HKV, S, D)
    v = v_new.reshape(B * HKV, S, D)
    for i in range(S):
        st.k_ring[:, st.ring_ptr] = k[:, i]
        st.v_ring[:, st.ring_ptr] = v[:, i]
        st.ring_ptr += 1
        if st.ring_ptr >= GROUP_SIZE:
            flush_staging(st)


def flush_staging(st: DecodeState) -> None:
    kp, ks = quantize_per_token(st.k_ring, st.k_bits)
    vp, vs = quantize_per_token(st.v_ring, st.v_bits)
    st.k_packed = np.concatenate([st.k_packed, kp], axis=1)
    st.v_packed = np.concatenate([st.v_packed, vp], axis=1)
    st.k_scale = np.concatenate([st.k_scale, ks], axis=1)
    st.v_scale = np.concatenate([st.v_scale, vs], axis=1)
    st.ring_ptr = 0


# ---------------------------------------------------------------------------
# a6-a11: four-segment decode attention
# ---------------------------------------------------------------------------


def decode_fp64(q: np.ndarray, k_packed, v_packed, k_scale, v_scale,
                k_topk, v_topk, k_staging, v_staging, k_window, v_window,
                k_bits: int = 4, v_bits: int = 4, kv_repeat: int = 1,
                sm_scale: Optional[float] = None, abs_v: bool = False) -> np.ndarray:
    """Exact (float64) restatement of fused_d_stage_decode
    (src/ops/decode_d_stage.py:916-1005, kernel math :599-691 and :221-267):
    softmax over [deq(prefix) | topk | staging | window] of q . k * sm_scale,
    with the int4 prefix dequantised as code * scale (the kernel factors the
    per-token scales out of the dot products, F8), GQA head h -> KV head h // R.

    q [BH_Q, D] -> out float64 [BH_Q, D].  abs_v=True attends over |V| instead
    (used by tests as the magnitude that bf16 rounding errors scale with).
    """
    BHQ, D = q.shape
    BHK = BHQ // kv_repeat
    if sm_scale is None:
        sm_scale = D ** -0.5
    kq = unpack_codes(k_packed, k_bits).astype(np.float64) * k_scale.astype(np.float64)[..., None]
    vq = unpack_codes(v_packed, v_bits).astype(np.float64) * v_scale.astype(np.float64)[..., None]
    K = np.concatenate([kq, k_topk, k_staging, k_window], axis=1).astype(np.float64)
    V = np.concatenate([vq, v_topk, v_staging, v_window], axis=1).astype(np.float64)
    if abs_v:   # sum_t p_t |v_t| / l: the scale of rounding errors in P and in the output
        V = np.abs(V)
    qg = q.astype(np.float64).reshape(BHK, kv_repeat, D)            # head h -> KV head h // R
    s = np.einsum("hrd,hnd->hrn", qg, K) * sm_scale
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=2, keepdims=True)
    return np.einsum("hrn,hnd->hrd", p, V).reshape(BHQ, D)


# ---------------------------------------------------------------------------
# legacy decode format (src/ops/d_stage_cache.py)
# ---------------------------------------------------------------------------


def legacy_unpack(packed: np.ndarray, nbits: int) -> np.ndarray:
    """Offset-encoded codes of the legacy format -> float32 values.
    int4 (src/ops/d_stage_cache.py:1020-1028): byte j holds channel 2j in the
    HIGH nibble and 2j+1 in the low nibble, value u - 8.  int2 (:1074-1087):
    byte k holds channel 4k+i in bits (7-2i, 6-2i), value u - 1.5.
    packed uint8 [..., D*nbits/8] -> [..., D]."""
    b = np.asarray(packed).astype(np.uint8).astype(np.int32)
    if nbits == 4:
        parts = [(b >> 4) - 8, (b & 15) - 8]
        return np.stack(parts, axis=-1).reshape(*b.shape[:-1], 2 * b.shape[-1]).astype(np.float32)
    if nbits == 2:
        parts = [((b >> (6 - 2 * i)) & 3).astype(np.float32) - 1.5 for i in range(4)]
        return np.stack(parts, axis=-1).reshape(*b.shape[:-1], 4 * b.shape[-1]).astype(np.float32)
    raise ValueError(f"legacy format bits must be 2 or 4, got {nbits}")


def legacy_values(packed: np.ndarray, scale: np.ndarray, nbits: int, group: int = GROUP_SIZE) -> np.ndarray:
    """Exact float64 values (code value) * scale[token // group][channel]:
    packed [BH, N, D*nbits/8], scale fp16 [BH, G, D] -> [BH, N, D]
    (the K_int * sk / V_int * sv products of src/ops/d_stage_cache.py:1041-1044,
    :1088-1092)."""
    v = legacy_unpack(packed, nbits).astype(np.float64)
    N = v.shape[1]
    g = np.arange(N) // group
    return v * scale.astype(np.float64)[:, g, :]


def legacy_dequant_bf16(packed: np.ndarray, scale: np.ndarray, nbits: int, group: int = GROUP_SIZE) -> np.ndarray:
    """(K_int * sk).to(bfloat16) (src/ops/d_stage_cache.py:1045): the exact
    product rounded once to bf16, as bf16 bits [BH, N, D] (uint16)."""
    x = legacy_values(packed, scale, nbits, group)
    return f32_to_bf16_bits(x.astype(np.float32))     # the product is exact in float32


def legacy_decode_fp64(q: np.ndarray, k_packed, v_packed, k_scale, v_scale,
                       k_topk, v_topk, k_staging, v_staging, k_window, v_window,
                       k_bits: int = 4, v_bits: int = 4, kv_repeat: int = 1,
                       sm_scale: Optional[float] = None, group: int = GROUP_SIZE,
                       abs_v: bool = False, bf16_operands: bool = False) -> np.ndarray:
    """Float64 restatement of the legacy four-segment decode
    (fused_decode_attention_k4v4 / splitk_decode_attention_k4v4(_mma),
    src/ops/d_stage_cache.py:396-502, :595-822, :955-1245): softmax over
    [prefix | topk | staging | window] of q . k * sm_scale with the prefix
    values of legacy_values; q [BH_Q, D], KV head of query head h = h // R.
    bf16_operands=True rounds the prefix values to bf16 first, as the MMA
    variant's K_deq / V_deq (:1045, :1092).  Returns [BH_Q, D] float64."""
    BHQ, D = q.shape
    BHK = BHQ // kv_repeat
    if sm_scale is None:
        sm_scale = D ** -0.5
    if k_packed.shape[1] > 0:
        kq = legacy_values(k_packed, k_scale, k_bits, group)
        vq = legacy_values(v_packed, v_scale, v_bits, group)
        if bf16_operands:
            kq = bf16_round(kq.astype(np.float32)).astype(np.float64)
            vq = bf16_round(vq.astype(np.float32)).astype(np.float64)
    else:
        kq = np.zeros((BHK, 0, D))
        vq = np.zeros((BHK, 0, D))
    K = np.concatenate([kq, k_topk, k_staging, k_window], axis=1).astype(np.float64)
    V = np.concatenate([vq, v_topk, v_staging, v_window], axis=1).astype(np.float64)
    if abs_v:
        V = np.abs(V)
    qg = q.astype(np.float64).reshape(BHK, kv_repeat, D)
    s = np.einsum("hrd,hnd->hrn", qg, K) * sm_scale
    s -= s.max(axis=2, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=2, keepdims=True)
    return np.einsum("hrn,hnd->hrd", p, V).reshape(BHQ, D)


def decode_fp64_state(q: np.ndarray, st: DecodeState, kv_repeat: int, sm_scale=None,
                      abs_v: bool = False) -> np.ndarray:
    return decode_fp64(q, st.k_packed, st.v_packed, st.k_scale, st.v_scale,
                       st.k_topk, st.v_topk, st.k_staging, st.v_staging,
                       st.k_window, st.v_window, st.k_bits, st.v_bits, kv_repeat, sm_scale, abs_v)


def decode_bf16_eager(q, st: DecodeState, kv_repeat: int, B: int):
    """The reference's PyTorch eager decode (src/ops/d_stage_kv_cache.py:309-354):
    dequantise to fp16 then bf16, concatenate [prefix, topk, staging, window],
    expand GQA, then bf16 matmul -> bf16 softmax -> bf16 matmul.  Runs on the
    CPU with torch.  q [BH_Q, D] (bf16 values) -> float32 [BH_Q, D]."""
    import torch
    return decode_bf16_eager_torch(torch.from_numpy(np.asarray(q, np.float32)),
                                   prepare_eager_state(st), kv_repeat, B).float().numpy()


def prepare_eager_state(st: DecodeState):
    """Torch CPU tensors for decode_bf16_eager_torch (kept separate so that a
    timing loop measures only the per-step decode work)."""
    import torch
    bf = torch.bfloat16
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return dict(
        k_packed=t(st.k_packed), v_packed=t(st.v_packed),
        k_scale=t(st.k_scale), v_scale=t(st.v_scale),
        k_topk=t(st.k_topk.astype(np.float32)).to(bf), v_topk=t(st.v_topk.astype(np.float32)).to(bf),
        k_staging=t(st.k_staging.astype(np.float32)).to(bf), v_staging=t(st.v_staging.astype(np.float32)).to(bf),
        k_window=t(st.k_window.astype(np.float32)).to(bf), v_window=t(st.v_window.astype(np.float32)).to(bf),
        k_bits=st.k_bits, v_bits=st.v_bits)


def _torch_dequant(packed, scale, bits):
    import torch
    if bits == 4:
        x = packed.to(torch.int32) & 0xFF
        lo = ((x & 0x0F) << 28) >> 28
        hi = (((x >> 4) & 0x0F) << 28) >> 28
        q = torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 2).float()
    elif bits == 8:
        q = packed.float()
    else:
        x = packed.to(torch.int32) & 0xFF
        parts = [(((x >> (2 * j)) & 0x03) << 30) >> 30 for j in range(4)]
        q = torch.stack(parts, dim=-1).reshape(*packed.shape[:-1], packed.shape[-1] * 4).float()
    return (q * scale.float().unsqueeze(-1)).to(torch.float16)


def decode_bf16_eager_torch(q, es: dict, kv_repeat: int, B: int):
    """Per-step body of decode_bf16_eager on torch CPU tensors."""
    import torch
    bf = torch.bfloat16
    BHQ, D = q.shape
    HQ = BHQ // B
    HKV = HQ // kv_repeat
    kp = _torch_dequant(es["k_packed"], es["k_scale"], es["k_bits"]).to(bf)
    vp = _torch_dequant(es["v_packed"], es["v_scale"], es["v_bits"]).to(bf)
    K = torch.cat([kp, es["k_topk"], es["k_staging"], es["k_window"]], dim=1)
    V = torch.cat([vp, es["v_topk"], es["v_staging"], es["v_window"]], dim=1)
    NT = K.shape[1]
    K = K.reshape(B, HKV, NT, D).unsqueeze(2).expand(B, HKV, kv_repeat, NT, D).reshape(B, HQ, NT, D)
    V = V.reshape(B, HKV, NT, D).unsqueeze(2).expand(B, HKV, kv_repeat, NT, D).reshape(B, HQ, NT, D)
    qq = q.to(bf).reshape(B, HQ, 1, D)
    scores = (qq @ K.transpose(-1, -2)) * (D ** -0.5)
    out = torch.softmax(scores, dim=-1) @ V
    return out.reshape(BHQ, D)


# ---------------------------------------------------------------------------
# Seeded synthetic inputs (the benchmark's data distribution)
# ---------------------------------------------------------------------------


@dataclass
class DecodeInputs:
    B: int
    HQ: int
    HKV: int
    N: int
    D: int
    W: int
    S: int
    rho: float
    keys: np.ndarray          # [B, HKV, N, D] prefill keys (bf16 values)
    values: np.ndarray
    query_tail: np.ndarray    # [B, HQ, W, D] last W prefill queries
    k_new: np.ndarray         # [B, HKV, S, D] decode-time tokens (staging)
    v_new: np.ndarray
    q_dec: np.ndarray         # [B*HQ, D] the decode query
    planted: np.ndarray       # [B, HKV, n_plant] planted vertical-line positions


def make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, D=128, W=128, S=37, rho=0.05,
                       seed=0, plant_ratio=0.05) -> DecodeInputs:
    """Seeded Gaussian inputs with outlier channels and planted vertical lines.

    torch.Generator().manual_seed(seed) on the CPU draws, in order:
      query tail [B, HQ, W, D], keys [B, HKV, N, D], values [B, HKV, N, D],
      per-(KV head, channel) key offsets ~ N(0, 2) (std sqrt(2)),
      per (b, KV head) the planted positions (randperm of the non-window
      prefix, first int(plant_ratio * N)), staging keys/values [B, HKV, S, D],
      and the decode query [B*HQ, D].
    Keys get their head's offset on every token.  A planted position's key is
    offset + 3 * sqrt(D) * u, u the unit mean direction of the KV group's
    query tail.  Everything is rounded to bf16.
    """
    import torch
    g = torch.Generator().manual_seed(seed)
    G = HQ // HKV
    qt = torch.randn(B, HQ, W, D, generator=g)
    k = torch.randn(B, HKV, N, D, generator=g)
    v = torch.randn(B, HKV, N, D, generator=g)
    off = torch.randn(HKV, D, generator=g) * math.sqrt(2.0)
    k = k + off[None, :, None, :]
    qt_b = qt.to(torch.bfloat16).float()
    n_plant = min(int(plant_ratio * N), max(0, N - W))
    planted = np.zeros((B, HKV, n_plant), dtype=np.int64)
    if N <= W:                   # no non-window prefix: nothing to plant
        n_plant = 0
        planted = np.zeros((B, HKV, 0), dtype=np.int64)
    for b in range(B):
        for h in range(HKV):
            if n_plant == 0:
                continue
            u = qt_b[b, h * G:(h + 1) * G].reshape(-1, D).mean(dim=0)
            u = u / u.norm()
            pos = torch.randperm(N - W, generator=g)[:n_plant]
            k[b, h, pos, :] = off[h] + 3.0 * math.sqrt(D) * u
            planted[b, h, :len(pos)] = np.sort(pos.numpy())
    k_new = torch.randn(B, HKV, S, D, generator=g) + off[None, :, None, :]
    v_new = torch.randn(B, HKV, S, D, generator=g)
    q_dec = torch.randn(B * HQ, D, generator=g)
    cv = lambda t: t.to(torch.bfloat16).float().numpy()
    return DecodeInputs(B, HQ, HKV, N, D, W, S, rho, cv(k), cv(v), cv(qt),
                        cv(k_new), cv(v_new), cv(q_dec), planted)


def build_decode_state(inp: DecodeInputs) -> DecodeState:
    """freeze() the prefill cache, then append the S staging tokens."""
    st = freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, inp.HQ // inp.HKV)
    append_staging(st, inp.k_new, inp.v_new)
    return st


# ---------------------------------------------------------------------------
# a12-a15: hybrid prefill (src/ops/sage_unified.py:499-622 with
# src/ops/vendor/sageattention/triton/quant_per_block.py:21-101)
# ---------------------------------------------------------------------------

PREFILL_BLOCK_M = 128   # query rows per block (Q int8 scale granularity, window alignment)
PREFILL_BLOCK_N = 64    # key rows per tile (rest-K int8 scale granularity)


def per_block_int8(x: np.ndarray, sm: float, blk: int) -> Tuple[np.ndarray, np.ndarray]:
    """quant_per_block_int8_kernel (quant_per_block.py:21-46): over blocks of
    `blk` rows of x [..., L, D]: xs = fp32(x) * fp32(sm); scale = amax / 127;
    code = trunc(xs / scale + 0.5 * sign) (round half away from zero), all in
    fp32.  A block of zeros gets scale 0 and codes 0.  Returns (codes int8,
    scale float32 [..., ceil(L / blk)])."""
    xf = np.asarray(x, dtype=np.float32) * np.float32(sm)
    L = xf.shape[-2]
    nb = (L + blk - 1) // blk
    codes = np.zeros(xf.shape, dtype=np.int8)
    scales = np.zeros(xf.shape[:-2] + (nb,), dtype=np.float32)
    for i in range(nb):
        blk_x = xf[..., i * blk:(i + 1) * blk, :]
        amax = np.abs(blk_x).max(axis=(-2, -1))
        scale = (amax / np.float32(127.0)).astype(np.float32)
        scales[..., i] = scale
        with np.errstate(divide="ignore", invalid="ignore"):
            r = (blk_x / scale[..., None, None]).astype(np.float32)
            r = (r + np.where(r >= 0, np.float32(0.5), np.float32(-0.5))).astype(np.float32)
        r = np.where(scale[..., None, None] > 0, r, 0)
        codes[..., i * blk:(i + 1) * blk, :] = np.trunc(r).astype(np.int8)
    return codes, scales


def smooth_keys(k: np.ndarray, smooth: bool = True, fp16: bool = False) -> Tuple[np.ndarray, np.ndarray]:
    """K-smoothing (sage_unified.py:565-570): km = bf16 mean over the sequence
    (exact float64 sum, one RNE rounding), ks = bf16(fp32(k) - fp32(km)).
    fp16=True (an fp16 model, k holding fp16 values): the same in fp16.
    Returns (km [..., 1, D], ks)."""
    if not smooth:
        return np.zeros(k.shape[:-2] + (1, k.shape[-1]), np.float32), np.asarray(k, np.float32)
    if fp16:
        km = mean_f16(k, axis=-2)[..., None, :]
        return km, to_fp16((np.asarray(k, np.float32) - km).astype(np.float32))
    km = mean_bf16(k, axis=-2)[..., None, :]
    ks = bf16_round((np.asarray(k, np.float32) - km).astype(np.float32))
    return km, ks


def to_fp16(x: np.ndarray) -> np.ndarray:
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def prefill_lists(vidx_row: np.ndarray, N: int, W: int):
    """reorder_kv_for_vertical (sage_unified.py:499-547) for one (b, h_q) row.
    The vertical list is the indices clamped to [0, P), P = N - W, sorted
    ascending (a repeated index stays repeated and is attended twice, as the
    reference's gather does); rest = the positions of [0, P) not in it,
    ascending.  Per query block b the counts of each below the 64-aligned
    window start wla(b) (searchsorted, left).  Returns (vert, rest, nv, nr)."""
    P = max(0, N - W)
    nblk = (N + PREFILL_BLOCK_M - 1) // PREFILL_BLOCK_M
    if P == 0:
        z = np.zeros(nblk, np.int64)
        return np.zeros(0, np.int64), np.zeros(0, np.int64), z, z
    vert = np.sort(np.clip(np.asarray(vidx_row, np.int64), 0, P - 1))
    mask = np.zeros(P, bool)
    mask[vert] = True
    rest = np.nonzero(~mask)[0]
    wla = np.array([window_start(b, W) for b in range(nblk)], np.int64)
    nv = np.searchsorted(vert, wla, side="left")
    nr = np.searchsorted(rest, wla, side="left")
    return vert, rest, nv, nr


def window_start(b: int, W: int) -> int:
    """First key of query block b's fp16 window segment (sage_unified.py:482-485
    and :538-541): floor64(max(0, 128 b - (W - 1)))."""
    return max(0, PREFILL_BLOCK_M * b - (W - 1)) // PREFILL_BLOCK_N * PREFILL_BLOCK_N


def prefill_operands(q, k, v, sm_scale: Optional[float] = None, smooth: bool = True, fp16: bool = False):
    """The wrapper's operand preparation (sage_unified.py:559-584):
    c = fp32(sm_scale * log2e); Q int8 per 128-row block of x = fp32(q) * c
    (codes, scales); q16 = fp16(bf16(fp32(q) * c)); km and the smoothed keys
    ks = bf16(k - km) as fp16; v16 = fp16(v).  fp16=True (an fp16 model: q,
    k, v hold fp16 values) takes the reference's fp16 branch (:569, :575-576):
    q16 = fp16(fp32(q) * c), km and ks rounded to fp16.  Returns a dict."""
    D = q.shape[-1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    c = np.float32(sm_scale * LOG2E)
    q8, qsc = per_block_int8(q, c, PREFILL_BLOCK_M)
    qc = (np.asarray(q, np.float32) * c).astype(np.float32)
    q16 = to_fp16(qc if fp16 else bf16_round(qc))
    km, ks = smooth_keys(k, smooth, fp16)
    return dict(c=c, q8=q8, q_scale=qsc, q16=q16, km=km, k16=to_fp16(ks), v16=to_fp16(v))


FP8_MAX = 448.0            # src/ops/sage_unified_fp8.py:44
S_FP8_OFFSET = 8.807       # src/ops/vendor/sageattention/csrc/qattn/attn_utils.cuh:30


def e4m3_round(x) -> np.ndarray:
    """OCP fp8 e4m3 (e4m3fn: bias 7, 3 mantissa bits, no infinities, max 448)
    round-to-nearest-even with saturation to +-448 (the satfinite conversion of
    src/ops/vendor/sageattention/csrc/qattn/attn_utils.cuh:478-493).  Returns
    the rounded values as float64."""
    x = np.asarray(x, np.float64)
    a = np.minimum(np.abs(x), FP8_MAX)
    with np.errstate(divide="ignore"):
        e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    e = np.maximum(e, -6.0)                      # subnormal spacing 2^-9 below 2^-6
    quantum = np.exp2(e - 3.0)
    r = np.round(a / quantum) * quantum          # numpy rounds half to even
    r = np.minimum(r, FP8_MAX)
    return np.where(x < 0, -r, r)


def fp8_v_operands(v):
    """Per-channel V scale over the whole sequence (no mean, smooth_v=False) and
    the e4m3 codes of v / scale (src/ops/vendor/sageattention/quant.py:136-166,
    csrc/fused/fused.cu:319-430): scale = fp32(max|v| / 448) per (b, kv head,
    channel); v8 = e4m3(fp32(v) / scale); zero where scale is zero.  Also
    returns fp16(fp32(v) / scale), the scaled fp16 values the hybrid kernel
    feeds its vertical and window tiles in fp8 mode."""
    v32 = np.asarray(v, np.float32)
    vs = (np.max(np.abs(v32), axis=2, keepdims=True) / np.float32(FP8_MAX)).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(vs > 0, v32 / np.where(vs > 0, vs, 1), 0).astype(np.float32)
    return vs, e4m3_round(ratio), to_fp16(ratio)


def per_block_fp8(x: np.ndarray, sm: float, blk: int) -> Tuple[np.ndarray, np.ndarray]:
    """_quant_per_block_fp8_kernel (src/ops/sage_unified_fp8.py:52-88) over
    blocks of `blk` rows of x [..., L, D]: xs = fp32(x) * fp32(sm); scale =
    fp32(amax / 448), 1 where that is not positive; code = e4m3(clamp(
    fp32(xs / scale), +-448)) rounded to nearest even.  Returns (the e4m3
    values as float64, scale float32 [..., ceil(L / blk)])."""
    xf = np.asarray(x, dtype=np.float32) * np.float32(sm)
    L = xf.shape[-2]
    nb = (L + blk - 1) // blk
    codes = np.zeros(xf.shape, dtype=np.float64)
    scales = np.zeros(xf.shape[:-2] + (nb,), dtype=np.float32)
    for i in range(nb):
        blk_x = xf[..., i * blk:(i + 1) * blk, :]
        amax = np.abs(blk_x).max(axis=(-2, -1))
        scale = (amax / np.float32(FP8_MAX)).astype(np.float32)
        scale = np.where(scale > 0, scale, np.float32(1.0)).astype(np.float32)
        scales[..., i] = scale
        r = (blk_x / scale[..., None, None]).astype(np.float32)
        r = np.clip(r, -FP8_MAX, FP8_MAX)
        codes[..., i * blk:(i + 1) * blk, :] = e4m3_round(r)
    return codes, scales


FP8_AMBIGUITY = 2.0 ** -14  # relative fp32 deviation of a kernel's p' from the exact one


def _round_span(x: np.ndarray, rnd, rel: float) -> np.ndarray:
    """|rnd(x (1 + rel)) - rnd(x (1 - rel))|: zero unless x lies within a
    relative `rel` of a rounding boundary of `rnd`, else the step between the
    two neighbours either rounding may take."""
    return np.abs(rnd(x * (1.0 + rel)) - rnd(x * (1.0 - rel)))


def hybrid_prefill_fp64(q, k, v, vidx, W: int, sm_scale: Optional[float] = None, smooth: bool = True,
                        int8_rest: bool = True, abs_v: bool = False, pv_mode: str = "fp16",
                        qk_mode: str = "int8", blocks=None, fp8_detail: bool = False, fp16: bool = False):
    """float64 restatement of sage_vertical_attention_v2 (sage_unified.py:550-622,
    kernel :398-496).  q [B, HQ, N, D], k/v [B, HKV, N, D] (bf16 values),
    vidx [B, HQ, T].  For query row i of block b (128 rows):
      rest keys (not vertical, position < wla(b)): s = (q8 . k8) * q_scale * k_scale
        (Q int8 per 128-row block with sm_scale*log2e folded in, K smoothed then
        int8 per 64-row block of the rest list, round half away from zero);
      vertical keys below wla(b) and window keys wla(b) <= j <= i:
        s = q16 . k16 with q16 = fp16(bf16(q * sm*log2e)), k16 = fp16(ks);
    one base-2 softmax over all of them, values fp16(v).  int8_rest=False
    scores the rest keys with q16 . k16 too (a check of the partition alone).
    abs_v=True returns sum p |v| / l instead (an error scale).

    pv_mode='fp8' follows the INT8-QK / FP8-PV kernel of the vendored
    SageAttention (qk_int_sv_f8_cuda_sm90.cu:300-345, :490-512 and
    attn_utils.cuh:354-458) on the rest keys: p' = exp2(s - m + 8.807)
    (m = the row max), P8 = e4m3(p'), V8 = e4m3(v / vs) with the per-channel
    scale vs = max|v| / 448; the vertical and window keys keep fp16 operands in
    the same units, fp16(p') and fp16(v / vs); o = (sum P V) / (sum p') * vs.
    qk_mode='fp8' scores the rest keys as sage_vertical_attention_v2_fp8
    (src/ops/sage_unified_fp8.py:158-311, quantiser :52-148): Q per 128-row
    block and rest K per 64-entry block in e4m3 (per_block_fp8),
    s = (q8 . k8) * q_scale * k_scale, everything else unchanged.

    blocks: the 128-row query blocks to compute (default all); rows of other
    blocks are left zero.  fp16: q, k, v are an fp16 model's (prefill_operands).

    fp8_detail (pv_mode='fp8'): also return `slack` and `exact_rows`.
    slack [B, HQ, N, D] = sum over keys j of |V_j| vs / l times the step
    between the two e4m3 (rest keys) or fp16 (vertical / window keys)
    neighbours of p'_j when p'_j lies within a relative FP8_AMBIGUITY of a
    rounding boundary (zero otherwise): the most a kernel whose p'
    deviates from the exact value by that much in fp32 can differ from this
    restatement through the rounding of P'.  exact_rows [B, HQ, N] marks
    the rows whose maximum score is attained (within 1e-6 in log2 units) by
    a key of the first 64-key tile the kernel visits (rest tiles, then
    vertical, then window, each in list order): for those the kernel's
    running maximum is the row maximum from its first tile on, so it rounds
    the same p'_j as this restatement.

    Returns float64 [B, HQ, N, D] (or (out, slack, exact_rows))."""
    B, HQ, N, D = q.shape
    HKV = k.shape[1]
    G = HQ // HKV
    op = prefill_operands(q, k, v, sm_scale, smooth, fp16)
    q8, qsc, q16, k16, v16 = op["q8"], op["q_scale"], op["q16"], op["k16"], op["v16"]
    quant = per_block_int8
    if qk_mode == "fp8":
        q8, qsc = per_block_fp8(q, op["c"], PREFILL_BLOCK_M)
        quant = per_block_fp8
    fp8 = pv_mode == "fp8"
    if fp8:
        vs, v8, v16 = fp8_v_operands(v)              # v16 := fp16(v / vs) here
    if abs_v:
        v16 = np.abs(v16)
        if fp8:
            v8 = np.abs(v8)
    out = np.zeros((B, HQ, N, D), np.float64)
    detail = fp8 and fp8_detail
    if detail:
        slack = np.zeros((B, HQ, N, D), np.float64)
        exact_rows = np.zeros((B, HQ, N), bool)
    nblk = (N + PREFILL_BLOCK_M - 1) // PREFILL_BLOCK_M
    blk_list = range(nblk) if blocks is None else [int(x) for x in blocks]
    for b in range(B):
        for h in range(HQ):
            hk = h // G
            vert, rest, nv, nr = prefill_lists(vidx[b, h], N, W)
            if len(rest):
                k8r, ksr = quant(k16[b, hk, rest], 1.0, PREFILL_BLOCK_N)
            for blk in blk_list:
                wla = window_start(blk, W)
                rows = np.arange(blk * PREFILL_BLOCK_M, min(N, (blk + 1) * PREFILL_BLOCK_M))
                qrow = q16[b, h, rows].astype(np.float64)
                segs_s, segs_v = [], []
                if nr[blk] > 0:
                    n = nr[blk]
                    if int8_rest:
                        kscale = np.repeat(ksr.astype(np.float64), PREFILL_BLOCK_N)[:n]
                        # integer (or e4m3) dot products, exact in float64
                        s = q8[b, h, rows].astype(np.float64) @ k8r[:n].astype(np.float64).T
                        segs_s.append(s * float(qsc[b, h, blk]) * kscale[None, :])
                    else:
                        segs_s.append(qrow @ k16[b, hk, rest[:n]].astype(np.float64).T)
                    segs_v.append((v8 if fp8 else v16)[b, hk, rest[:n]])
                if nv[blk] > 0:
                    idx = vert[:nv[blk]]
                    segs_s.append(qrow @ k16[b, hk, idx].astype(np.float64).T)
                    segs_v.append(v16[b, hk, idx])
                jw = np.arange(wla, min(N, (blk + 1) * PREFILL_BLOCK_M))
                sw = qrow @ k16[b, hk, jw].astype(np.float64).T
                segs_s.append(np.where(jw[None, :] <= rows[:, None], sw, -np.inf))
                segs_v.append(v16[b, hk, jw])
                S = np.concatenate(segs_s, axis=1)
                V = np.concatenate(segs_v, axis=0).astype(np.float64)
                if not fp8:
                    p = np.exp2(S - S.max(axis=1, keepdims=True))
                    out[b, h, rows] = (p @ V) / p.sum(axis=1, keepdims=True)
                    continue
                p = np.exp2((S - S.max(axis=1, keepdims=True)) + S_FP8_OFFSET)
                n_rest = nr[blk]
                pq = np.concatenate([e4m3_round(p[:, :n_rest]),
                                     to_fp16(p[:, n_rest:].astype(np.float32)).astype(np.float64)], axis=1)
                vsc = vs[b, hk, 0].astype(np.float64)[None, :]
                out[b, h, rows] = (pq @ V) / p.sum(axis=1, keepdims=True) * vsc
                if detail:
                    f16 = lambda x: to_fp16(x.astype(np.float32)).astype(np.float64)
                    span = np.concatenate([_round_span(p[:, :n_rest], e4m3_round, FP8_AMBIGUITY),
                                           _round_span(p[:, n_rest:], f16, FP8_AMBIGUITY)], axis=1)
                    slack[b, h, rows] = (span @ np.abs(V)) / p.sum(axis=1, keepdims=True) * vsc
                    n_vert = int(nv[blk])
                    if n_rest > 0:
                        first = slice(0, min(PREFILL_BLOCK_N, n_rest))
                    elif n_vert > 0:
                        first = slice(0, min(PREFILL_BLOCK_N, n_vert))
                    else:
                        first = slice(0, min(PREFILL_BLOCK_N, len(jw)))
                    exact_rows[b, h, rows] = S[:, first].max(axis=1) >= S.max(axis=1) - 1e-6
    if detail:
        return out, slack, exact_rows
    return out


def unified_prefill_fp64(q, k, v, W: int, sm_scale: Optional[float] = None, smooth: bool = True,
                         int8: bool = True, abs_v: bool = False, blocks=None, fp16: bool = False):
    """float64 restatement of sage_unified_attention (sage_unified.py:234-313,
    kernel _attn_fwd_unified :112-231).  W > 0: int8 keys below wla(b), the
    fp16 causal window wla(b) <= j <= i; this is hybrid_prefill_fp64 with no
    vertical lines.  W = 0: every key j <= i scored in int8,
    s = (q8 . k8) * q_scale * k_scale with K (smoothed) quantised per 64
    positions over the whole sequence (the int8 prefix segment :166-177 and
    the causal int8 diagonal :204-217).  int8=False scores every key with
    q16 . k16 instead, which checks the W = 0 partition alone.  blocks: the
    128-row query blocks to compute (default all; other rows stay zero)."""
    B, HQ, N, D = q.shape
    if W > 0:
        return hybrid_prefill_fp64(q, k, v, np.zeros((B, HQ, 0), np.int64), W, sm_scale, smooth,
                                   int8_rest=int8, abs_v=abs_v, blocks=blocks, fp16=fp16)
    HKV = k.shape[1]
    G = HQ // HKV
    op = prefill_operands(q, k, v, sm_scale, smooth, fp16)
    q8, qsc, q16, k16, v16 = op["q8"], op["q_scale"], op["q16"], op["k16"], op["v16"]
    if abs_v:
        v16 = np.abs(v16)
    out = np.zeros((B, HQ, N, D), np.float64)
    for b in range(B):
        for hk in range(HKV):
            k8, ksc = per_block_int8(k16[b, hk], 1.0, PREFILL_BLOCK_N)
            kscale = np.repeat(ksc.astype(np.float64), PREFILL_BLOCK_N)[:N]
            for h in range(hk * G, (hk + 1) * G):
                nblk = (N + PREFILL_BLOCK_M - 1) // PREFILL_BLOCK_M
                for blk in (range(nblk) if blocks is None else [int(x) for x in blocks]):
                    rows = np.arange(blk * PREFILL_BLOCK_M, min(N, (blk + 1) * PREFILL_BLOCK_M))
                    n = rows[-1] + 1
                    if int8:
                        s = q8[b, h, rows].astype(np.float64) @ k8[:n].astype(np.float64).T
                        s = s * float(qsc[b, h, blk]) * kscale[None, :n]
                    else:
                        s = q16[b, h, rows].astype(np.float64) @ k16[b, hk, :n].astype(np.float64).T
                    s = np.where(np.arange(n)[None, :] <= rows[:, None], s, -np.inf)
                    p = np.exp2(s - s.max(axis=1, keepdims=True))
                    out[b, h, rows] = (p @ v16[b, hk, :n].astype(np.float64)) / p.sum(axis=1, keepdims=True)
    return out


def exact_causal_attention(q, k, v, sm_scale: Optional[float] = None) -> np.ndarray:
    """softmax(q k^T * sm_scale + causal mask) v in float64, GQA by head // G."""
    B, HQ, N, D = q.shape
    G = HQ // k.shape[1]
    if sm_scale is None:
        sm_scale = D ** -0.5
    out = np.zeros((B, HQ, N, D), np.float64)
    mask = np.tril(np.ones((N, N), bool))
    for b in range(B):
        for h in range(HQ):
            s = q[b, h].astype(np.float64) @ k[b, h // G].astype(np.float64).T * sm_scale
            s = np.where(mask, s, -np.inf)
            s -= s.max(axis=1, keepdims=True)
            p = np.exp(s)
            out[b, h] = (p / p.sum(axis=1, keepdims=True)) @ v[b, h // G].astype(np.float64)
    return out


def make_prefill_inputs(B=1, HQ=32, HKV=8, N=8192, D=128, W=128, rho=0.05, seed=0, plant_ratio=0.05):
    """Seeded prefill inputs: Q, K, V ~ N(0,1) [B, H, N, D], per-(KV head,
    channel) K offsets ~ N(0, 2), planted vertical lines (as in
    make_decode_inputs, aligned with each KV group's last-W query mean).
    Returns (q, k, v) as bf16 values in float32 arrays."""
    import torch
    g = torch.Generator().manual_seed(seed)
    G = HQ // HKV
    q = torch.randn(B, HQ, N, D, generator=g)
    k = torch.randn(B, HKV, N, D, generator=g)
    v = torch.randn(B, HKV, N, D, generator=g)
    off = torch.randn(HKV, D, generator=g) * math.sqrt(2.0)
    k = k + off[None, :, None, :]
    qb = q.to(torch.bfloat16).float()
    n_plant = min(int(plant_ratio * N), max(0, N - W))
    for b in range(B):
        for h in range(HKV):
            if n_plant == 0:
                continue
            u = qb[b, h * G:(h + 1) * G, N - W:].reshape(-1, D).mean(dim=0)
            u = u / u.norm()
            pos = torch.randperm(N - W, generator=g)[:n_plant]
            k[b, h, pos, :] = off[h] + 3.0 * math.sqrt(D) * u
    cv = lambda t: t.to(torch.bfloat16).float().numpy()
    return cv(q), cv(k), cv(v)
