/*
 * hyq.h — C ABI of libhyq.so, the MI355X (gfx950) implementation of HyQuant's
 * hybrid-precision attention hot path.
 *
 * Conventions (every entry point):
 *   - all pointers are device pointers the caller owns; nothing is retained;
 *   - strides are in ELEMENTS of the pointed-to type; the innermost (channel)
 *     dimension is always contiguous;
 *   - work is enqueued asynchronously on `stream` (a hipStream_t; NULL = the
 *     legacy default stream); nothing synchronises;
 *   - the return value is HYQ_OK (0) or a negative status; hyq_last_error()
 *     returns a message for the calling thread's last failure.
 * Element types: bf16 and fp16 are passed as 16-bit storage (uint16_t), int4
 * codes as packed bytes (int8_t).
 */
#ifndef HYQ_H
#define HYQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HYQ_OK 0
#define HYQ_EINVAL (-22)   /* bad shape, stride, alignment or argument     */
#define HYQ_ENOTSUP (-95)  /* valid but unsupported configuration          */
#define HYQ_EDEVICE (-5)   /* HIP runtime / launch failure                  */
#define HYQ_ENOSPC (-28)   /* workspace or capacity too small               */

/* Message for the calling thread's last non-zero status ("" if none). */
const char* hyq_last_error(void);

/* ABI version of this library (incremented on any signature change). */
int hyq_abi_version(void);

/*
 * Per-token symmetric quantisation + packing.
 * Replaces quantize_per_token (src/ops/decode_d_stage.py:50-77) with
 * _pack_int4 (:104-111) / _pack_int2 (:126-133), and the staging flush's
 * quantisation (src/ops/d_stage_kv_cache.py:209-217).
 *   x      bf16 (x_is_fp16 = 0) or fp16 [bh, n, d]  strides (x_stride_bh, x_stride_n)
 *   packed int8 [bh, n, d*nbits/8] strides (p_stride_bh, p_stride_n)
 *   scale  fp16 [bh, n]            strides (s_stride_bh, 1)
 * scale = fp16(max(amax, 1e-5) / (2^(nbits-1)-1)) computed in fp32,
 * code  = clamp(round_half_even(x / scale), -2^(nbits-1), 2^(nbits-1)-1),
 * int4: even channel in the low nibble.  nbits in {2,4,8}; d = 8 * 2^k <= 512.
 * The output may be a window of a larger buffer (append at an offset).
 */
int hyq_quant_pack(const uint16_t* x, int32_t x_is_fp16, int64_t bh, int64_t n, int32_t d,
                   int64_t x_stride_bh, int64_t x_stride_n, int32_t nbits,
                   int8_t* packed, int64_t p_stride_bh, int64_t p_stride_n,
                   uint16_t* scale, int64_t s_stride_bh, void* stream);

/*
 * Per-token dequantisation.  Replaces dequantize_per_token
 * (src/ops/decode_d_stage.py:80-101) with _unpack_int4 (:114-123) /
 * _unpack_int2 (:136-149):
 *   packed int8 [bh, n, d*nbits/8] strides (p_stride_bh, p_stride_n)
 *   scale  fp16 [bh, n]            strides (s_stride_bh, 1)
 *   out    fp16 [bh, n, d]         strides (o_stride_bh, o_stride_n), rows 16-byte aligned
 * out = fp16(fp32(code) * fp32(scale)) (RNE); nbits in {2,4,8}; d = 8 * 2^k <= 512.
 */
int hyq_dequant(const int8_t* packed, int64_t bh, int64_t n, int32_t d,
                int64_t p_stride_bh, int64_t p_stride_n, int32_t nbits,
                const uint16_t* scale, int64_t s_stride_bh,
                uint16_t* out, int64_t o_stride_bh, int64_t o_stride_n, void* stream);

/*
 * Dequantisation of the legacy decode format: the [bh, n, d*nbits/8] uint8
 * prefix and [bh, G, d] fp16 per-group-per-channel scales read by
 * fused_decode_attention_k4v4 / splitk_decode_attention_k4v4(_mma)
 * (src/ops/d_stage_cache.py:281-373, :955-1087; their unpack and scale
 * loads).  Codes are offset-encoded: int4 even channel in the HIGH nibble,
 * value u - 8; int2 channel 4k+i in bits (7-2i, 6-2i) of byte k, value u - 1.5.
 *   packed uint8 [bh, n, d*nbits/8] strides (p_stride_bh, p_stride_n)
 *   scale  fp16  [bh, ceil(n/group), d] strides (s_stride_bh, s_stride_g, 1), rows 16-byte aligned
 *   out    bf16  [bh, n, d]         strides (o_stride_bh, o_stride_n), rows 16-byte aligned
 * out = bf16(fp32(value) * fp32(scale[token / group][channel])) (RNE);
 * nbits in {2,4}; d = 8 * 2^k <= 512.
 */
int hyq_legacy_dequant(const uint8_t* packed, int64_t bh, int64_t n, int32_t d,
                       int64_t p_stride_bh, int64_t p_stride_n, int32_t nbits,
                       const uint16_t* scale, int64_t s_stride_bh, int64_t s_stride_g, int32_t group,
                       uint16_t* out, int64_t o_stride_bh, int64_t o_stride_n, void* stream);

/*
 * Four-segment hybrid decode attention for one query token per head.
 * Replaces fused_d_stage_decode (src/ops/decode_d_stage.py:916-1005) and its
 * split-K path fused_d_stage_decode_splitk (:823-913) with kernels
 * _splitk_partial_kernel (:481-743) and _splitk_reduce_kernel (:746-782).
 * The three bf16 segments are passed separately (no host-side concatenation,
 * cf. :848-849); seg 0 = top-k vertical lines, 1 = staging, 2 = window.
 * Softmax runs over [int4 prefix | seg0 | seg1 | seg2] jointly.
 */
typedef struct hyq_decode_params {
    const uint16_t* q;    int64_t q_stride;        /* bf16 [bh_kv*kv_repeat, d]   */
    uint16_t* out;        int64_t out_stride;      /* bf16 [bh_kv*kv_repeat, d]   */
    const int8_t* k_packed; int64_t kp_stride_bh, kp_stride_n;  /* [bh_kv, n_quant, d/2] */
    const int8_t* v_packed; int64_t vp_stride_bh, vp_stride_n;
    const uint16_t* k_scale; int64_t ks_stride_bh;  /* fp16 [bh_kv, n_quant], token-contiguous */
    const uint16_t* v_scale; int64_t vs_stride_bh;
    int64_t n_quant;
    const uint16_t* seg_k[3]; int64_t seg_k_stride_bh[3]; int64_t seg_k_stride_n[3];
    const uint16_t* seg_v[3]; int64_t seg_v_stride_bh[3]; int64_t seg_v_stride_n[3];
    int64_t seg_n[3];
    int32_t bh_kv;        /* batch * kv heads                                  */
    int32_t kv_repeat;    /* query heads per kv head, 1..16                     */
    int32_t head_dim;     /* 128                                                */
    int32_t k_bits, v_bits; /* 2, 4 or 8 each (packed rows of 16 * bits bytes)  */
    float sm_scale;       /* softmax scale (reference default head_dim^-0.5)   */
    int32_t split_tokens; /* int4 tokens per workgroup; 0 = automatic           */
    /* Optional ragged lengths (NULL = the full n_quant / seg_n[0] for every
     * head): int32 device arrays [bh_kv] with each head's valid prefix tokens
     * and valid tokens of segment 0; the tensors stay padded to n_quant /
     * seg_n[0] and the rows past a head's length are never read.  Replaces
     * the seq_lens_quant / seq_lens_bf16 of fused_d_stage_decode_batched
     * (src/ops/decode_d_stage.py:1008-1129). */
    const int32_t* seq_lens_quant;
    const int32_t* seq_lens_seg0;
    /* HYQ_DT_* bits for an fp16 model (0 = all bf16).  fused_d_stage_decode
     * (src/ops/decode_d_stage.py:537-541, 240-263) rounds fp16 q and fp16
     * segment tiles to bf16 before its products and writes out in q.dtype
     * (:866, :782): HYQ_DT_Q_FP16 and HYQ_DT_SEG_FP16 apply that rounding
     * to q and to the three segments, HYQ_DT_OUT_FP16 rounds the fp32 result
     * to fp16 instead of bf16. */
    int32_t dtype_flags;
} hyq_decode_params;
#define HYQ_DT_Q_FP16 1
#define HYQ_DT_SEG_FP16 2
#define HYQ_DT_OUT_FP16 4
/* Alignment: q 16-byte aligned (row stride % 8 == 0), out 8-byte aligned (row
 * stride % 4 == 0), k_packed 16-byte aligned (8 for 2-bit K), v_packed aligned
 * to v_bits bytes, head strides likewise, bf16 segments 16-byte aligned. */

/* Bytes of device workspace hyq_decode_hybrid needs for these parameters:
 * a fixed 2 MiB area of per-head arrival counters (bh_kv <= 16384) followed
 * by the per-chunk partial results.  The workspace must be zero-filled once
 * when it is allocated; every completed call leaves the counter area at zero
 * again, so a workspace is reusable across calls of any shape without
 * clearing.  The call
 * enqueues one kernel on `stream`; calls that share one workspace must be
 * ordered on one stream. */
size_t hyq_decode_workspace_size(const hyq_decode_params* p);

int hyq_decode_hybrid(const hyq_decode_params* p, void* workspace,
                      size_t workspace_bytes, void* stream);

/*
 * hyq_decode_hybrid without a workspace argument and without any allocation.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The arrival counters, (m, l) table and partials live
 * in a 16 MiB array of library device memory, one per GPU, held until the
 * process ends; a call whose workspace (hyq_decode_workspace_size) exceeds
 * 16 MiB returns HYQ_ENOSPC.  The first call on a device looks the array up
 * and clears its counter area on `stream`.  Calls on one GPU share the array:
 * calls that overlap in time on one GPU (different streams, or host threads)
 * race and must be ordered by the caller; calls ordered on one stream are
 * safe.  Results are bit-identical to hyq_decode_hybrid's.
 */
int hyq_decode_hybrid_noalloc(const hyq_decode_params* p, void* stream);

/*
 * Decode over the legacy format, reading the codes directly.  Replaces
 * fused_decode_attention_k4v4 (src/ops/d_stage_cache.py:504-591),
 * splitk_decode_attention_k4v4 (:825-951) and
 * splitk_decode_attention_k4v4_mma (:1247-1366, K_BITS / V_BITS of 4 or 2):
 * the prefix codes and their per-(group, channel) fp16 scales are
 * dequantised in registers to the bf16 values of hyq_legacy_dequant (up to
 * an exact power of two that the kernel compensates), and attention runs
 * with bf16 K/V and P operands and fp32 accumulation, over the prefix and
 * three bf16 segments (top-k, staging, window), one softmax.  Codes are
 * offset-encoded: int4 has channel 2j in the HIGH nibble of byte j, value
 * u - 8; int2 has channel 4j + i in bits 7-2i..6-2i of byte j, value u - 1.5.
 *   q, out    bf16 [bh_kv * kv_repeat, 128] (row strides)
 *   k_codes   uint8 [bh_kv, n, 16 * k_bits] strides (kc_stride_bh, kc_stride_n),
 *             rows 4 * k_bits-byte aligned
 *   v_codes   uint8 [bh_kv, n, 16 * v_bits] strides (vc_stride_bh, vc_stride_n),
 *             rows v_bits-byte aligned
 *   k_scale, v_scale fp16 [bh_kv, ceil(n / group), 128] strides (bh, g, 1), rows 16-byte aligned
 *   seg_k, seg_v bf16 [bh_kv, seg_n, 128] with contiguous 128-element rows
 *     (head strides seg_*_stride_bh), 16-byte aligned
 * Limits: head_dim 128, k_bits and v_bits 2 or 4, kv_repeat 1..16, n and
 * each seg_n <= 2^24, code row strides <= 4096 bytes, group a positive
 * multiple of 16, each head's scale rows under 4 GiB.  Workspace rules as for
 * hyq_decode_hybrid (size from hyq_decode_legacy_workspace_size).
 */
typedef struct {
    const uint16_t* q; int64_t q_stride;
    uint16_t* out; int64_t out_stride;
    const uint8_t* k_codes; int64_t kc_stride_bh, kc_stride_n;
    const uint8_t* v_codes; int64_t vc_stride_bh, vc_stride_n;
    const uint16_t* k_scale; int64_t ks_stride_bh, ks_stride_g;
    const uint16_t* v_scale; int64_t vs_stride_bh, vs_stride_g;
    int64_t n;            /* prefix tokens                                       */
    int32_t group;        /* tokens per scale row (the reference's 128)          */
    int32_t k_bits, v_bits; /* code widths: 2 or 4                               */
    const uint16_t* seg_k[3]; int64_t seg_k_stride_bh[3];
    const uint16_t* seg_v[3]; int64_t seg_v_stride_bh[3];
    int64_t seg_n[3];
    int32_t bh_kv, kv_repeat, head_dim;
    float sm_scale;
} hyq_legacy_params;

size_t hyq_decode_legacy_workspace_size(const hyq_legacy_params* p);
int hyq_decode_legacy(const hyq_legacy_params* p, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Full-precision bf16 decode attention over one contiguous KV per head, the
 * hand-written split-K comparator at the same shapes (no reference
 * counterpart on this path other than the FA2 baseline of README.md:62-71).
 *   q/out bf16 [bh_kv*kv_repeat, d]; k, v bf16 [bh_kv, n, d].
 * Workspace rules as for hyq_decode_hybrid (size from
 * hyq_decode_bf16_workspace_size).
 */
size_t hyq_decode_bf16_workspace_size(int32_t bh_kv, int32_t kv_repeat, int64_t n, int32_t d);
int hyq_decode_bf16(const uint16_t* q, int64_t q_stride, uint16_t* out, int64_t out_stride,
                    const uint16_t* k, int64_t k_stride_bh, int64_t k_stride_n,
                    const uint16_t* v, int64_t v_stride_bh, int64_t v_stride_n,
                    int64_t n, int32_t bh_kv, int32_t kv_repeat, int32_t d, float sm_scale,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Vertical-line selector.  Replaces compute_vertical_indices
 * (src/patch/_common.py:144-190) for both of its call sites:
 *   prefill (src/patch/patch_llama.py:165-169): group = 1, q = all query heads,
 *     each query head scores the keys of its KV head (GQA-native);
 *   freeze (src/ops/d_stage_kv_cache.py:131-136): group = kv_repeat, the
 *     query tail is first averaged over each GQA group (one output per KV head).
 *   q    bf16 [b, hq_in, q_len, d]  strides (qs_b, qs_h, qs_t)
 *   k    bf16 [b, hk, >= p, d]      strides (ks_b, ks_h, ks_n); positions [0, p) are scored
 *   out  int64 [b, hq_in/group, top_k] (score desc, index asc)
 * qm = bf16(mean over the last `tail` queries [of bf16(mean over the group)]),
 * score = bf16(exact dot(qm, k)), top_k chosen by the caller
 * (reference: min(max(1, ceil(p * top_ratio)), p)).  is_fp16 = 1: q and k
 * are an fp16 model's, and the means and scores are rounded to fp16 (the
 * reference computes them in the model dtype).  d = 128, p < 2^31, top_k <= 2^30,
 * top_k <= p, at most 16 output heads per key head.  The workspace size
 * depends on top_k: winner sets too large for LDS are sorted in it.
 */
size_t hyq_vertical_select_workspace_size(int32_t b, int32_t h_out, int64_t p, int32_t top_k);
int hyq_vertical_select(const uint16_t* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, int32_t q_len,
                        int32_t hq_in, int32_t group, const uint16_t* k, int64_t ks_b, int64_t ks_h,
                        int64_t ks_n, int32_t hk, int64_t p, int32_t b, int32_t d, int32_t tail,
                        int32_t top_k, int32_t is_fp16, int64_t* out_idx, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * Prefill -> decode cache reorganisation.  Replaces the body of
 * DStageLayerCache.freeze after the selector (src/ops/d_stage_kv_cache.py:138-179):
 * given keys/values bf16 [b, hk, n, d] and the selected prefix positions
 * topk_idx int64 [b*hk, top_k] (in [0, n-w)), writes
 *   k/v_topk  bf16 [b*hk, top_k, d]   rows in topk_idx order
 *   k/v_window bf16 [b*hk, w, d]      the last w rows
 *   k/v_packed + k/v_scale            the other n-w-top_k prefix rows in
 *                                     ascending position, quantised per token
 *                                     exactly as hyq_quant_pack (k_bits, v_bits),
 *                                     any of the nine pairs of 2, 4 and 8 bits.
 * is_fp16 = 1: keys/values and the top-k / window copies are fp16 (an fp16
 * model; the codes and scales are those of hyq_quant_pack on fp16 input).
 * Precondition: each row of topk_idx holds distinct positions in [0, n-w)
 * (the selector's output).  Violations cannot make the call touch memory
 * outside its arguments: an index outside [0, n-w) copies a zero row into
 * k/v_topk and marks nothing, and the compact outputs are never written past
 * their n-w-top_k rows (with repeated or out-of-range indices some of those
 * rows stay unwritten).
 * Workspace: hyq_freeze_workspace_size(b*hk, n-w) bytes (a position bitmap).
 */
size_t hyq_freeze_workspace_size(int32_t bh, int64_t p);
int hyq_freeze_reorganise(const uint16_t* k, int64_t ks_b, int64_t ks_h, int64_t ks_n,
                          const uint16_t* v, int64_t vs_b, int64_t vs_h, int64_t vs_n,
                          int32_t b, int32_t hk, int64_t n, int32_t d, int32_t w,
                          const int64_t* topk_idx, int32_t top_k, int32_t k_bits, int32_t v_bits,
                          int32_t is_fp16, int8_t* kp, int64_t kp_bh, int64_t kp_n, int8_t* vp, int64_t vp_bh, int64_t vp_n,
                          uint16_t* ksc, int64_t ksc_bh, uint16_t* vsc, int64_t vsc_bh,
                          uint16_t* kt, int64_t kt_bh, int64_t kt_n, uint16_t* vt, int64_t vt_bh, int64_t vt_n,
                          uint16_t* kw, int64_t kw_bh, int64_t kw_n, uint16_t* vw, int64_t vw_bh, int64_t vw_n,
                          void* workspace, size_t workspace_bytes, void* stream);


/*
 * Per-block symmetric int8 quantisation.  Replaces per_block_int8 /
 * quant_per_block_int8_kernel (src/ops/vendor/sageattention/triton/
 * quant_per_block.py:21-101) for one tensor:
 *   x     bf16 (x_is_fp16 = 0) or fp16 [b, h, len, d], strides (xs_b, xs_h, xs_n),
 *         rows 16-byte aligned
 *   km    optional bf16 [b, h, d] (strides km_b, km_h): x <- bf16(x - km) first
 *   out   int8 [b, h, len, d], strides (os_b, os_h, os_n), rows 8-byte aligned
 *   scale fp32 [b, h, ceil(len / blk)], strides (ss_b, ss_h, 1)
 * Per block of blk rows: y = fp32(x) * sm, scale = amax(|y|) / 127,
 * code = trunc(y / scale + 0.5 * sign(y)) with IEEE fp32 division; a zero
 * block has scale 0 and codes 0.  d == 128.
 */
int hyq_per_block_int8(const void* x, int32_t x_is_fp16, int64_t xs_b, int64_t xs_h, int64_t xs_n,
                       int32_t b, int32_t h, int64_t len, int32_t d, float sm, int32_t blk,
                       const void* km, int64_t km_b, int64_t km_h,
                       void* out, int64_t os_b, int64_t os_h, int64_t os_n,
                       float* scale, int64_t ss_b, int64_t ss_h, void* stream);

/*
 * Rest / vertical index lists of the hybrid prefill.  Replaces the index part
 * of reorder_kv_for_vertical (src/ops/sage_unified.py:499-547), per (b, h):
 *   vert   int32 [b*h, t]     vidx clamped to [0, p) and sorted ascending
 *                             (repeats kept), p = max(0, n - window)
 *   rest   int32 [b*h, p]     the positions of [0, p) not in vert, ascending;
 *                             the first rcount[b*h] entries are valid
 *   nr, nv int32 [b*h, ceil(n/128)]  entries of rest / vert below the window
 *                             start of each 128-row query block,
 *                             wla = floor64(max(0, 128 blk - (window - 1)))
 * vidx int64 [b, h, t] with strides (vi_b, vi_h, vi_t).  p, t <= 2^24.
 * Workspace: hyq_prefill_lists_workspace_size(b, h, n, t, window) bytes, zero
 * (NULL allowed) while one head's lists fit the device's LDS, else a per-head
 * scratch for them, 4-byte aligned.
 */
size_t hyq_prefill_lists_workspace_size(int32_t b, int32_t h, int64_t n, int64_t t, int32_t window);
int hyq_prefill_lists(const int64_t* vidx, int64_t vi_b, int64_t vi_h, int64_t vi_t,
                      int32_t b, int32_t h, int64_t n, int64_t t, int32_t window,
                      int32_t* vert, int32_t* rest, int32_t* rcount, int32_t* nr, int32_t* nv,
                      void* workspace, size_t workspace_bytes, void* stream);

/* Arguments of hyq_prefill_hybrid (strides in elements, channels contiguous). */
typedef struct hyq_prefill_params {
    const void* q; int64_t q_stride_b, q_stride_h, q_stride_n;    /* bf16 [B, HQ, N, 128]  */
    const void* k; int64_t k_stride_b, k_stride_h, k_stride_n;    /* bf16 [B, HKV, N, 128] */
    const void* v; int64_t v_stride_b, v_stride_h, v_stride_n;    /* bf16 [B, HKV, N, 128] */
    const int64_t* vidx; int64_t vi_stride_b, vi_stride_h, vi_stride_t;  /* int64 [B, HQ, T] */
    void* out; int64_t o_stride_b, o_stride_h, o_stride_n;        /* bf16 [B, HQ, N, 128]  */
    int32_t batch, hq, hkv, head_dim;
    int64_t n, t;
    int32_t window;       /* local window W */
    int32_t smooth_k;     /* subtract the per-channel K mean before quantising */
    int32_t pv_mode;      /* 0: fp16 P.V; 1: OCP e4m3 P.V on the rest tiles */
    double sm_scale;      /* <= 0: head_dim^-0.5 */
    /* 1: q, k, v and out are fp16 (an fp16 model), 0: bf16.  The reference
     * (src/ops/sage_unified.py:565-580) forms the K mean, k - km and
     * q * sm_scale * log2e in the model dtype before .to(float16), and
     * returns q.dtype: an fp16 model rounds each once to fp16. */
    int32_t dtype_fp16;
} hyq_prefill_params;

/*
 * Hybrid-precision causal prefill attention.  Replaces
 * sage_vertical_attention_v2 (src/ops/sage_unified.py:550-622) and its kernel
 * _attn_fwd_vertical_v2 (:398-496); pv_mode 1 follows the FP8 P.V semantics
 * of the SM90 kernel (csrc/qattn/qk_int_sv_f8_cuda_sm90.cu:290-340, 490-512):
 * per-channel V scale amax/448, P scaled by 448 before the e4m3 cast.
 * For query block blk (128 rows) the keys are: rest positions below wla
 * (int8 Q . int8 K with per-block scales), vertical positions below wla and
 * the causal window wla <= j <= i (fp16 Q . fp16 K); one softmax; bf16 out.
 * Workspace: hyq_prefill_workspace_size(...) bytes, 256-byte aligned.
 * Limits: head_dim 128, N <= 2^24 (32-bit byte offsets of 256-byte rows per
 * head), N - window <= 2^24, T <= 2^24.
 */
size_t hyq_prefill_workspace_size(int32_t b, int32_t hq, int32_t hkv, int64_t n, int64_t t,
                                  int32_t window, int32_t pv_mode);
int hyq_prefill_hybrid(const hyq_prefill_params* params, void* workspace, size_t workspace_bytes,
                       void* stream);

/*
 * FP8-QK hybrid prefill.  Replaces sage_vertical_attention_v2_fp8
 * (src/ops/sage_unified_fp8.py:312-398, kernel :206-309, quantiser :52-148):
 * the partition of hyq_prefill_hybrid with the rest keys scored in OCP e4m3,
 * Q per 128-row block (x = q * sm_scale * log2e) and rest K per 64-entry
 * block with scale amax / 448 (1 for an all-zero block) and codes
 * e4m3(clamp(x / scale, +-448)); vertical and window tiles in fp16; fp16 P.V
 * (pv_mode must be 0).  Workspace as hyq_prefill_hybrid.
 */
int hyq_prefill_hybrid_fp8qk(const hyq_prefill_params* params, void* workspace, size_t workspace_bytes,
                             void* stream);

/*
 * Window-only INT8-QK prefill.  Replaces sage_unified_attention
 * (src/ops/sage_unified.py:234-313) and its kernel _attn_fwd_unified
 * (:112-231), the prefill of the sage_w / sage_w0 modes.  Same parameters as
 * hyq_prefill_hybrid with t = 0 (vidx unused); window > 0: int8 keys below
 * wla and the fp16 causal window wla <= j <= i, i.e. the hybrid partition
 * without vertical lines; window = 0: every key j <= i through int8 Q . K
 * (64-key K blocks, causal mask on the diagonal block).  Workspace:
 * hyq_prefill_workspace_size(b, hq, hkv, n, 0, window, pv_mode).
 */
int hyq_prefill_unified(const hyq_prefill_params* params, void* workspace, size_t workspace_bytes,
                        void* stream);

#ifdef __cplusplus
}
#endif
#endif /* HYQ_H */
