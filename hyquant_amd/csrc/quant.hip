// Per-token symmetric quantisation and nibble/crumb packing (the staging flush
// and the freeze quantiser), and the inverse dequantisation.  Semantics follow
// quantize_per_token / dequantize_per_token, src/ops/decode_d_stage.py:50-101,
// and _pack_int4/_pack_int2 / _unpack_int4/_unpack_int2 (:104-149):
//   scale = fp16(fp32(max(amax, 1e-5)) / qmax)        (IEEE fp32 divide, RNE)
//   code  = clamp(rint_half_even(x / fp32(scale)), qmin, qmax)
//   deq   = fp16(fp32(code) * fp32(scale))            (the product is exact)
// x is bf16 or fp16 (both are widened exactly to fp32 first).
// Layout: a group of d/8 lanes owns one token row; each lane loads 8
// channels with one 128-bit load and writes its packed bytes (dequantisation:
// reads the packed bytes of 8 channels, writes 16 bytes), so a wavefront
// moves 64*16 contiguous bytes per instruction.  HBM-bound.
#include "hyq_common.h"

#include <cstdio>
#include <string>

namespace hyq {
namespace {

template <int NBITS, bool F16>
__global__ __launch_bounds__(256) void quant_pack_kernel(
    const uint16_t* __restrict__ x, int64_t n, int64_t total, int lpt_log2,
    int64_t xs_bh, int64_t xs_n, int8_t* __restrict__ packed, int64_t ps_bh, int64_t ps_n,
    uint16_t* __restrict__ scale, int64_t ss_bh) {
    const int lpt = 1 << lpt_log2;                 // lanes per token
    const int lane = threadIdx.x & 63;
    const int sub = lane & (lpt - 1);              // lane within its token group
    const int64_t tokens_per_block = (256 >> lpt_log2);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * tokens_per_block + (threadIdx.x >> lpt_log2);
    const bool valid = t < total;
    const int64_t tt = valid ? t : total - 1;
    const int64_t ib = tt / n;
    const int64_t in = tt - ib * n;

    const uint4 raw = *reinterpret_cast<const uint4*>(x + ib * xs_bh + in * xs_n + sub * 8);
    float v[8];
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (F16) {
            v[2 * i] = f16_bits_to_f32(static_cast<uint16_t>(w[i]));
            v[2 * i + 1] = f16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16));
        } else {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    if (lpt == 16) {
        amax = max16_dpp(amax);
    } else {
        for (int m = 1; m < lpt; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    }
    amax = fmaxf(amax, 1e-5f);
    _Float16 s16;
    uint32_t c[8];                                  // code i in the low NBITS bits
    quant_row_codes<NBITS>(v, amax, s16, c);
    if (!valid) return;
    int8_t* prow = packed + ib * ps_bh + in * ps_n;
    if (NBITS == 4) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= static_cast<uint32_t>(c[i] & 15) << (4 * i);
        reinterpret_cast<uint32_t*>(prow)[sub] = word;
    } else if (NBITS == 8) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo |= static_cast<uint32_t>(c[i] & 255) << (8 * i);
            hi |= static_cast<uint32_t>(c[i + 4] & 255) << (8 * i);
        }
        reinterpret_cast<uint2*>(prow)[sub] = make_uint2(lo, hi);
    } else {
        uint32_t half = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) half |= static_cast<uint32_t>(c[i] & 3) << (2 * i);
        reinterpret_cast<uint16_t*>(prow)[sub] = static_cast<uint16_t>(half);
    }
    if (sub == 0) scale[ib * ss_bh + in] = __builtin_bit_cast(uint16_t, s16);
}

// code of channel i (0..7) of a lane's packed bytes, sign-extended
template <int NBITS>
__device__ __forceinline__ int code_at(uint32_t lo, uint32_t hi, int i) {
    if constexpr (NBITS == 4) return static_cast<int>(lo << (28 - 4 * i)) >> 28;
    else if constexpr (NBITS == 2) return static_cast<int>(lo << (30 - 2 * i)) >> 30;
    else return static_cast<int>((i < 4 ? lo : hi) << (24 - 8 * (i & 3))) >> 24;
}

template <int NBITS>
__global__ __launch_bounds__(256) void dequant_kernel(
    const int8_t* __restrict__ packed, int64_t n, int64_t total, int lpt_log2, int64_t ps_bh, int64_t ps_n,
    const uint16_t* __restrict__ scale, int64_t ss_bh, uint16_t* __restrict__ out, int64_t os_bh, int64_t os_n) {
    const int lpt = 1 << lpt_log2;
    const int sub = threadIdx.x & (lpt - 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (256 >> lpt_log2) + (threadIdx.x >> lpt_log2);
    if (t >= total) return;
    const int64_t ib = t / n, in = t - ib * n;
    const int8_t* prow = packed + ib * ps_bh + in * ps_n;
    uint32_t lo, hi = 0;
    if constexpr (NBITS == 4) {
        lo = reinterpret_cast<const uint32_t*>(prow)[sub];
    } else if constexpr (NBITS == 8) {
        const uint2 w = reinterpret_cast<const uint2*>(prow)[sub];
        lo = w.x; hi = w.y;
    } else {
        lo = reinterpret_cast<const uint16_t*>(prow)[sub];
    }
    // fp16(code * scale) as sign | fp16(|code| * |scale|): the product of the
    // magnitudes is exact in fp32 and rounds like the signed one, and the
    // sign is set explicitly because the compiler fuses the product and the
    // fp16 rounding into one fma with a +0 addend, which turns a -0 product
    // (negative code, zero scale) into +0
    const uint16_t sbits = scale[ib * ss_bh + in];
    const float smag = f16_bits_to_f32(static_cast<uint16_t>(sbits & 0x7fffu));
    const uint32_t ssign = sbits & 0x8000u;
    auto deq = [&](int c) -> uint32_t {
        const _Float16 m = static_cast<_Float16>(static_cast<float>(c < 0 ? -c : c) * smag);
        return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, m)) | ((c < 0 ? 0x8000u : 0u) ^ ssign);
    };
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        o[j] = deq(code_at<NBITS>(lo, hi, 2 * j)) | (deq(code_at<NBITS>(lo, hi, 2 * j + 1)) << 16);
    reinterpret_cast<uint4*>(out + ib * os_bh + in * os_n)[sub] = make_uint4(o[0], o[1], o[2], o[3]);
}

// Dequantisation of the legacy decode format of src/ops/d_stage_cache.py
// (the layout its fused / split-K kernels read, :281-373, :1019-1087):
// offset-encoded unsigned codes, int4 with the even channel in the HIGH
// nibble (value u - 8), int2 with channel 4k + i in bits 7-2i..6-2i (value
// u - 1.5), and one fp16 scale per (group of `group` tokens, channel),
// [bh, n / group, d].  out = bf16(fp32(u - offset) * fp32(scale)), RNE, as the
// reference's (K_int * sk).to(tl.bfloat16) (:1041-1045); the product is exact
// in fp32, and its sign is set explicitly (see dequant_kernel).  A lane owns
// 8 channels of one token: the scale row's 16 bytes and the packed bytes in
// one load each, 16 output bytes in one store.
template <int NBITS>
__global__ __launch_bounds__(256) void legacy_dequant_kernel(
    const uint8_t* __restrict__ packed, int64_t n, int64_t total, int lpt_log2, int64_t ps_bh, int64_t ps_n,
    const uint16_t* __restrict__ scale, int64_t ss_bh, int64_t ss_g, int group, uint16_t* __restrict__ out,
    int64_t os_bh, int64_t os_n) {
    const int lpt = 1 << lpt_log2;
    const int sub = threadIdx.x & (lpt - 1);
    const int64_t t = static_cast<int64_t>(blockIdx.x) * (256 >> lpt_log2) + (threadIdx.x >> lpt_log2);
    if (t >= total) return;
    const int64_t ib = t / n, in = t - ib * n;
    const uint8_t* prow = packed + ib * ps_bh + in * ps_n;
    const uint4 sraw = reinterpret_cast<const uint4*>(scale + ib * ss_bh + (in / group) * ss_g)[sub];
    const uint32_t sw[4] = {sraw.x, sraw.y, sraw.z, sraw.w};
    // twice the signed value of channel 8 sub + c: 2u - 16 (int4) or 2u - 3 (int2)
    int twice[8];
    if constexpr (NBITS == 4) {
        const uint32_t w = reinterpret_cast<const uint32_t*>(prow)[sub];   // channels 8sub .. 8sub+7
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t b = (w >> (8 * i)) & 0xffu;
            twice[2 * i] = 2 * static_cast<int>(b >> 4) - 16;
            twice[2 * i + 1] = 2 * static_cast<int>(b & 15u) - 16;
        }
    } else {
        const uint32_t w = reinterpret_cast<const uint16_t*>(prow)[sub];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t b = (w >> (8 * i)) & 0xffu;
#pragma unroll
            for (int j = 0; j < 4; ++j) twice[4 * i + j] = 2 * static_cast<int>((b >> (6 - 2 * j)) & 3u) - 3;
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t h[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) h[e] = legacy_twice_to_bf16(twice[2 * j + e], (sw[j] >> (16 * e)) & 0xffffu);
        o[j] = h[0] | (h[1] << 16);
    }
    reinterpret_cast<uint4*>(out + ib * os_bh + in * os_n)[sub] = make_uint4(o[0], o[1], o[2], o[3]);
}

int lanes_log2(int d) {
    int l = 0;
    while ((1 << l) < d / 8) ++l;
    return l;
}

bool ok_dim(int d) { return d > 0 && d % 8 == 0 && d <= 512 && ((d / 8) & (d / 8 - 1)) == 0; }

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" int hyq_quant_pack(const uint16_t* x, int32_t x_is_fp16, int64_t bh, int64_t n, int32_t d,
                              int64_t x_stride_bh, int64_t x_stride_n, int32_t nbits,
                              int8_t* packed, int64_t p_stride_bh, int64_t p_stride_n,
                              uint16_t* scale, int64_t s_stride_bh, void* stream) {
    if (bh < 0 || n < 0) return fail(HYQ_EINVAL, "hyq_quant_pack: negative shape");
    if (nbits != 2 && nbits != 4 && nbits != 8)
        return fail(HYQ_EINVAL, "nbits must be 2, 4, or 8, got " + std::to_string(nbits));
    if (!ok_dim(d))
        return fail(HYQ_ENOTSUP, "hyq_quant_pack: head dim must be 8*2^k <= 512, got " + std::to_string(d));
    if (bh == 0 || n == 0) return HYQ_OK;
    if (!x || !packed || !scale) return fail(HYQ_EINVAL, "hyq_quant_pack: null pointer");
    if (!aligned(x, 16) || x_stride_n % 8 || x_stride_bh % 8)
        return fail(HYQ_EINVAL, "hyq_quant_pack: x must be 16-byte aligned with strides divisible by 8");
    const int pbytes = nbits;  // packed bytes per lane (8 channels)
    if (!aligned(packed, pbytes) || p_stride_n % pbytes || p_stride_bh % pbytes)
        return fail(HYQ_EINVAL, "hyq_quant_pack: packed output misaligned");
    if (!aligned(scale, 2)) return fail(HYQ_EINVAL, "hyq_quant_pack: scale misaligned");
    const int lpt_log2 = lanes_log2(d);
    const int64_t total = bh * n;
    const int64_t tpb = 256 >> lpt_log2;
    const int64_t blocks = (total + tpb - 1) / tpb;
    if (blocks > 0x7fffffffLL) return fail(HYQ_ENOTSUP, "hyq_quant_pack: too many tokens");
    hipStream_t s = static_cast<hipStream_t>(stream);
    dim3 grid(static_cast<unsigned>(blocks)), block(256);
#define HYQ_QUANT(NB, F)                                                                            \
    quant_pack_kernel<NB, F><<<grid, block, 0, s>>>(x, n, total, lpt_log2, x_stride_bh, x_stride_n, \
                                                    packed, p_stride_bh, p_stride_n, scale, s_stride_bh)
    const bool f16 = x_is_fp16 != 0;
    if (nbits == 4) {
        if (f16) HYQ_QUANT(4, true); else HYQ_QUANT(4, false);
    } else if (nbits == 8) {
        if (f16) HYQ_QUANT(8, true); else HYQ_QUANT(8, false);
    } else {
        if (f16) HYQ_QUANT(2, true); else HYQ_QUANT(2, false);
    }
#undef HYQ_QUANT
    return check_launch("hyq_quant_pack");
}

extern "C" int hyq_dequant(const int8_t* packed, int64_t bh, int64_t n, int32_t d, int64_t p_stride_bh,
                           int64_t p_stride_n, int32_t nbits, const uint16_t* scale, int64_t s_stride_bh,
                           uint16_t* out, int64_t o_stride_bh, int64_t o_stride_n, void* stream) {
    if (bh < 0 || n < 0) return fail(HYQ_EINVAL, "hyq_dequant: negative shape");
    if (nbits != 2 && nbits != 4 && nbits != 8)
        return fail(HYQ_EINVAL, "nbits must be 2, 4, or 8, got " + std::to_string(nbits));
    if (!ok_dim(d)) return fail(HYQ_ENOTSUP, "hyq_dequant: head dim must be 8*2^k <= 512, got " + std::to_string(d));
    if (bh == 0 || n == 0) return HYQ_OK;
    if (!packed || !scale || !out) return fail(HYQ_EINVAL, "hyq_dequant: null pointer");
    const int pbytes = nbits;  // packed bytes per lane (8 channels)
    if (!aligned(packed, pbytes) || p_stride_n % pbytes || p_stride_bh % pbytes)
        return fail(HYQ_EINVAL, "hyq_dequant: packed input misaligned");
    if (!aligned(scale, 2)) return fail(HYQ_EINVAL, "hyq_dequant: scale misaligned");
    if (!aligned(out, 16) || o_stride_n % 8 || o_stride_bh % 8)
        return fail(HYQ_EINVAL, "hyq_dequant: out must be 16-byte aligned with strides divisible by 8");
    const int lpt_log2 = lanes_log2(d);
    const int64_t total = bh * n;
    const int64_t tpb = 256 >> lpt_log2;
    const int64_t blocks = (total + tpb - 1) / tpb;
    if (blocks > 0x7fffffffLL) return fail(HYQ_ENOTSUP, "hyq_dequant: too many tokens");
    hipStream_t s = static_cast<hipStream_t>(stream);
    dim3 grid(static_cast<unsigned>(blocks)), block(256);
    if (nbits == 4)
        dequant_kernel<4><<<grid, block, 0, s>>>(packed, n, total, lpt_log2, p_stride_bh, p_stride_n, scale, s_stride_bh,
                                                 out, o_stride_bh, o_stride_n);
    else if (nbits == 8)
        dequant_kernel<8><<<grid, block, 0, s>>>(packed, n, total, lpt_log2, p_stride_bh, p_stride_n, scale, s_stride_bh,
                                                 out, o_stride_bh, o_stride_n);
    else
        dequant_kernel<2><<<grid, block, 0, s>>>(packed, n, total, lpt_log2, p_stride_bh, p_stride_n, scale, s_stride_bh,
                                                 out, o_stride_bh, o_stride_n);
    return check_launch("hyq_dequant");
}

extern "C" int hyq_legacy_dequant(const uint8_t* packed, int64_t bh, int64_t n, int32_t d, int64_t p_stride_bh,
                                  int64_t p_stride_n, int32_t nbits, const uint16_t* scale, int64_t s_stride_bh,
                                  int64_t s_stride_g, int32_t group, uint16_t* out, int64_t o_stride_bh,
                                  int64_t o_stride_n, void* stream) {
    if (bh < 0 || n < 0) return fail(HYQ_EINVAL, "hyq_legacy_dequant: negative shape");
    if (nbits != 2 && nbits != 4) return fail(HYQ_EINVAL, "hyq_legacy_dequant: nbits must be 2 or 4, got " + std::to_string(nbits));
    if (!ok_dim(d)) return fail(HYQ_ENOTSUP, "hyq_legacy_dequant: head dim must be 8*2^k <= 512, got " + std::to_string(d));
    if (group <= 0) return fail(HYQ_EINVAL, "hyq_legacy_dequant: group must be positive");
    if (bh == 0 || n == 0) return HYQ_OK;
    if (!packed || !scale || !out) return fail(HYQ_EINVAL, "hyq_legacy_dequant: null pointer");
    const int pbytes = nbits;  // packed bytes per lane (8 channels)
    if (!aligned(packed, pbytes) || p_stride_n % pbytes || p_stride_bh % pbytes)
        return fail(HYQ_EINVAL, "hyq_legacy_dequant: packed input misaligned");
    if (!aligned(scale, 16) || s_stride_g % 8 || s_stride_bh % 8)
        return fail(HYQ_EINVAL, "hyq_legacy_dequant: scale rows must be 16-byte aligned with strides divisible by 8");
    if (!aligned(out, 16) || o_stride_n % 8 || o_stride_bh % 8)
        return fail(HYQ_EINVAL, "hyq_legacy_dequant: out must be 16-byte aligned with strides divisible by 8");
    const int lpt_log2 = lanes_log2(d);
    const int64_t total = bh * n;
    const int64_t tpb = 256 >> lpt_log2;
    const int64_t blocks = (total + tpb - 1) / tpb;
    if (blocks > 0x7fffffffLL) return fail(HYQ_ENOTSUP, "hyq_legacy_dequant: too many tokens");
    hipStream_t s = static_cast<hipStream_t>(stream);
    dim3 grid(static_cast<unsigned>(blocks)), block(256);
    if (nbits == 4)
        legacy_dequant_kernel<4><<<grid, block, 0, s>>>(packed, n, total, lpt_log2, p_stride_bh, p_stride_n, scale,
                                                        s_stride_bh, s_stride_g, group, out, o_stride_bh, o_stride_n);
    else
        legacy_dequant_kernel<2><<<grid, block, 0, s>>>(packed, n, total, lpt_log2, p_stride_bh, p_stride_n, scale,
                                                        s_stride_bh, s_stride_g, group, out, o_stride_bh, o_stride_n);
    return check_launch("hyq_legacy_dequant");
}
