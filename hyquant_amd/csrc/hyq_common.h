// Shared helpers for the gfx950 kernels of libhyq.so: status reporting,
// bit-exact bf16/fp16 conversions and wavefront-wide reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stdint.h>
#include <string>

#include "../../include/hyq.h"

namespace hyq {

void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

// ---- bit-exact conversions -------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// max over each aligned group of 16 lanes with DPP row operations (quad
// swaps, then the half-row and row mirrors), no LDS permute
__device__ __forceinline__ float max16_dpp(float v) {
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
    };
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0xb1>{}));    // quad_perm [1,0,3,2]
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x4e>{}));    // quad_perm [2,3,0,1]
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x141>{}));   // row_half_mirror
    v = fmaxf(v, dpp(v, std::integral_constant<int, 0x140>{}));   // row_mirror
    return v;
}

// Score maxima as plain v_max3_f32 / v_max_f32: fmaxf must quiet signalling
// NaNs, so the compiler puts a v_max_f32 x, x in front of every operand it
// cannot prove canonical (MFMA results, masked selects).  Attention scores
// are finite or -inf, never NaN.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
__device__ __forceinline__ float vmax2(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// sum over each aligned group of 16 lanes, the same four steps (each adds
// the value of a disjoint lane set: the pair, the other pair of the quad,
// the other quad of the half-row, the other half-row)
__device__ __forceinline__ float sum16_dpp(float v) {
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
    };
    v += dpp(v, std::integral_constant<int, 0xb1>{});
    v += dpp(v, std::integral_constant<int, 0x4e>{});
    v += dpp(v, std::integral_constant<int, 0x141>{});
    v += dpp(v, std::integral_constant<int, 0x140>{});
    return v;
}

// The correctly rounded fp32 quotient v / sf of a quantiser (finite sf > 0,
// |v| <= 128 sf) from inv = RN(1 / sf) computed once per row: q = RN(v inv),
// the residual r = v - q sf (exact by fma) and one fma correction
// (Markstein's correction step).  Checked against the IEEE division on the
// GPU for every finite fp16 scale and every bf16 and fp16 value in that
// range: every 2-, 4- and 8-bit code agrees.  Three VALU operations instead
// of the division sequence with a quarter-rate reciprocal per element.
__device__ __forceinline__ float quot_rn(float v, float sf, float inv) {
    const float q = v * inv;
    const float r = __builtin_fmaf(-q, sf, v);
    return __builtin_fmaf(r, inv, q);
}

// Scale and codes of one row of the K/V quantisers (bit-exact contract:
// s16 = fp16(amax / qmax), sf = fp32(s16), code = clamp(RNE(x / sf),
// -qmax - 1, qmax), amax already clamped at 1e-5), without IEEE divisions:
//   - fp16(amax * RN(1 / qmax)) equals fp16(amax / qmax) for every 16-bit amax
//     (all positive bf16 and fp16 patterns, clamped at 1e-5) and qmax = 7, 127
//     (checked exhaustively on the GPU; qmax = 1 is exact);
//   - RN(1 / sf) is v_rcp_f32(sf) with one Newton step for every finite fp16
//     sf (checked exhaustively on the GPU; the raw v_rcp_f32 differs for 2746
//     of the 31743 scales);
//   - x / sf by quot_rn, and the IEEE division where sf overflowed fp16;
//   - RNE(q) is the integer in the low mantissa bits of q + 1.5 * 2^23 (exact
//     for |q| < 2^22; here |q| <= 128), clamped as that bit pattern, whose
//     low NBITS bits are the two's-complement code.
// pat[i] holds code i in its low NBITS bits.
template <int NBITS>
__device__ __forceinline__ void quant_row_codes(const float (&v)[8], float amax, _Float16& s16, uint32_t (&pat)[8]) {
    constexpr int QMAX = (1 << (NBITS - 1)) - 1;
    constexpr int QMIN = -(1 << (NBITS - 1));
    constexpr float RQ = 1.0f / static_cast<float>(QMAX);     // RN(1 / qmax), folded at compile time
    constexpr int MAGIC = 0x4B400000;                          // bits of 1.5 * 2^23
    s16 = static_cast<_Float16>(amax * RQ);
    const float sf = static_cast<float>(s16);
    float q[8];
    if (sf <= 65504.0f) {
        const float r0 = __builtin_amdgcn_rcpf(sf);
        const float inv = __builtin_fmaf(__builtin_fmaf(-sf, r0, 1.0f), r0, r0);
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = quot_rn(v[i], sf, inv);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = v[i] / sf;
    }
    // The clamp only binds for 8 bits.  With qmax = 7 or 1, |x| <= amax and
    // amax >= 1e-5, sf is at most 2.1% below amax / qmax (fp16 subnormal
    // steps of 2^-24 against amax / qmax >= 1.43e-6, or 2^-11 relative for
    // normal scales; an overflowing scale gives q = 0), so |q| < 7.15 (int4)
    // or < 1.01 (int2) and RNE(q) is already within [qmin, qmax].  With
    // qmax = 127 a subnormal sf can leave q near 168.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int t = __float_as_int(q[i] + 12582912.0f);
        pat[i] = static_cast<uint32_t>(NBITS == 8 ? min(max(t, MAGIC + QMIN), MAGIC + QMAX) : t);
    }
}

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}

// round-to-nearest-even float -> bf16 bits (finite inputs; NaN stays NaN)
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<uint16_t>(u >> 16);
}

// One element of the legacy decode format (src/ops/d_stage_cache.py:1019-1045,
// :1063-1092) as bf16 bits: `twice` is twice the signed code value (2u - 16
// for int4, 2u - 3 for int2), `sb` the fp16 bits of its scale.  The product
// is formed in magnitude (exact in fp32), rounded once, and given the sign of
// the code times the scale, so a zero code with a negative scale is -0.
__device__ __forceinline__ uint32_t legacy_twice_to_bf16(int twice, uint32_t sb) {
    const float mag = 0.5f * static_cast<float>(twice < 0 ? -twice : twice) *
                      f16_bits_to_f32(static_cast<uint16_t>(sb & 0x7fffu));
    return f32_to_bf16_rne(mag) | ((twice < 0 ? 0x8000u : 0u) ^ (sb & 0x8000u));
}

// two floats -> packed bf16 pair (RNE), low half = a
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    bf16x2_t v = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
    return __builtin_bit_cast(uint32_t, v);
}

// packed fp16 pair -> packed bf16 pair, each value rounded to nearest even
// (an fp16 value is exact in float, so this is the one rounding of
// tensor.to(torch.bfloat16) / Triton's .to(tl.bfloat16))
__device__ __forceinline__ uint32_t f16x2_to_bf16x2(uint32_t w) {
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f16x2_t h = __builtin_bit_cast(f16x2_t, w);
    return pack_bf16x2(static_cast<float>(h[0]), static_cast<float>(h[1]));
}

// float -> fp16 bits, round to nearest even (overflow to inf)
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}

// round a float64 to float32 toward zero with a sticky bit (round-to-odd):
// a later RNE rounding of the result to any format of at most 22 significand
// bits equals one RNE rounding of x
__device__ __forceinline__ float f64_to_f32_odd(double x) {
    float f = __double2float_rz(x);
    uint32_t u = __float_as_uint(f);
    if (static_cast<double>(f) != x) u |= 1u;
    return __uint_as_float(u);
}

// float64 -> bf16 with one correct RNE rounding
__device__ __forceinline__ uint16_t f64_to_bf16_rne(double x) { return f32_to_bf16_rne(f64_to_f32_odd(x)); }

// float64 -> fp16 with one correct RNE rounding
__device__ __forceinline__ uint16_t f64_to_f16_rne(double x) { return f32_to_f16_bits(f64_to_f32_odd(x)); }

// ---- wavefront helpers (wave64) ---------------------------------------------

__device__ __forceinline__ float wave_xor_f32(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

}  // namespace hyq
