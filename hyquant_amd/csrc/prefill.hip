// Hybrid-precision causal prefill attention for gfx950 (MI355X).
//
// Semantics (sage_vertical_attention_v2, src/ops/sage_unified.py:550-622 with
// its kernel :398-496 and the per-block quantiser
// src/ops/vendor/sageattention/triton/quant_per_block.py:21-101):
//   c   = fp32(sm_scale * log2e)
//   Q   int8 per 128-row block of x = fp32(q) * c: scale = amax / 127,
//       code = trunc(x / scale + 0.5 * sign(x))          (F14)
//   q16 = fp16(bf16(x)); km = bf16 mean of k over the sequence (optional);
//   k16 = fp16(bf16(k - km)); v16 = fp16(v)
//   per query head: the clamped vertical indices sorted ascending (vert) and
//   the other positions of [0, N - W) ascending (rest); rest keys are
//   re-quantised to int8 per 64-entry block of the rest list (sm = 1).
//   For query block b (128 rows) with window start wla(b) = floor64(max(0,
//   128 b - (W - 1))), one base-2 online softmax runs over
//     rest entries < wla:  s = (q8 . k8) * (q_scale * k_scale)
//     vert entries < wla:  s = q16 . k16
//     keys wla <= j <= i:  s = q16 . k16                (causal, F13)
//   and O = sum p v16 / sum p, written as bf16.
//
// Launch sequence of hyq_prefill_hybrid (all on the caller's stream):
//   kv_stats_kernel / kv_final_kernel   per-channel K sum (fp64, fixed order)
//                                        -> km; per-channel |V| max (fp8 V scale)
//   kv_convert_kernel                   k16, v16 (and fp8 V) per KV head
//   lists_kernel                         per query head: sorted vertical list,
//                                        rest list, per-block counts (nr, nv)
//   gather_kernel                        rest K -> int8 per 64-block (+ scale),
//                                        rest V and vertical K/V rows per head
//   prefill_main_kernel                  one workgroup per (query block, head)
//
// prefill_main_kernel: 4 wavefronts, wavefront w owns query rows 32w..32w+31
// of the block as two 16-row sub-blocks (sb).  Q is quantised in the kernel
// (the workgroup is exactly one 128-row scale block) and kept in registers
// as MFMA B operands.  Keys stream in 64-key tiles straight from HBM into
// LDS (buffer loads to LDS, rows XOR-swizzled by 16-byte chunk), double
// buffered, one barrier per tile; the next tile's loads are issued right
// after that barrier and land while the current tile is computed.  Per tile
// and wavefront:
//   S^T = K . Q^T   rest tiles: v_mfma_i32_16x16x64_i8 (16 per tile), or
//                   with FP8 QK v_mfma_scale_f32_16x16x128_f8f6f4 (8);
//                   vert/window tiles: v_mfma_f32_16x16x32_f16 (32 per tile);
//                   output lane (c, g) holds keys 16kb + 4g + r of query c.
//   softmax         lazy running max (raised only when a tile exceeds it by
//                   more than 8 in log2 units), p = exp2(s - m).
//   O^T = V^T . P^T v_mfma_f32_16x16x32_f16 (32 per tile) with the V^T
//                   operand read from the row-major V tile by LDS transpose
//                   reads (ds_read_b64_tr_b16), and the row sums of P from
//                   one more MFMA against an all-ones operand; fp8 P.V uses
//                   v_mfma_f32_16x16x32_fp8_fp8 and ds_read_b64_tr_b8.
// Accumulation is fp32 throughout (the reference accumulates each 64-key
// P.V product in fp16).
#include "hyq_common.h"

#include <algorithm>
#include <cmath>
#include <string>
#include <utility>

namespace hyq {
namespace {

constexpr int PD = 128;                  // head_dim
constexpr int BM = 128;                  // query rows per block (Q scale block)
constexpr int BN = 64;                   // keys per tile (rest-K scale block)
constexpr int PF_THREADS = 256;
constexpr int RS8 = PD;                  // LDS bytes of an int8 / e4m3 tile row (K, fp8 V)
constexpr int RS16 = 2 * PD;             // LDS bytes of an fp16 tile row (K, V)
constexpr int TBUF = BN * RS16;          // bytes of one K or V tile buffer
constexpr float PF_SLACK = 8.0f;
constexpr float PF_M_INIT = -1.0e30f;
constexpr float FP8_MAX = 448.0f;        // src/ops/sage_unified_fp8.py:44
constexpr float S_FP8_OFFSET = 8.807f;   // vendor/sageattention/csrc/qattn/attn_utils.cuh:30 (log2 448)
constexpr int LIST_THREADS = 1024;
// The main kernel's buffer descriptors take 32-bit byte sizes and offsets:
// fp16 rows of 256 bytes (rest V, vertical rows, the window) stay below 2^32
// bytes per head up to 2^24 rows, so a head has at most 2^24 positions.
constexpr int64_t MAX_N = 1 << 24;        // sequence length per head
constexpr int64_t MAX_T = 1 << 24;        // vertical indices per head
constexpr int64_t MAX_P = 1 << 24;        // prefix positions N - W per head
constexpr int STAT_ROWS = 128;           // rows per kv_stats chunk

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

enum : int { T_REST = 0, T_VERT = 1, T_WIN = 2 };

// Raw buffer loads: the descriptor's range covers a tile source's valid rows,
// the row position travels in the scalar offset and the lane's place in the
// tile in the vector offset.  Loads at or past the range (scalar + vector
// offset >= range) return zeros, so no per-lane clamp or 64-bit address is
// formed.
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc pf_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// LDS DMA: 64 lanes x 16 bytes from a buffer (range checked) into 1 KiB of
// LDS at dst (wave-uniform), lane l at dst + 16 l; no VGPR holds the data
typedef __attribute__((address_space(3))) void* LdsPtr;
__device__ __forceinline__ void pf_dma16(Rsrc r, uint8_t* dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsPtr)(dst), 16, voff, soff, 0, 0);
}

// gfx950 LDS transpose reads: within each 16-lane group, lane j of
// ds_read_b64_tr_b16 receives element (j & 3) of the 8-byte pieces that lanes
// 4e + (j >> 2) address (e = 0..3), and lane j of ds_read_b64_tr_b8 receives
// byte (j & 7) of the pieces that lanes 2e + (j >> 3) address (e = 0..7).
// They are issued as inline asm: the compiler cannot tell which LDS object
// the intrinsic forms read, so it drains every in-flight LDS DMA (the next
// tile's) before them.  The asm reads are ordered after the step's barrier
// (volatile asm), and lds_wait ties their results to an explicit lgkmcnt
// wait before any use.
__device__ __forceinline__ uint32_t lds_addr(const uint8_t* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) const uint8_t*)(p)));
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_tr16(uint32_t addr) {
    u32x2 r;
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
template <int OFF>
__device__ __forceinline__ u32x2 lds_tr8(uint32_t addr) {
    u32x2 r;
    asm volatile("ds_read_b64_tr_b8 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
__device__ __forceinline__ void lds_wait(u32x2& a, u32x2& b, u32x2& c, u32x2& d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
// f(integral_constant<int, 0>) .. f(integral_constant<int, N - 1>): loop bodies
// whose index must be a compile-time constant (LDS read offsets are asm
// immediates)
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl(f, std::make_integer_sequence<int, N>{});
}
// 16-byte LDS reads in the same style (the K tile of the fp16 P.V loop)
template <int OFF>
__device__ __forceinline__ i32x4 lds_rd128(uint32_t addr) {
    i32x4 r;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
    return r;
}
// a copy the compiler cannot see through: per-lane offsets derived from it
// at their point of use are recomputed there rather than hoisted and held
// in registers through loops that do not need them
__device__ __forceinline__ uint32_t opaque_v(uint32_t x) {
    asm volatile("" : "+v"(x));
    return x;
}
__device__ __forceinline__ void lds_wait2(i32x4& a, i32x4& b) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void lds_wait4(i32x4& a, i32x4& b, i32x4& c, i32x4& d) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d));
}
__device__ __forceinline__ void lds_wait8(i32x4& a, i32x4& b, i32x4& c, i32x4& d, i32x4& e, i32x4& f, i32x4& g,
                                          i32x4& h) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f), "+v"(g), "+v"(h));
}


__device__ __forceinline__ int window_start(int blk, int W) {
    const int x = BM * blk - (W - 1);
    return (x > 0 ? x : 0) / BN * BN;
}

// quant_per_block_int8_kernel's rounding (quant_per_block.py:40-45): IEEE
// fp32 division, +-0.5 added in fp32, truncation toward zero.  A zero block
// (scale 0) gives code 0.
__device__ __forceinline__ int pb_code(float x, float scale) {
    if (!(scale > 0.0f)) return 0;
    float r = x / scale;
    r = r + (r >= 0.0f ? 0.5f : -0.5f);
    return static_cast<int>(r);
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xffu) | ((static_cast<uint32_t>(b) & 0xffu) << 8) |
           ((static_cast<uint32_t>(c) & 0xffu) << 16) | (static_cast<uint32_t>(d) << 24);
}

__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    const f16x2 v = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float bf16_round_f32(float x) { return bf16_to_f32(f32_to_bf16_rne(x)); }
// a bf16 or (f16 != 0) fp16 element -> float (exact)
__device__ __forceinline__ float half_to_f32(uint16_t h, int f16) {
    return f16 ? f16_bits_to_f32(h) : bf16_to_f32(h);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// max / sum over the four lanes c, c+16, c+32, c+48 (gfx950 row swaps)
__device__ __forceinline__ float quad_max(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float quad_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max of one sub-block's 16 scores of a tile (a tree of depth 3)
__device__ __forceinline__ float tile_max16(const float (&v)[4][4]) {
    const float a = vmax3(v[0][0], v[0][1], v[0][2]), b = vmax3(v[0][3], v[1][0], v[1][1]);
    const float c = vmax3(v[1][2], v[1][3], v[2][0]), d = vmax3(v[2][1], v[2][2], v[2][3]);
    const float e = vmax3(v[3][0], v[3][1], v[3][2]);
    return vmax2(vmax3(a, b, c), vmax3(d, e, v[3][3]));
}
// max over the four lanes c, c+16, c+32, c+48 with the same plain maxima
__device__ __forceinline__ float quad_max_raw(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = vmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return vmax2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// OCP e4m3 (gfx950 conversion, RNE), saturated to +-448 first
__device__ __forceinline__ uint32_t pack_e4m3x4(float a, float b, float c, float d) {
    auto cl = [](float x) { return fminf(fmaxf(x, -FP8_MAX), FP8_MAX); };
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(cl(a), cl(b), 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(cl(c), cl(d), r, true);
    return static_cast<uint32_t>(r);
}

// FP8-QK quantiser code of per_block_fp8_e4m3 (src/ops/sage_unified_fp8.py:
// 52-88): e4m3(clamp(x / scale, +-448)), IEEE fp32 division, round to
// nearest even.
__device__ __forceinline__ float fp8_ratio(float x, float scale) {
    return fminf(fmaxf(x / scale, -FP8_MAX), FP8_MAX);
}

// four values already inside [-448, 448] -> e4m3 codes (round to nearest
// even), no clamp: the FP8-QK ratios are clamped by fp8_ratio, and the P'
// operands exp2(s - m + 8.807 - guard) with the exact running max lie in
// [0, 447.98]
__device__ __forceinline__ uint32_t pack_e4m3x4_raw(float a, float b, float c, float d) {
    int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
    return static_cast<uint32_t>(r);
}

// ---------------------------------------------------------------------------
// K mean / V max statistics
// ---------------------------------------------------------------------------

// grid (ceil(N / 128), B*HKV); thread t: channels 2(t%64), 2(t%64)+1, rows
// chunk*128 + t/64 + 4i.  Partial sums are float64 and reduced in a fixed
// order, so km does not depend on scheduling.
__global__ __launch_bounds__(256) void kv_stats_kernel(const uint16_t* __restrict__ k, int64_t k_b, int64_t k_h,
                                                       int64_t k_n, const uint16_t* __restrict__ v, int64_t v_b,
                                                       int64_t v_h, int64_t v_n, int HKV, int N, int nch, int f16,
                                                       double* __restrict__ kpart, float* __restrict__ vpart) {
    __shared__ double s_sum[4][PD];
    __shared__ float s_max[4][PD];
    const int bhk = blockIdx.y, b = bhk / HKV, hk = bhk % HKV;
    const int chunk = blockIdx.x;
    const int cp = threadIdx.x & 63, ph = threadIdx.x >> 6;
    const uint16_t* kb = k + b * k_b + hk * k_h + 2 * cp;
    const uint16_t* vb = v + b * v_b + hk * v_h + 2 * cp;
    double s0 = 0.0, s1 = 0.0;
    float m0 = 0.0f, m1 = 0.0f;
    const int r_end = min(N, (chunk + 1) * STAT_ROWS);
    const int r0 = chunk * STAT_ROWS + ph;
    const int nr = r_end > r0 ? (r_end - r0 + 3) / 4 : 0;     // rows r0, r0 + 4, ...
    auto add = [&](uint32_t kk, uint32_t vv) {
        s0 += static_cast<double>(half_to_f32(static_cast<uint16_t>(kk), f16));
        s1 += static_cast<double>(half_to_f32(static_cast<uint16_t>(kk >> 16), f16));
        m0 = fmaxf(m0, fabsf(half_to_f32(static_cast<uint16_t>(vv), f16)));
        m1 = fmaxf(m1, fabsf(half_to_f32(static_cast<uint16_t>(vv >> 16), f16)));
    };
    // sixteen rows' loads in flight before their adds, which stay in row order
    int i = 0;
    for (; i + 16 <= nr; i += 16) {
        uint32_t kk[16], vv[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int64_t r = r0 + 4 * (i + j);
            kk[j] = *reinterpret_cast<const uint32_t*>(kb + r * k_n);
            vv[j] = *reinterpret_cast<const uint32_t*>(vb + r * v_n);
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) add(kk[j], vv[j]);
    }
    for (; i < nr; ++i) {
        const int64_t r = r0 + 4 * i;
        add(*reinterpret_cast<const uint32_t*>(kb + r * k_n), *reinterpret_cast<const uint32_t*>(vb + r * v_n));
    }
    s_sum[ph][2 * cp] = s0;
    s_sum[ph][2 * cp + 1] = s1;
    s_max[ph][2 * cp] = m0;
    s_max[ph][2 * cp + 1] = m1;
    __syncthreads();
    if (threadIdx.x < PD) {
        const int ch = threadIdx.x;
        const double s = ((s_sum[0][ch] + s_sum[1][ch]) + s_sum[2][ch]) + s_sum[3][ch];
        const float m = fmaxf(fmaxf(s_max[0][ch], s_max[1][ch]), fmaxf(s_max[2][ch], s_max[3][ch]));
        kpart[(static_cast<int64_t>(bhk) * nch + chunk) * PD + ch] = s;
        vpart[(static_cast<int64_t>(bhk) * nch + chunk) * PD + ch] = m;
    }
}

// grid (B*HKV), 128 threads: km = the model dtype's rounding of sum / N (one
// rounding of the float64 quotient), fp8 V scale = max|v| / 448.
__global__ __launch_bounds__(128) void kv_final_kernel(const double* __restrict__ kpart,
                                                       const float* __restrict__ vpart, int nch, int N, int smooth,
                                                       int f16, uint16_t* __restrict__ km, float* __restrict__ vscale) {
    const int bhk = blockIdx.x, ch = threadIdx.x;
    const double* kp = kpart + static_cast<int64_t>(bhk) * nch * PD + ch;
    const float* vp = vpart + static_cast<int64_t>(bhk) * nch * PD + ch;
    double s = 0.0;
    float m = 0.0f;
    // eight chunks' loads in flight, added in chunk order (the sum is the
    // same sequential float64 sum)
    int i = 0;
    for (; i + 8 <= nch; i += 8) {
        double a[8];
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            a[j] = kp[(i + j) * PD];
            x[j] = vp[(i + j) * PD];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            s += a[j];
            m = fmaxf(m, x[j]);
        }
    }
    for (; i < nch; ++i) {
        s += kp[i * PD];
        m = fmaxf(m, vp[i * PD]);
    }
    const double mean = s / static_cast<double>(N);
    km[bhk * PD + ch] = !smooth ? static_cast<uint16_t>(0) : f16 ? f64_to_f16_rne(mean) : f64_to_bf16_rne(mean);
    vscale[bhk * PD + ch] = m / FP8_MAX;
}

// grid (ceil(N*16 / 256), B*HKV): thread = 8 channels of one row.
//   bf16 model: k16 = fp16(bf16(k - km)); fp16 model: k16 = fp16(k - km)
//   (the difference in float32, rounded to the model dtype, then
//   .to(float16)); v16 = fp16(v); fp8 PV: v8 = e4m3(v / vscale) and
//   v16 = fp16(v / vscale)
__global__ __launch_bounds__(256) void kv_convert_kernel(const uint16_t* __restrict__ k, int64_t k_b, int64_t k_h,
                                                         int64_t k_n, const uint16_t* __restrict__ v, int64_t v_b,
                                                         int64_t v_h, int64_t v_n, int HKV, int N, int f16,
                                                         const uint16_t* __restrict__ km,
                                                         const float* __restrict__ vscale, uint16_t* __restrict__ k16,
                                                         uint16_t* __restrict__ v16, uint8_t* __restrict__ v8) {
    const int bhk = blockIdx.y, b = bhk / HKV, hk = bhk % HKV;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = idx >> 4;
    const int co = static_cast<int>(idx & 15);
    if (row >= N) return;
    const u32x4 kk = *reinterpret_cast<const u32x4*>(k + b * k_b + hk * k_h + row * k_n + 8 * co);
    const u32x4 vv = *reinterpret_cast<const u32x4*>(v + b * v_b + hk * v_h + row * v_n + 8 * co);
    // the 8 channel means in one 16-byte load (km rows are 256-byte aligned)
    const u32x4 mm = *reinterpret_cast<const u32x4*>(km + bhk * PD + 8 * co);
    float kf[8], vf[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t kw = kk[e >> 1], vw = vv[e >> 1], mw = mm[e >> 1];
        kf[e] = half_to_f32(static_cast<uint16_t>((e & 1) ? (kw >> 16) : kw), f16);
        vf[e] = half_to_f32(static_cast<uint16_t>((e & 1) ? (vw >> 16) : vw), f16);
        const float d = kf[e] - half_to_f32(static_cast<uint16_t>((e & 1) ? (mw >> 16) : mw), f16);
        kf[e] = f16 ? d : bf16_round_f32(d);     // pack_f16x2 below rounds to fp16
    }
    const int64_t o = (static_cast<int64_t>(bhk) * N + row) * PD + 8 * co;
    const u32x4 ko = {pack_f16x2(kf[0], kf[1]), pack_f16x2(kf[2], kf[3]), pack_f16x2(kf[4], kf[5]),
                      pack_f16x2(kf[6], kf[7])};
    const u32x4 vo = {pack_f16x2(vf[0], vf[1]), pack_f16x2(vf[2], vf[3]), pack_f16x2(vf[4], vf[5]),
                      pack_f16x2(vf[6], vf[7])};
    *reinterpret_cast<u32x4*>(k16 + o) = ko;
    if (v8 != nullptr) {
        // fp8 PV: e4m3(v / vscale) for the rest keys and fp16(v / vscale) for
        // the vertical and window keys, so that all tiles accumulate in one unit
        float q[8];
        const f32x4 vs0 = *reinterpret_cast<const f32x4*>(vscale + bhk * PD + 8 * co);
        const f32x4 vs1 = *reinterpret_cast<const f32x4*>(vscale + bhk * PD + 8 * co + 4);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float s = e < 4 ? vs0[e] : vs1[e - 4];
            q[e] = s > 0.0f ? vf[e] / s : 0.0f;
        }
        const u32x2 p = {pack_e4m3x4(q[0], q[1], q[2], q[3]), pack_e4m3x4(q[4], q[5], q[6], q[7])};
        *reinterpret_cast<u32x2*>(v8 + o) = p;
        const u32x4 qo = {pack_f16x2(q[0], q[1]), pack_f16x2(q[2], q[3]), pack_f16x2(q[4], q[5]), pack_f16x2(q[6], q[7])};
        *reinterpret_cast<u32x4*>(v16 + o) = qo;
    } else {
        *reinterpret_cast<u32x4*>(v16 + o) = vo;
    }
}

// ---------------------------------------------------------------------------
// rest / vertical lists (reorder_kv_for_vertical, sage_unified.py:499-547)
// ---------------------------------------------------------------------------

__device__ int block_exclusive_scan(int v, int* s_w) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    int x = v;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(x, o, 64);
        if (lane >= o) x += y;
    }
    if (lane == 63) s_w[w] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        int acc = 0;
        for (int i = 0; i < nw; ++i) {
            const int t = s_w[i];
            s_w[i] = acc;
            acc += t;
        }
        s_w[nw] = acc;
    }
    __syncthreads();
    return s_w[w] + x - v;
}

// grid (B*HQ), 1024 threads.  Per row: sorted list [n2], bitmap [nw], rest
// count before each word [nw], in dynamic LDS, or (GL) in this row's slice
// of a global scratch when they do not fit the LDS budget.
template <bool GL>
__global__ __launch_bounds__(LIST_THREADS) void lists_kernel(const int64_t* __restrict__ vidx, int64_t vi_b,
                                                             int64_t vi_h, int64_t vi_t, int HQ, int T, int n2,
                                                             int P, int nblk, int W, int32_t* __restrict__ vert,
                                                             int32_t* __restrict__ rest, int32_t* __restrict__ rcount,
                                                             int32_t* __restrict__ nr, int32_t* __restrict__ nv,
                                                             int* __restrict__ gscratch) {
    extern __shared__ int s_lists[];
    __shared__ int s_scan[LIST_THREADS / 64 + 1];
    const int nw = (P + 31) >> 5;
    const int bh = blockIdx.x, b = bh / HQ, h = bh % HQ;
    int* const lbase = GL ? gscratch + static_cast<int64_t>(bh) * (n2 + 2 * static_cast<int64_t>(nw)) : s_lists;
    int* s_sort = lbase;
    uint32_t* s_bm = reinterpret_cast<uint32_t*>(lbase + n2);
    int* s_pre = lbase + n2 + nw;
    const int tid = threadIdx.x;
    const int64_t* vrow = vidx + b * vi_b + h * vi_h;
    for (int i = tid; i < n2; i += LIST_THREADS) {
        int x = 0x7fffffff;
        if (i < T) {
            const int64_t y = vrow[i * vi_t];
            x = static_cast<int>(y < 0 ? 0 : (y > P - 1 ? P - 1 : y));
        }
        s_sort[i] = x;
    }
    for (int i = tid; i < nw; i += LIST_THREADS) s_bm[i] = 0u;
    __syncthreads();
    for (int kk = 2; kk <= n2; kk <<= 1) {
        for (int j = kk >> 1; j > 0; j >>= 1) {
            for (int i = tid; i < n2; i += LIST_THREADS) {
                const int ixj = i ^ j;
                if (ixj > i) {
                    const int a = s_sort[i], c = s_sort[ixj];
                    if ((a > c) == ((i & kk) == 0)) {
                        s_sort[i] = c;
                        s_sort[ixj] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    int32_t* vout = vert + static_cast<int64_t>(bh) * T;
    for (int i = tid; i < T; i += LIST_THREADS) {
        const int x = s_sort[i];
        vout[i] = x;
        atomicOr(&s_bm[x >> 5], 1u << (x & 31));
    }
    __syncthreads();
    // compaction of the unset bits of [0, P) in ascending order
    const int per = (nw + LIST_THREADS - 1) / LIST_THREADS;
    const int w0 = min(nw, tid * per), w1 = min(nw, w0 + per);
    auto free_bits = [&](int wi) {
        uint32_t m = ~s_bm[wi];
        const int tail = P - 32 * wi;
        if (tail < 32) m &= (1u << tail) - 1u;
        return m;
    };
    int cnt = 0;
    for (int wi = w0; wi < w1; ++wi) cnt += __popc(free_bits(wi));
    int off = block_exclusive_scan(cnt, s_scan);
    const int total = s_scan[LIST_THREADS >> 6];
    int32_t* rout = rest + static_cast<int64_t>(bh) * P;
    for (int wi = w0; wi < w1; ++wi) {
        s_pre[wi] = off;
        uint32_t m = free_bits(wi);
        while (m) {
            const int bit = __ffs(m) - 1;
            m &= m - 1u;
            rout[off++] = 32 * wi + bit;
        }
    }
    if (tid == 0) rcount[bh] = total;
    __syncthreads();
    for (int blk = tid; blk < nblk; blk += LIST_THREADS) {
        const int wla = window_start(blk, W);
        int lo = 0, hi = T;                      // first entry >= wla
        while (lo < hi) {
            const int mid = (lo + hi) >> 1;
            if (s_sort[mid] < wla) lo = mid + 1; else hi = mid;
        }
        const int wl = min(wla, P);
        int r;
        if (wl >= P) {
            r = total;
        } else {
            const int wi = wl >> 5, sh = wl & 31;
            r = s_pre[wi] + __popc(free_bits(wi) & ((1u << sh) - 1u));
        }
        nv[static_cast<int64_t>(bh) * nblk + blk] = lo;
        nr[static_cast<int64_t>(bh) * nblk + blk] = r;
    }
}

// grid (nsb + nvb, B*HQ), 256 threads.  Blocks [0, nsb): 64 entries of the
// rest list -> int8 K (per-64 block scale, sm = 1) and V rows (fp16 or fp8);
// blocks [nsb, nsb + nvb): 64 entries of the vertical list -> fp16 K and V.
// Thread t: row t/4 of the block, channels 32(t%4) .. +31.
__global__ __launch_bounds__(256) void gather_kernel(
    const uint16_t* __restrict__ k16, const uint16_t* __restrict__ v16, const uint8_t* __restrict__ v8, int HQ,
    int G, int HKV, int N, int P, int T, int nsb, const int32_t* __restrict__ rest,
    const int32_t* __restrict__ rcount, const int32_t* __restrict__ vert, int8_t* __restrict__ k8r,
    float* __restrict__ k8r_scale, uint8_t* __restrict__ vr, uint16_t* __restrict__ kv16,
    uint16_t* __restrict__ vv16, int k_fp8) {
    __shared__ float s_amax[4];
    const int bh = blockIdx.y, b = bh / HQ, h = bh % HQ;
    const int64_t bhk = static_cast<int64_t>(b) * HKV + h / G;
    const int tid = threadIdx.x, r = tid >> 2, qq = tid & 3;
    if (static_cast<int>(blockIdx.x) < nsb) {
        const int rc = rcount[bh];
        const int base = blockIdx.x * BN;
        if (base >= rc) return;                                 // uniform per block
        const int cnt = min(BN, rc - base);
        const bool ok = r < cnt;
        u32x4 kk[4] = {};
        if (ok) {
            const int pos = rest[static_cast<int64_t>(bh) * P + base + r];
            const uint16_t* src = k16 + (bhk * N + pos) * PD + 32 * qq;
#pragma unroll
            for (int i = 0; i < 4; ++i) kk[i] = reinterpret_cast<const u32x4*>(src)[i];
            const int64_t dst = (static_cast<int64_t>(bh) * P + base + r) * PD;
            // V rows are plain copies: 16-byte chunk qq + 4 i of the row, so
            // the four lanes of a row cover 64 contiguous bytes per instruction
            if (v8 != nullptr) {
                const u32x4* vs = reinterpret_cast<const u32x4*>(v8 + (bhk * N + pos) * PD);
                u32x4* vd = reinterpret_cast<u32x4*>(vr + dst);
                vd[qq] = vs[qq];
                vd[qq + 4] = vs[qq + 4];
            } else {
                const u32x4* vs = reinterpret_cast<const u32x4*>(v16 + (bhk * N + pos) * PD);
                u32x4* vd = reinterpret_cast<u32x4*>(vr + 2 * dst);
#pragma unroll
                for (int i = 0; i < 4; ++i) vd[qq + 4 * i] = vs[qq + 4 * i];
            }
        }
        float x[32];
        float amax = 0.0f;
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const uint32_t wv = kk[e >> 3][(e >> 1) & 3];
            x[e] = f16_bits_to_f32(static_cast<uint16_t>((e & 1) ? (wv >> 16) : wv));
            amax = fmaxf(amax, fabsf(x[e]));
        }
        amax = wave_max(amax);
        if ((tid & 63) == 0) s_amax[tid >> 6] = amax;
        __syncthreads();
        amax = fmaxf(fmaxf(s_amax[0], s_amax[1]), fmaxf(s_amax[2], s_amax[3]));
        // int8: amax / 127; e4m3 (FP8-QK): amax / 448, 1 for an all-zero block
        float scale = amax / (k_fp8 ? FP8_MAX : 127.0f);
        if (k_fp8 && !(scale > 0.0f)) scale = 1.0f;
        if (tid == 0) k8r_scale[static_cast<int64_t>(bh) * nsb + blockIdx.x] = scale;
        if (ok) {
            uint32_t wds[8];
#pragma unroll
            for (int i = 0; i < 8; ++i)
                wds[i] = k_fp8 ? pack_e4m3x4_raw(fp8_ratio(x[4 * i], scale), fp8_ratio(x[4 * i + 1], scale),
                                               fp8_ratio(x[4 * i + 2], scale), fp8_ratio(x[4 * i + 3], scale))
                               : pack4_i8(pb_code(x[4 * i], scale), pb_code(x[4 * i + 1], scale),
                                          pb_code(x[4 * i + 2], scale), pb_code(x[4 * i + 3], scale));
            u32x4* dst = reinterpret_cast<u32x4*>(k8r + (static_cast<int64_t>(bh) * P + base + r) * PD + 32 * qq);
            dst[0] = u32x4{wds[0], wds[1], wds[2], wds[3]};
            dst[1] = u32x4{wds[4], wds[5], wds[6], wds[7]};
        }
    } else {
        const int base = (blockIdx.x - nsb) * BN;
        if (base + r >= T) return;
        const int pos = vert[static_cast<int64_t>(bh) * T + base + r];
        const u32x4* ks = reinterpret_cast<const u32x4*>(k16 + (bhk * N + pos) * PD);
        const u32x4* vs = reinterpret_cast<const u32x4*>(v16 + (bhk * N + pos) * PD);
        const int64_t dst = (static_cast<int64_t>(bh) * T + base + r) * PD;
        u32x4* kd = reinterpret_cast<u32x4*>(kv16 + dst);
        u32x4* vd = reinterpret_cast<u32x4*>(vv16 + dst);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            kd[qq + 4 * i] = ks[qq + 4 * i];
            vd[qq + 4 * i] = vs[qq + 4 * i];
        }
    }
}

// ---------------------------------------------------------------------------
// per-block int8 quantiser (per_block_int8, quant_per_block.py:49-101)
// ---------------------------------------------------------------------------

// grid (ceil(L / blk), H, B), 256 threads; thread t handles channels
// 8(t%16)..+7 of rows t/16, t/16 + 16, ...  x = fp32(bf16(in - km)) * sm
// (km optional; in bf16 or fp16).
__global__ __launch_bounds__(256) void per_block_int8_kernel(const uint16_t* __restrict__ in, int is_fp16,
                                                             int64_t i_b, int64_t i_h, int64_t i_n, int L, int blk,
                                                             float sm, const uint16_t* __restrict__ km,
                                                             int64_t km_b, int64_t km_h, int8_t* __restrict__ out,
                                                             int64_t o_b, int64_t o_h, int64_t o_n,
                                                             float* __restrict__ scale, int64_t s_b, int64_t s_h) {
    __shared__ float s_amax[4];
    const int bi = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, co = tid & 15, r0 = tid >> 4;
    const uint16_t* src = in + b * i_b + h * i_h + 8 * co;
    float kmv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) kmv[e] = km ? bf16_to_f32(km[b * km_b + h * km_h + 8 * co + e]) : 0.0f;
    float amax = 0.0f;
    const int row_end = min(L, (bi + 1) * blk);
    auto value = [&](uint32_t w, int e) {
        const uint16_t bits = static_cast<uint16_t>((e & 1) ? (w >> 16) : w);
        float x = is_fp16 ? f16_bits_to_f32(bits) : bf16_to_f32(bits);
        if (km) x = bf16_round_f32(x - kmv[e]);
        return x * sm;
    };
    for (int r = bi * blk + r0; r < row_end; r += 16) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(src + r * i_n);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(value(w[e >> 1], e)));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) s_amax[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(s_amax[0], s_amax[1]), fmaxf(s_amax[2], s_amax[3]));
    const float sc = amax / 127.0f;
    if (tid == 0) scale[b * s_b + h * s_h + bi] = sc;
    for (int r = bi * blk + r0; r < row_end; r += 16) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(src + r * i_n);
        int c[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) c[e] = pb_code(value(w[e >> 1], e), sc);
        const u32x2 o = {pack4_i8(c[0], c[1], c[2], c[3]), pack4_i8(c[4], c[5], c[6], c[7])};
        *reinterpret_cast<u32x2*>(out + b * o_b + h * o_h + r * o_n + 8 * co) = o;
    }
}

// ---------------------------------------------------------------------------
// main attention kernel
// ---------------------------------------------------------------------------

struct PfArgs {
    const uint16_t* q; int64_t q_b, q_h, q_n;
    uint16_t* out; int64_t o_b, o_h, o_n;
    const int8_t* k8r; const float* k8r_scale; const uint16_t* vr;   // rest, per query head [BH][P][128]
    const uint16_t* kv16; const uint16_t* vv16;                      // vertical, per query head [BH][T][128]
    const uint16_t* k16; const uint16_t* v16;                        // window source, per KV head [BHK][N][128]
    const int32_t* nr; const int32_t* nv;                            // [BH][nblk]
    int B, HQ, HKV, N, nblk, W, P, T, nsb;
    float c;                                                          // fp32(sm_scale * log2e)
    int total, per_xcd;
    const float* vscale;                                              // fp8 PV: [BHK][128] per-channel V scale
    int rest_causal;       // all keys int8 up to the diagonal (rest list = positions, causal mask, no window)
    int f16;               // q and out are fp16 (an fp16 model), else bf16
};

__device__ __forceinline__ f32x4 mfma_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ i32x4 mfma_i8(const i32x4& a, const i32x4& b, const i32x4& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// 16 x 16 x 128 e4m3 product (format 0 on both sides, unit block scales:
// e8m0 127 = 2^0)
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
__device__ __forceinline__ f32x4 mfma_f8_k128(const i32x8& a, const i32x8& b) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0, 127, 0,
                                                            127);
}
__device__ __forceinline__ f32x4 mfma_fp8(const u32x2& a, const u32x2& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(__builtin_bit_cast(long, a), __builtin_bit_cast(long, b), c, 0, 0, 0);
}

// PV8: fp8 PV on the rest tiles (P' = exp2(s - m + 8.807) as e4m3 against
// e4m3(v / vscale)); the vertical and window tiles keep fp16 operands in the
// same units (fp16(P'), fp16(v / vscale)); the epilogue multiplies by vscale.
// The running max is exact in this mode (no lazy slack), so P' <= 448.
// QF8: the rest tiles score Q and K in OCP e4m3 (sage_vertical_attention_v2_fp8,
// src/ops/sage_unified_fp8.py:158-311): Q per 128-row block and rest K per
// 64-entry block with scale amax / 448 (1 for an all-zero block), one
// v_mfma_scale_f32_16x16x128_f8f6f4 per 16 keys over all 128 channels (the
// lane's 32 channels are the same 16 + 16 bytes the int8 path splits over
// two MFMAs; Q and K use the same channel order, so the dot product is whole).
template <bool PV8, bool QF8>
__global__ __launch_bounds__(PF_THREADS, 2) void prefill_main_kernel(PfArgs a) {
    // two tile buffers as four distinct LDS objects: the compiler then knows a
    // DMA into one buffer cannot alias reads of the other and does not drain
    // the next tile's DMAs before computing the current one
    __shared__ __attribute__((aligned(16))) uint8_t s_k0[TBUF];
    __shared__ __attribute__((aligned(16))) uint8_t s_k1[TBUF];
    __shared__ __attribute__((aligned(16))) uint8_t s_v0[TBUF];
    __shared__ __attribute__((aligned(16))) uint8_t s_v1[TBUF];
    __shared__ float s_red[4];

    // XCD-aware order: consecutive items (same head, heaviest block first) land on one XCD
    const int wg = blockIdx.x;
    const int item = (wg & 7) * a.per_xcd + (wg >> 3);
    if (item >= a.total) return;
    const int bh = item / a.nblk;
    const int blk = a.nblk - 1 - (item - bh * a.nblk);
    const int b = bh / a.HQ, h = bh - b * a.HQ;
    const int G = a.HQ / a.HKV;
    const int64_t bhk = static_cast<int64_t>(b) * a.HKV + h / G;
    // the wavefront index is uniform: read into a scalar register, so the LDS
    // DMA destinations and scalar offsets built from it need no per-lane
    // (waterfall) loop
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c16 = lane & 15, g = lane >> 4;

    // ---- Q block: load, quantise (int8 per block scale), fp16 copy --------
    // q * c of sub-block sb, channels 64 cc + 16 g .. + 15 of row c16 (zeros
    // past the last row)
    auto q_chunk = [&](const uint16_t* qbase, int cr, int gr, int sb, int cc, float (&xv)[16])
                       __attribute__((always_inline)) {
        const int row = BM * blk + 32 * w + 16 * sb + cr;
        const bool ok = row < a.N;
        const uint16_t* qrow = qbase + b * a.q_b + h * a.q_h + static_cast<int64_t>(ok ? row : 0) * a.q_n;
        u32x4 lo = {}, hi = {};
        if (ok) {
            lo = *reinterpret_cast<const u32x4*>(qrow + 64 * cc + 16 * gr);
            hi = *reinterpret_cast<const u32x4*>(qrow + 64 * cc + 16 * gr + 8);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const uint32_t wd = (e < 8) ? lo[e >> 1] : hi[(e - 8) >> 1];
            xv[e] = half_to_f32(static_cast<uint16_t>((e & 1) ? (wd >> 16) : wd), a.f16) * a.c;
        }
    };
    // the fp16 operand of the fp16 tiles: q_scaled = (q * c) in the model
    // dtype, then .to(float16) (a bf16 model rounds twice, an fp16 model once)
    f16x8 qh[2][4];
    auto make_qh = [&](int sb, int cc, const float (&xv)[16]) __attribute__((always_inline)) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const float* z = xv + 8 * hf;
            float zr[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) zr[e] = a.f16 ? z[e] : bf16_round_f32(z[e]);
            const u32x4 hv = {pack_f16x2(zr[0], zr[1]), pack_f16x2(zr[2], zr[3]), pack_f16x2(zr[4], zr[5]),
                              pack_f16x2(zr[6], zr[7])};
            qh[sb][2 * cc + hf] = __builtin_bit_cast(f16x8, hv);
        }
    };
    float x[2][2][16];
    float amax = 0.0f;
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            q_chunk(a.q, c16, g, sb, cc, x[sb][cc]);
#pragma unroll
            for (int e = 0; e < 16; ++e) amax = fmaxf(amax, fabsf(x[sb][cc][e]));
        }
    amax = wave_max(amax);
    if (lane == 0) s_red[w] = amax;
    __syncthreads();
    // uniform over the workgroup: held in a scalar register, so that the score
    // scale below and every test on it stay scalar (no per-lane branches)
    const float q_amax = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int,
        fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3])))));
    float q_scale = q_amax / (QF8 ? FP8_MAX : 127.0f);
    if (QF8 && !(q_scale > 0.0f)) q_scale = 1.0f;
    i32x4 q8[2][2];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const float* xv = x[sb][cc];
            uint32_t wd[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                wd[i] = QF8 ? pack_e4m3x4_raw(fp8_ratio(xv[4 * i], q_scale), fp8_ratio(xv[4 * i + 1], q_scale),
                                            fp8_ratio(xv[4 * i + 2], q_scale), fp8_ratio(xv[4 * i + 3], q_scale))
                            : pack4_i8(pb_code(xv[4 * i], q_scale), pb_code(xv[4 * i + 1], q_scale),
                                       pb_code(xv[4 * i + 2], q_scale), pb_code(xv[4 * i + 3], q_scale));
            q8[sb][cc] = i32x4{static_cast<int>(wd[0]), static_cast<int>(wd[1]), static_cast<int>(wd[2]),
                               static_cast<int>(wd[3])};
            // the fp16 P.V kernels build this copy after the rest tiles (it
            // is not held in registers through them)
            if constexpr (PV8) make_qh(sb, cc, x[sb][cc]);
        }
    }

    // ---- tile schedule -------------------------------------------------------
    int nr_b = a.nr[static_cast<int64_t>(bh) * a.nblk + blk];
    const int nv_b = a.nv[static_cast<int64_t>(bh) * a.nblk + blk];
    int wla = window_start(blk, a.W);
    const int wend = min(a.N, BM * (blk + 1));
    if (a.rest_causal) {        // the rest list is every position: int8 through the diagonal block
        nr_b = wend;
        wla = wend;
    }
    const int nrt = (nr_b + BN - 1) / BN;
    const int nvt = (nv_b + BN - 1) / BN;
    const int nwt = (wend - wla + BN - 1) / BN;
    const int ntiles = nrt + nvt + nwt;
    const float* ksc_row = a.k8r_scale + static_cast<int64_t>(bh) * a.nsb;

    // Tiles go from HBM straight into LDS (LDS DMA, no register staging).
    // Rows are stored whole, 128 B (int8 / e4m3) or 256 B (fp16), with
    // their 16-byte chunks XOR-swizzled by row so that the reads below hit
    // distinct banks; the swizzle is applied on the load side (each DMA lane
    // picks the global chunk that belongs at its LDS position):
    //   K int8 / e4m3   position = chunk ^ (row & 7)
    //   K fp16          position = chunk ^ (row & 15)
    //   V fp16          position = chunk ^ 2 (row & 7)   (fp16 P.V kernels)
    //                   position = chunk ^ 2 (row & 3)   (fp8 P.V kernel)
    //   V e4m3          position = chunk ^ ((row & 3) | 4 ((row >> 4) & 1))
    // One DMA writes 1 KiB: 8 rows of 128 B or 4 rows of 256 B; wavefront w
    // issues DMAs q = 2w, 2w + 1 (128-B rows) or q = 4w .. 4w + 3 (256-B
    // rows).  Rows past a source's valid rows read zeros (their scores are
    // masked and their P is zero).
    const uint32_t dk8 = static_cast<uint32_t>((lane >> 3) * RS8 + 16 * ((lane & 7) ^ (lane >> 3)));
    const uint32_t dk16 = static_cast<uint32_t>((lane >> 4) * RS16 + 16 * ((lane & 15) ^ (lane >> 4)));
    // (fp16 V with fp16 P.V: the 8 rows a 32-lane half of each transpose read
    // touches sit on 8 distinct bank groups; DMA q writes rows 4q .. 4q + 3,
    // so row & 7 is 4 (q & 1) + (lane >> 4) and the odd DMAs take this
    // offset with 128 XOR-ed in)
    const uint32_t dv16 = static_cast<uint32_t>((lane >> 4) * RS16 + 16 * ((lane & 15) ^ (2 * ((lane >> 4) & 3))));
    const uint32_t dv8 = static_cast<uint32_t>((lane >> 3) * RS8 +
                                               16 * ((lane & 7) ^ (((lane >> 3) & 3) | ((w & 1) << 2))));
    float m_run[2] = {PF_M_INIT, PF_M_INIT};
    // softmax denominators: PV8 sums P' on the VALU (l_run, per lane, summed
    // over the quad at the end); fp16 PV sums the fp16 P operands with one
    // more MFMA per 32 keys against an all-ones A (lsum, every lane holds its
    // column's full sum), which takes 32 adds per tile off the VALU
    float l_run[2] = {0.0f, 0.0f};
    f32x4 lsum[2] = {f32x4{0.0f, 0.0f, 0.0f, 0.0f}, f32x4{0.0f, 0.0f, 0.0f, 0.0f}};
    // fp16 P.V: O^T in 16 x 16 blocks [sub-block][16 channels] (lane (c, g):
    // row c of the sub-block, channels 16 cb + 4 g + 0..3)
    f32x4 acc[2][8];
#pragma unroll
    for (int sb = 0; sb < 2; ++sb)
#pragma unroll
        for (int cb = 0; cb < 8; ++cb) acc[sb][cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // fp8 P.V: O^T in 32 x 32 blocks of 32 channels (lane l: row l % 32 of
    // the wavefront, channels 32 cbk + 8 (i >> 2) + 4 (l >> 5) + (i & 3) in
    // register i), the layout of v_mfma_scale_f32_32x32x64_f8f6f4
    f32x16 acc32[4];
#pragma unroll
    for (int cbk = 0; cbk < 4; ++cbk)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc32[cbk][i] = 0.0f;

    {
        // ---- the tiles as three runs, each its own loop ---------------------
        // Tiles t < nrt are rest tiles, then nvt vertical tiles, then nwt
        // window tiles.  A run fixes its kind at compile time and its K / V
        // sources (buffer resources) before its loop, so a tile costs only its
        // DMA offsets: no per-tile source selection, no reload of kernel
        // arguments, no scalar-memory load whose wait would also drain the LDS
        // reads (the rest tiles' k_scale arrives by a vector load a tile ahead,
        // under the tile's DMA wait).  Tile t uses buffer pair t & 1 (chosen at
        // run time: the K and V reads are inline asm, so the compiler does not
        // order them after the other buffer's in-flight DMAs); the last tile of
        // a run prefetches the next run's first tile.
        const Rsrc rsc = pf_rsrc(ksc_row, static_cast<uint32_t>(nrt) * 4u);
        auto sources = [&](auto KT, Rsrc& rk, Rsrc& rv) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            if constexpr (KIND == T_REST) {
                rk = pf_rsrc(a.k8r + static_cast<int64_t>(bh) * a.P * PD, static_cast<uint32_t>(nr_b) * RS8);
                if constexpr (PV8)     // e4m3 V rows of 128 bytes
                    rv = pf_rsrc(reinterpret_cast<const uint8_t*>(a.vr) + static_cast<int64_t>(bh) * a.P * PD,
                                 static_cast<uint32_t>(nr_b) * RS8);
                else
                    rv = pf_rsrc(a.vr + static_cast<int64_t>(bh) * a.P * PD, static_cast<uint32_t>(nr_b) * RS16);
            } else if constexpr (KIND == T_VERT) {
                rk = pf_rsrc(a.kv16 + static_cast<int64_t>(bh) * a.T * PD, static_cast<uint32_t>(nv_b) * RS16);
                rv = pf_rsrc(a.vv16 + static_cast<int64_t>(bh) * a.T * PD, static_cast<uint32_t>(nv_b) * RS16);
            } else {
                rk = pf_rsrc(a.k16 + bhk * a.N * PD, static_cast<uint32_t>(wend) * RS16);
                rv = pf_rsrc(a.v16 + bhk * a.N * PD, static_cast<uint32_t>(wend) * RS16);
            }
        };
        // first key (window) or list entry (rest, vertical) of tile t of run KIND
        auto first_of = [&](auto KT, int t) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            if constexpr (KIND == T_REST) return BN * t;
            else if constexpr (KIND == T_VERT) return BN * (t - nrt);
            else return wla + BN * (t - nrt - nvt);
        };
        // the K DMAs and the V DMAs of one tile into buffer par
        auto issue_k = [&](auto KT, const Rsrc& rk, int i0, int par) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            uint8_t* kd = par ? s_k1 : s_k0;
            const uint32_t r0 = static_cast<uint32_t>(i0);
            if constexpr (KIND == T_REST) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int q = 2 * w + i;
                    pf_dma16(rk, kd + 1024 * q, dk8, r0 * RS8 + 1024 * q);
                }
            } else {
                // DMA q = 4 w + i writes rows 4 q + (lane >> 4), whose row & 15
                // is 4 i + (lane >> 4): the source chunk is (lane & 15) ^
                // (lane >> 4) ^ 4 i, i.e. the offset of i = 0 with 64 i
                // XOR-ed in (recomputed here, not held through other runs)
                const uint32_t vo0 = opaque_v(dk16);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int q = 4 * w + i;
                    pf_dma16(rk, kd + 1024 * q, vo0 ^ (64u * i), r0 * RS16 + 1024 * q);
                }
            }
        };
        auto issue_v = [&](auto KT, const Rsrc& rv, int i0, int par) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            uint8_t* vd = par ? s_v1 : s_v0;
            const uint32_t r0 = static_cast<uint32_t>(i0);
            if constexpr (PV8 && KIND == T_REST) {
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int q = 2 * w + i;
                    pf_dma16(rv, vd + 1024 * q, dv8, r0 * RS8 + 1024 * q);
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int q = 4 * w + i;
                    pf_dma16(rv, vd + 1024 * q, (!PV8 && (i & 1)) ? (dv16 ^ 128u) : dv16, r0 * RS16 + 1024 * q);
                }
            }
        };
        auto issue = [&](auto KT, const Rsrc& rk, const Rsrc& rv, int i0, int par) __attribute__((always_inline)) {
            issue_k(KT, rk, i0, par);
            issue_v(KT, rv, i0, par);
        };
        // the first tile of the run after KIND (the rare cross-run prefetch)
        auto issue_next_run = [&](auto KT, int t, int par) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            Rsrc rk, rv;
            if constexpr (KIND == T_REST) {
                if (t < nrt + nvt) {
                    sources(std::integral_constant<int, T_VERT>{}, rk, rv);
                    issue(std::integral_constant<int, T_VERT>{}, rk, rv, first_of(std::integral_constant<int, T_VERT>{}, t), par);
                    return;
                }
            }
            if constexpr (KIND != T_WIN) {
                sources(std::integral_constant<int, T_WIN>{}, rk, rv);
                issue(std::integral_constant<int, T_WIN>{}, rk, rv, first_of(std::integral_constant<int, T_WIN>{}, t), par);
            }
        };

        // per-lane LDS byte offsets of the reads within a buffer
        //   rest K (128-B rows):   chunk g and 4 + g of row 16 kb + c16
        //   fp16 K (256-B rows):   chunk 8 (m >> 1) + 2g + (m & 1) of row 16 kb + c16
        //   fp16 V (transposed):   the lds_tr16 addressing of channel block cb
        const uint32_t ok8a = c16 * RS8 + 16 * (g ^ (c16 & 7));
        // (ok16 of chunk 8 (m >> 1) + 2g + (m & 1) is that of m = 0 with
        // 16 (m & 1) + 128 (m >> 1) XOR-ed in)
        const uint32_t ok16 = c16 * RS16 + 16 * ((2 * g) ^ c16);
        // (row 4 g + (c16 >> 2) + 16 k: chunk 2 cb + ((c16 & 3) >> 1) stored at
        // chunk ^ 2 (row & 7); block cb is block 0 with 32 cb XOR-ed in)
        const uint32_t ov0 = (4 * g + (c16 >> 2)) * RS16 + 8 * (c16 & 1) +
                             16 * (((c16 & 3) >> 1) ^ (2 * ((4 * g + (c16 >> 2)) & 7)));
        // fp8 P.V kernel, vertical / window tiles: the V^T operand of
        // v_mfma_f32_32x32x16_f16 (32 channels x 16 keys): lane l = 16 G + j
        // receives channel 32 cbk + 16 (G & 1) + j of keys 16 kb + 8 (G >> 1) +
        // 4 rd + e (e = 0..3) from read rd; as the addressing lane a = j it
        // names row 16 kb + 8 (G >> 1) + 4 rd + (a >> 2), channels 32 cbk +
        // 16 (G & 1) + 4 (a & 3) .. + 3, in chunk 4 cbk + 2 (G & 1) + ((a & 3) >> 1)
        // stored at chunk ^ 2 (row & 3).  Blocks cbk and cbk + 2 differ by a
        // constant 128 bytes, kb and rd by whole rows.
        uint32_t ovh[2];
#pragma unroll
        for (int cbk = 0; cbk < 2; ++cbk)
            ovh[cbk] = (8 * (g >> 1) + (c16 >> 2)) * RS16 + 8 * (c16 & 1) +
                       16 * ((4 * cbk + 2 * (g & 1) + ((c16 & 3) >> 1)) ^ (2 * (c16 >> 2)));
        // fp8 P.V kernel, rest tiles: the V^T operand of
        // v_mfma_scale_f32_32x32x64_f8f6f4 (32 channels x 64 keys, e4m3): byte
        // i of lane l holds channel 32 cbk + l % 32 of key kp(i) + 8 (l >> 5),
        // kp(i) = 16 (i >> 2) + (i & 3) for i < 16 and 16 ((i - 16) >> 2) + 4 +
        // (i & 3) above (the key order of P after the row swap below).  Read rd
        // (ds_read_b64_tr_b8) fills bytes 8 rd .. 8 rd + 7: the addressing lane
        // a = j of group G names key kb0(rd) + 16 (a >> 3) + ((a >> 1) & 3) +
        // 8 (G >> 1), kb0 = 0, 32, 4, 36, channels 32 cbk + 16 (G & 1) + 8 (a & 1)
        // .. + 7: chunk 2 cbk + (G & 1), stored at chunk ^ (a >> 1) (the e4m3 V
        // swizzle: (row & 3) | 4 ((row >> 4) & 1) is a >> 1 for these rows).
        uint32_t ov8[4];
#pragma unroll
        for (int cbk = 0; cbk < 4; ++cbk)
            ov8[cbk] = (16 * (c16 >> 3) + ((c16 >> 1) & 3) + 8 * (g >> 1)) * RS8 + 8 * (c16 & 1) +
                       16 * ((2 * cbk + (g & 1)) ^ (c16 >> 1));
        const uint32_t kbase[2] = {lds_addr(s_k0), lds_addr(s_k1)};
        const uint32_t vbase[2] = {lds_addr(s_v0), lds_addr(s_v1)};
        const u32x4 onew = {0x3c003c00u, 0x3c003c00u, 0x3c003c00u, 0x3c003c00u};   // fp16 1.0

        // S^T = K . Q^T of a rest tile (int8 or e4m3) from K at kb; the fp8
        // P.V kernel reads the whole K block at once, the fp16 P.V kernels
        // (whose pipelined steps hold two score tiles) key block kbk + 1
        // during the MFMAs of kbk
        // (RT: int8 scores stay raw int32 bits in s, converted by the caller)
        auto qk_rest_t = [&](auto RT, uint32_t kb, float (&s)[2][4][4]) __attribute__((always_inline)) {
            // (chunk 4 + g is chunk g with 64 bytes XOR-ed in)
            const uint32_t aa = kb + ok8a, ab = kb + (opaque_v(ok8a) ^ 64u);
            auto mm = [&](int kbk, const i32x4& k0, const i32x4& k1) __attribute__((always_inline)) {
                if constexpr (QF8) {
                    const i32x8 av = {k0[0], k0[1], k0[2], k0[3], k1[0], k1[1], k1[2], k1[3]};
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb) {
                        const i32x8 bv = {q8[sb][0][0], q8[sb][0][1], q8[sb][0][2], q8[sb][0][3],
                                          q8[sb][1][0], q8[sb][1][1], q8[sb][1][2], q8[sb][1][3]};
                        const f32x4 sf = mfma_f8_k128(av, bv);
#pragma unroll
                        for (int r = 0; r < 4; ++r) s[sb][kbk][r] = sf[r];
                    }
                } else {
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb) {
                        i32x4 si = mfma_i8(k0, q8[sb][0], i32x4{0, 0, 0, 0});
                        si = mfma_i8(k1, q8[sb][1], si);
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            // (the element is copied out first: a bit cast of a
                            // vector element in place reads element 0)
                            const int sr = si[r];
                            s[sb][kbk][r] = decltype(RT)::value ? __builtin_bit_cast(float, sr) : static_cast<float>(sr);
                        }
                    }
                }
            };
            if constexpr (PV8) {
                i32x4 ka[4][2];
                ka[0][0] = lds_rd128<0 * 16 * RS8>(aa); ka[0][1] = lds_rd128<0 * 16 * RS8>(ab);
                ka[1][0] = lds_rd128<1 * 16 * RS8>(aa); ka[1][1] = lds_rd128<1 * 16 * RS8>(ab);
                ka[2][0] = lds_rd128<2 * 16 * RS8>(aa); ka[2][1] = lds_rd128<2 * 16 * RS8>(ab);
                ka[3][0] = lds_rd128<3 * 16 * RS8>(aa); ka[3][1] = lds_rd128<3 * 16 * RS8>(ab);
                lds_wait8(ka[0][0], ka[0][1], ka[1][0], ka[1][1], ka[2][0], ka[2][1], ka[3][0], ka[3][1]);
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk) mm(kbk, ka[kbk][0], ka[kbk][1]);
            } else {
                i32x4 ka[2][2];        // [stage][half]
                auto rd = [&](auto KBT, int st) __attribute__((always_inline)) {
                    constexpr int OFF = 16 * RS8 * decltype(KBT)::value;
                    ka[st][0] = lds_rd128<OFF>(aa);
                    ka[st][1] = lds_rd128<OFF>(ab);
                };
                rd(std::integral_constant<int, 0>{}, 0);
                static_for<4>([&](auto KBT) __attribute__((always_inline)) {
                    constexpr int kbk = decltype(KBT)::value, st = kbk & 1;
                    lds_wait2(ka[st][0], ka[st][1]);
                    if constexpr (kbk + 1 < 4) rd(std::integral_constant<int, kbk + 1>{}, st ^ 1);
                    mm(kbk, ka[st][0], ka[st][1]);
                });
            }
        };
        auto qk_rest = [&](uint32_t kb, float (&s)[2][4][4]) __attribute__((always_inline)) {
            qk_rest_t(std::false_type{}, kb, s);
        };
        // S^T = K . Q^T of an fp16 tile (vertical, window) from K at kb; the
        // reads of key block kbk + 1 in flight during the MFMAs of kbk
        auto qk_f16 = [&](uint32_t kb, float (&s)[2][4][4]) __attribute__((always_inline)) {
            f32x4 sf[2][4];
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk) sf[sb][kbk] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            i32x4 kr[2][4];
            const uint32_t o0 = opaque_v(ok16);
            const uint32_t ad[4] = {kb + o0, kb + (o0 ^ 16u), kb + (o0 ^ 128u), kb + (o0 ^ 144u)};
            auto rd = [&](auto KBT, int st) __attribute__((always_inline)) {
                constexpr int OFF = 16 * RS16 * decltype(KBT)::value;
                kr[st][0] = lds_rd128<OFF>(ad[0]);
                kr[st][1] = lds_rd128<OFF>(ad[1]);
                kr[st][2] = lds_rd128<OFF>(ad[2]);
                kr[st][3] = lds_rd128<OFF>(ad[3]);
            };
            rd(std::integral_constant<int, 0>{}, 0);
            static_for<4>([&](auto KBT) __attribute__((always_inline)) {
                constexpr int kbk = decltype(KBT)::value, st = kbk & 1;
                lds_wait4(kr[st][0], kr[st][1], kr[st][2], kr[st][3]);
                if constexpr (kbk + 1 < 4) rd(std::integral_constant<int, kbk + 1>{}, st ^ 1);
#pragma unroll
                for (int m = 0; m < 4; ++m) {
                    const f16x8 av = __builtin_bit_cast(f16x8, kr[st][m]);
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb) sf[sb][kbk] = mfma_f16(av, qh[sb][m], sf[sb][kbk]);
                }
            });
#pragma unroll
            for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk)
#pragma unroll
                    for (int r = 0; r < 4; ++r) s[sb][kbk][r] = sf[sb][kbk][r];
        };
        // -inf for the keys e of the tile a row may not see: e >= valid, and
        // with `causal` e > row
        auto mask_keys = [&](int i0, int valid, bool causal, float (&s)[2][4][4]) __attribute__((always_inline)) {
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                const int row = BM * blk + 32 * w + 16 * sb + c16;
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int e = i0 + 16 * kbk + 4 * g + r;
                        const bool ok = (e < valid) & (!causal | (e <= row));
                        s[sb][kbk][r] = ok ? s[sb][kbk][r] : -INFINITY;
                    }
            }
        };
        // online softmax (lazy max) of one tile and P -> fp16 B operands;
        // rest-tile scores stay integer-valued until the exponent (ssc =
        // q_scale k_scale, or 1 for fp16 tiles and all-zero blocks)
        auto softmax16 = [&](float ssc, float (&s)[2][4][4], u32x4 (&pw)[2][2]) __attribute__((always_inline)) {
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                // the test needs no cross-lane max: m_run is the same on the
                // four lanes of a row and ssc > 0, so some lane's own max
                // passes it exactly when the row max does; the row max is
                // formed only when the running max moves
                const float lmx = tile_max16(s[sb]) * ssc;
                if (__builtin_amdgcn_ballot_w64(lmx > m_run[sb] + PF_SLACK)) {
                    const float mx = quad_max_raw(lmx);
                    const float mnew = fmaxf(m_run[sb], mx);
                    const float alpha = __builtin_amdgcn_exp2f(m_run[sb] - mnew);
                    lsum[sb] *= alpha;
#pragma unroll
                    for (int cb = 0; cb < 8; ++cb) acc[sb][cb] *= alpha;
                    m_run[sb] = mnew;
                }
                float p[4][4];
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        p[kbk][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][kbk][r], ssc, -m_run[sb]));
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    pw[sb][j] = u32x4{pack_f16x2(p[2 * j][0], p[2 * j][1]), pack_f16x2(p[2 * j][2], p[2 * j][3]),
                                      pack_f16x2(p[2 * j + 1][0], p[2 * j + 1][1]),
                                      pack_f16x2(p[2 * j + 1][2], p[2 * j + 1][3])};
            }
        };
        // O^T += V^T . P^T from V at vb, and the row sums of P; the reads of
        // channel block cb + 1 in flight during the MFMAs of cb
        auto pv16 = [&](uint32_t vb, const u32x4 (&pw)[2][2]) __attribute__((always_inline)) {
            u32x2 v16[2][2][2];            // [stage][j][h]
            const uint32_t o0 = opaque_v(ov0);
            auto rd16 = [&](auto CBT, int st) __attribute__((always_inline)) {
                constexpr uint32_t cb = decltype(CBT)::value;
                const uint32_t ad = vb + (o0 ^ (32u * cb));
                v16[st][0][0] = lds_tr16<0>(ad);
                v16[st][0][1] = lds_tr16<16 * RS16>(ad);
                v16[st][1][0] = lds_tr16<32 * RS16>(ad);
                v16[st][1][1] = lds_tr16<48 * RS16>(ad);
            };
            rd16(std::integral_constant<int, 0>{}, 0);
            static_for<8>([&](auto CBT) __attribute__((always_inline)) {
                constexpr int cb = decltype(CBT)::value, st = cb & 1;
                lds_wait(v16[st][0][0], v16[st][0][1], v16[st][1][0], v16[st][1][1]);
                if constexpr (cb + 1 < 8) rd16(std::integral_constant<int, cb + 1>{}, st ^ 1);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const f16x8 av = __builtin_bit_cast(f16x8, u32x4{v16[st][j][0][0], v16[st][j][0][1],
                                                                     v16[st][j][1][0], v16[st][j][1][1]});
#pragma unroll
                    for (int sb = 0; sb < 2; ++sb)
                        acc[sb][cb] = mfma_f16(av, __builtin_bit_cast(f16x8, pw[sb][j]), acc[sb][cb]);
                }
            });
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
                    lsum[sb] = mfma_f16(__builtin_bit_cast(f16x8, onew), __builtin_bit_cast(f16x8, pw[sb][j]), lsum[sb]);
        };

        // fp8 P.V kernel: exact running max (P' = exp2(s - m + 8.807) stays at
        // or below 448, the e4m3 range), the row sums of P' on the VALU
        // (l_run); rest tiles pack P' as e4m3 (pk8[sb][kb]: keys 16 kb + 4 g +
        // 0..3), vertical and window tiles as fp16 (pw, as softmax16)
        auto softmax8 = [&](auto KT, float ssc, float (&s)[2][4][4], uint32_t (&pk8)[2][4], u32x4 (&pw)[2][2])
                            __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            float alpha[2] = {1.0f, 1.0f};
            bool resc = false;
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                const float lmx = tile_max16(s[sb]) * ssc;        // as in softmax16
                if (__builtin_amdgcn_ballot_w64(lmx > m_run[sb])) {
                    const float mx = quad_max_raw(lmx);
                    const float mnew = fmaxf(m_run[sb], mx);
                    alpha[sb] = __builtin_amdgcn_exp2f(m_run[sb] - mnew);
                    l_run[sb] *= alpha[sb];
                    m_run[sb] = mnew;
                    resc = true;
                }
            }
            if (resc) {                // acc32 lane l holds row l % 32: sub-block (l >> 4) & 1
                const float al = ((lane >> 4) & 1) ? alpha[1] : alpha[0];
#pragma unroll
                for (int cbk = 0; cbk < 4; ++cbk) acc32[cbk] *= al;
            }
#pragma unroll
            for (int sb = 0; sb < 2; ++sb) {
                // the rounding of mx, of the bias and of the fma can lift the
                // largest exponent by ulp(m) + 1e-6 above 8.807; the bias gives
                // that back so P' never passes 447.98 (no clamp before e4m3)
                const float bias = S_FP8_OFFSET - m_run[sb] - (fabsf(m_run[sb]) * 2.4e-7f + 1e-6f);
                float p[4][4];
                float ls = 0.0f;
#pragma unroll
                for (int kbk = 0; kbk < 4; ++kbk)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        p[kbk][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][kbk][r], ssc, bias));
                        ls += p[kbk][r];
                    }
                l_run[sb] += ls;
                if constexpr (KIND == T_REST) {
#pragma unroll
                    for (int kbk = 0; kbk < 4; ++kbk)
                        pk8[sb][kbk] = pack_e4m3x4_raw(p[kbk][0], p[kbk][1], p[kbk][2], p[kbk][3]);
                } else {
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        pw[sb][j] = u32x4{pack_f16x2(p[2 * j][0], p[2 * j][1]), pack_f16x2(p[2 * j][2], p[2 * j][3]),
                                          pack_f16x2(p[2 * j + 1][0], p[2 * j + 1][1]),
                                          pack_f16x2(p[2 * j + 1][2], p[2 * j + 1][3])};
                }
            }
        };
        // fp8 P.V kernel: P arrives in the score layout (lane (c, g): keys
        // 16 kb + 4 g + r of rows c (sub-block 0) and 16 + c (sub-block 1));
        // v_permlane16_swap of the two sub-blocks' registers leaves lane l with
        // row l % 32: its own keys then those of lane l ^ 16, i.e. keys
        // 16 kb + 8 (l >> 5) + 0..7 for fp16 P and the kp order above for e4m3 P.
        // O^T += V^T . P^T of a vertical / window tile (fp16 V at vb) with
        // v_mfma_f32_32x32x16_f16 per 16 keys and 32 channels
        auto pvh32 = [&](uint32_t vb, u32x4 (&pw)[2][2]) __attribute__((always_inline)) {
            u32x4 pb[4];               // B operand of key block kb
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const int j = kb >> 1, e0 = 2 * (kb & 1);
                const auto r0 = __builtin_amdgcn_permlane16_swap(pw[0][j][e0], pw[1][j][e0], false, false);
                const auto r1 = __builtin_amdgcn_permlane16_swap(pw[0][j][e0 + 1], pw[1][j][e0 + 1], false, false);
                pb[kb] = u32x4{r0[0], r1[0], r0[1], r1[1]};
            }
            const uint32_t ad[2] = {vb + ovh[0], vb + ovh[1]};
            u32x2 va[2][4][2];         // [stage][cbk][rd]: the 8 reads of key block kb
            auto rd = [&](auto KBT, int st) __attribute__((always_inline)) {
                constexpr int kb = decltype(KBT)::value;
                static_for<4>([&](auto CBT) __attribute__((always_inline)) {
                    constexpr int cbk = decltype(CBT)::value, OFF = (16 * kb) * RS16 + 128 * (cbk >> 1);
                    va[st][cbk][0] = lds_tr16<OFF>(ad[cbk & 1]);
                    va[st][cbk][1] = lds_tr16<OFF + 4 * RS16>(ad[cbk & 1]);
                });
            };
            rd(std::integral_constant<int, 0>{}, 0);
            static_for<4>([&](auto KBT) __attribute__((always_inline)) {
                constexpr int kb = decltype(KBT)::value, st = kb & 1;
                lds_wait(va[st][0][0], va[st][0][1], va[st][1][0], va[st][1][1]);
                lds_wait(va[st][2][0], va[st][2][1], va[st][3][0], va[st][3][1]);
                if constexpr (kb + 1 < 4) rd(std::integral_constant<int, kb + 1>{}, st ^ 1);
#pragma unroll
                for (int cbk = 0; cbk < 4; ++cbk) {
                    const f16x8 av = __builtin_bit_cast(f16x8, u32x4{va[st][cbk][0][0], va[st][cbk][0][1],
                                                                     va[st][cbk][1][0], va[st][cbk][1][1]});
                    acc32[cbk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, __builtin_bit_cast(f16x8, pb[kb]),
                                                                        acc32[cbk], 0, 0, 0);
                }
            });
        };
        // O^T += V^T . P'^T of a rest tile (e4m3 V at vb): one
        // v_mfma_scale_f32_32x32x64_f8f6f4 per 32 channels over all 64 keys
        // (unit block scales), the reads of block cbk + 1 in flight during the
        // MFMA of cbk
        auto pv8x = [&](uint32_t vb, uint32_t (&pk8)[2][4]) __attribute__((always_inline)) {
            uint32_t ba[4], bb[4];
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const auto r = __builtin_amdgcn_permlane16_swap(pk8[0][kb], pk8[1][kb], false, false);
                ba[kb] = r[0];
                bb[kb] = r[1];
            }
            const i32x8 bop = {static_cast<int>(ba[0]), static_cast<int>(ba[1]), static_cast<int>(ba[2]),
                               static_cast<int>(ba[3]), static_cast<int>(bb[0]), static_cast<int>(bb[1]),
                               static_cast<int>(bb[2]), static_cast<int>(bb[3])};
            u32x2 va[2][4];            // [stage][rd]
            auto rd = [&](auto CBT, int st) __attribute__((always_inline)) {
                const uint32_t ad = vb + ov8[decltype(CBT)::value];
                va[st][0] = lds_tr8<0>(ad);
                va[st][1] = lds_tr8<32 * RS8>(ad);
                va[st][2] = lds_tr8<4 * RS8>(ad);
                va[st][3] = lds_tr8<36 * RS8>(ad);
            };
            rd(std::integral_constant<int, 0>{}, 0);
            static_for<4>([&](auto CBT) __attribute__((always_inline)) {
                constexpr int cbk = decltype(CBT)::value, st = cbk & 1;
                lds_wait(va[st][0], va[st][1], va[st][2], va[st][3]);
                if constexpr (cbk + 1 < 4) rd(std::integral_constant<int, cbk + 1>{}, st ^ 1);
                const i32x8 aop = {static_cast<int>(va[st][0][0]), static_cast<int>(va[st][0][1]),
                                   static_cast<int>(va[st][1][0]), static_cast<int>(va[st][1][1]),
                                   static_cast<int>(va[st][2][0]), static_cast<int>(va[st][2][1]),
                                   static_cast<int>(va[st][3][0]), static_cast<int>(va[st][3][1])};
                acc32[cbk] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(aop, bop, acc32[cbk], 0, 0, 0, 127, 0, 127);
            });
        };

        // one run: tiles [t0, t1) of kind KIND
        float sc_next = 0.0f;      // k_scale of the next rest tile (vector load, a tile ahead)
        auto run = [&](auto KT, int t0, int t1) __attribute__((always_inline)) {
            constexpr int KIND = decltype(KT)::value;
            if (t0 >= t1) return;
            Rsrc rk, rv;
            sources(KT, rk, rv);
            const int valid = KIND == T_REST ? nr_b : KIND == T_VERT ? nv_b : wend;
            const bool causal = KIND == T_WIN || (KIND == T_REST && a.rest_causal);
            for (int t = t0; t < t1; ++t) {
                // this wavefront's DMAs of tile t have landed; the barrier
                // extends that to the workgroup and frees the other buffer pair
                // (read by tile t - 1)
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
                const int par = t & 1;
                const int i0 = first_of(KT, t);
                float sc = 1.0f;
                if constexpr (KIND == T_REST) {
                    sc = sc_next;
                    if (t + 1 < t1)
                        sc_next = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, 0, 4 * (t + 1), 0));
                }
                if (t + 1 < t1) issue(KT, rk, rv, i0 + BN, par ^ 1);
                else if (t + 1 < ntiles) issue_next_run(KT, t + 1, par ^ 1);

                float s[2][4][4];
                if constexpr (KIND == T_REST) qk_rest(kbase[par], s);
                else qk_f16(kbase[par], s);
                const int row0 = BM * blk + 32 * w;       // this wavefront's first row
                if (i0 + BN > valid || (causal && i0 + BN - 1 > row0)) mask_keys(i0, valid, causal, s);
                float ssc = 1.0f;
                if constexpr (KIND == T_REST) {
                    // a zero scale means all-zero codes on one side: every
                    // score is 0 and the scale 1 gives the same result (and
                    // keeps -inf * scale = -inf)
                    const float qks = q_scale * sc;
                    ssc = qks > 0.0f ? qks : 1.0f;
                }
                u32x4 pw[2][2];
                if constexpr (PV8) {
                    uint32_t pk8[2][4];
                    softmax8(KT, ssc, s, pk8, pw);
                    if constexpr (KIND == T_REST) pv8x(vbase[par], pk8);
                    else pvh32(vbase[par], pw);
                } else {
                    softmax16(ssc, s, pw);
                    pv16(vbase[par], pw);
                }
            }
        };
        if constexpr (PV8) {
            {
                // tile 0's DMAs (and scale) before the first run
                Rsrc rk, rv;
                if (nrt > 0) {
                    sources(std::integral_constant<int, T_REST>{}, rk, rv);
                    issue(std::integral_constant<int, T_REST>{}, rk, rv, 0, 0);
                    sc_next = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, 0, 0, 0));
                } else if (nvt > 0) {
                    sources(std::integral_constant<int, T_VERT>{}, rk, rv);
                    issue(std::integral_constant<int, T_VERT>{}, rk, rv, 0, 0);
                } else if (nwt > 0) {
                    sources(std::integral_constant<int, T_WIN>{}, rk, rv);
                    issue(std::integral_constant<int, T_WIN>{}, rk, rv, wla, 0);
                }
            }
            run(std::integral_constant<int, T_REST>{}, 0, nrt);
            run(std::integral_constant<int, T_VERT>{}, nrt, nrt + nvt);
            run(std::integral_constant<int, T_WIN>{}, nrt + nvt, ntiles);
        } else {
            // ---- fp16 P.V: software-pipelined runs -----------------------------
            // Step t exponentiates tile t's scores and multiplies P into O
            // while it forms the scores of tile t + 1: the QK MFMAs of tile
            // t + 1 share one instruction stream with the exponentials of tile
            // t, and the P.V MFMAs of tile t with the conversion, masking and
            // row maxima of tile t + 1, so that a wavefront keeps its matrix
            // core and its VALU busy together.  K runs one tile ahead of V:
            // entering step t the buffers hold K(t + 1) and V(t); the step
            // issues K(t + 2) into the buffer of K(t) (read by step t - 1) and
            // V(t + 1) into that of V(t - 1), so one barrier per step covers
            // both, across the runs too (the DMAs name any tile's kind).  Each
            // run starts with its first tile's scores alone and ends with its
            // last tile's P.V alone.  The arithmetic is the tile-at-a-time
            // order's: tile t + 1's maximum moves m (and rescales O) after
            // P(t) has been added to O.
            using KR = std::integral_constant<int, T_REST>;
            using KV = std::integral_constant<int, T_VERT>;
            using KW = std::integral_constant<int, T_WIN>;
            // the K (V) DMAs of tile t, whatever its kind (uniform branches)
            auto issue_k_any = [&](int t, int par) __attribute__((always_inline)) {
                Rsrc rk, rv;
                if (t < nrt) {
                    sources(KR{}, rk, rv);
                    issue_k(KR{}, rk, first_of(KR{}, t), par);
                } else if (t < nrt + nvt) {
                    sources(KV{}, rk, rv);
                    issue_k(KV{}, rk, first_of(KV{}, t), par);
                } else {
                    sources(KW{}, rk, rv);
                    issue_k(KW{}, rk, first_of(KW{}, t), par);
                }
            };
            auto issue_v_any = [&](int t, int par) __attribute__((always_inline)) {
                Rsrc rk, rv;
                if (t < nrt) {
                    sources(KR{}, rk, rv);
                    issue_v(KR{}, rv, first_of(KR{}, t), par);
                } else if (t < nrt + nvt) {
                    sources(KV{}, rk, rv);
                    issue_v(KV{}, rv, first_of(KV{}, t), par);
                } else {
                    sources(KW{}, rk, rv);
                    issue_v(KW{}, rv, first_of(KW{}, t), par);
                }
            };
            const int row0 = BM * blk + 32 * w;           // this wavefront's first row
            auto rfl = [](float x) __attribute__((always_inline)) {
                return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, x)));
            };
            // the row maxima of a tile's scores move m (and rescale O and the
            // row sums) when they pass it by more than the slack
            auto rescale = [&](const float (&lmx)[2]) __attribute__((always_inline)) {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    if (__builtin_amdgcn_ballot_w64(lmx[sb] > m_run[sb] + PF_SLACK)) {
                        const float mx = quad_max_raw(lmx[sb]);
                        const float mnew = fmaxf(m_run[sb], mx);
                        const float alpha = __builtin_amdgcn_exp2f(m_run[sb] - mnew);
                        lsum[sb] *= alpha;
#pragma unroll
                        for (int cb = 0; cb < 8; ++cb) acc[sb][cb] *= alpha;
                        m_run[sb] = mnew;
                    }
                }
            };
            // P = exp2(s ssc - m) as fp16 B operands
            auto exp_pack = [&](float ssc, const float (&s)[2][4][4], u32x4 (&pw)[2][2]) __attribute__((always_inline)) {
#pragma unroll
                for (int sb = 0; sb < 2; ++sb) {
                    float p[4][4];
#pragma unroll
                    for (int kbk = 0; kbk < 4; ++kbk)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            p[kbk][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[sb][kbk][r], ssc, -m_run[sb]));
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        pw[sb][j] = u32x4{pack_f16x2(p[2 * j][0], p[2 * j][1]), pack_f16x2(p[2 * j][2], p[2 * j][3]),
                                          pack_f16x2(p[2 * j + 1][0], p[2 * j + 1][1]),
                                          pack_f16x2(p[2 * j + 1][2], p[2 * j + 1][3])};
                }
            };
            float ks_pend = 0.0f;          // k_scale of tile t + 2, loaded during step t
            // one run: tiles [t0, t1) of kind KIND
            auto prun = [&](auto KT, int t0, int t1) __attribute__((always_inline)) {
                constexpr int KIND = decltype(KT)::value;
                if (t0 >= t1) return;
                const int valid = KIND == T_REST ? nr_b : KIND == T_VERT ? nv_b : wend;
                const bool causal = KIND == T_WIN || (KIND == T_REST && a.rest_causal);
                auto needs_mask = [&](int i0) __attribute__((always_inline)) {
                    return i0 + BN > valid || (causal && i0 + BN - 1 > row0);
                };
                // the scores of tile t (K in buffer t & 1), -inf masked
                auto scores = [&](auto MT, int t, float (&s)[2][4][4]) __attribute__((always_inline)) {
                    if constexpr (KIND == T_REST) qk_rest(kbase[t & 1], s);
                    else qk_f16(kbase[t & 1], s);
                    if constexpr (decltype(MT)::value) mask_keys(first_of(KT, t), valid, causal, s);
                };
                auto scale_of = [&](float ks) __attribute__((always_inline)) {
                    if constexpr (KIND == T_REST) {
                        const float qks = q_scale * ks;
                        return qks > 0.0f ? qks : 1.0f;
                    } else {
                        return 1.0f;
                    }
                };
                // int8 rest tiles hand their scores on as raw int32 bits
                constexpr bool RAW = KIND == T_REST && !QF8;
                // one piece of a next tile's P: scores (sb, kbk, 2 hf .. 2 hf +
                // 1) converted, masked, exponentiated with the current m and
                // packed; their maximum joins mx[sb]
                auto piece = [&](auto MT, auto PI, const float (&sn)[2][4][4], float ssc, int i0,
                                 u32x4 (&pn)[2][2], float (&mx)[2]) __attribute__((always_inline)) {
                    constexpr int pi = decltype(PI)::value, sb = pi >> 3, kbk = (pi >> 1) & 3, hf = pi & 1;
                    float v[2];
#pragma unroll
                    for (int e = 0; e < 2; ++e) {
                        const int r = 2 * hf + e;
                        float x = sn[sb][kbk][r];
                        if constexpr (RAW) x = static_cast<float>(__builtin_bit_cast(int, x));
                        if constexpr (decltype(MT)::value) {
                            const int row = BM * blk + 32 * w + 16 * sb + c16;
                            const int key = i0 + 16 * kbk + 4 * g + r;
                            const bool ok = (key < valid) & (!causal | (key <= row));
                            x = ok ? x : -INFINITY;
                        }
                        v[e] = x;
                    }
                    mx[sb] = (kbk == 0 && hf == 0) ? vmax2(v[0], v[1]) : vmax3(mx[sb], v[0], v[1]);
                    const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(v[0], ssc, -m_run[sb]));
                    const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(v[1], ssc, -m_run[sb]));
                    pn[sb][kbk >> 1][2 * (kbk & 1) + hf] = pack_f16x2(p0, p1);
                };
                // P.V of tile t (P = pc, V at vb) with the next tile's scores
                // turned into its P (pn) in between: after every second P.V
                // MFMA one piece (8 VALU instructions, two of them
                // exponentials); scheduling fences keep that interleave
                auto pv_fused = [&](auto MT, uint32_t vb, const u32x4 (&pc)[2][2], const float (&sn)[2][4][4],
                                    float ssc, int i0, u32x4 (&pn)[2][2], float (&lmx)[2]) __attribute__((always_inline)) {
                    float mx[2];
                    u32x2 v16[2][2][2];        // [stage][j][h]
                    const uint32_t o0 = opaque_v(ov0);
                    auto rd16 = [&](auto CBT, int st) __attribute__((always_inline)) {
                        constexpr uint32_t cb = decltype(CBT)::value;
                        const uint32_t ad = vb + (o0 ^ (32u * cb));
                        v16[st][0][0] = lds_tr16<0>(ad);
                        v16[st][0][1] = lds_tr16<16 * RS16>(ad);
                        v16[st][1][0] = lds_tr16<32 * RS16>(ad);
                        v16[st][1][1] = lds_tr16<48 * RS16>(ad);
                    };
                    rd16(std::integral_constant<int, 0>{}, 0);
                    static_for<8>([&](auto CBT) __attribute__((always_inline)) {
                        constexpr int cb = decltype(CBT)::value, st = cb & 1;
                        lds_wait(v16[st][0][0], v16[st][0][1], v16[st][1][0], v16[st][1][1]);
                        if constexpr (cb + 1 < 8) rd16(std::integral_constant<int, cb + 1>{}, st ^ 1);
                        static_for<2>([&](auto JT) __attribute__((always_inline)) {
                            constexpr int j = decltype(JT)::value;
                            const f16x8 av = __builtin_bit_cast(f16x8, u32x4{v16[st][j][0][0], v16[st][j][0][1],
                                                                             v16[st][j][1][0], v16[st][j][1][1]});
#pragma unroll
                            for (int sb = 0; sb < 2; ++sb)
                                acc[sb][cb] = mfma_f16(av, __builtin_bit_cast(f16x8, pc[sb][j]), acc[sb][cb]);
                            piece(MT, std::integral_constant<int, 2 * cb + j>{}, sn, ssc, i0, pn, mx);
                            __builtin_amdgcn_sched_barrier(0);
                        });
                    });
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int sb = 0; sb < 2; ++sb)
                            lsum[sb] = mfma_f16(__builtin_bit_cast(f16x8, onew), __builtin_bit_cast(f16x8, pc[sb][j]), lsum[sb]);
                    lmx[0] = mx[0] * ssc;
                    lmx[1] = mx[1] * ssc;
                    // P is used here (not only on the branch that keeps it), so
                    // that it is formed in its pieces rather than sunk past
                    // the slack test
                    asm volatile("" : "+v"(pn[0][0]), "+v"(pn[0][1]), "+v"(pn[1][0]), "+v"(pn[1][1]));
                };
                // one step with a next tile: its P is formed with the current m
                // while P(t) goes into O; when one of its row maxima passes m
                // by more than the slack (rare), O is rescaled after P(t) and
                // its scores and P are formed again with the new m
                auto body = [&](auto MT, int t, const u32x4 (&pc)[2][2], float ssc_n, u32x4 (&pn)[2][2])
                                __attribute__((always_inline)) {
                    float sn[2][4][4];
                    if constexpr (KIND == T_REST) qk_rest_t(std::integral_constant<bool, RAW>{}, kbase[(t + 1) & 1], sn);
                    else qk_f16(kbase[(t + 1) & 1], sn);
                    const int i0 = first_of(KT, t + 1);
                    float lmx[2];
                    pv_fused(MT, vbase[t & 1], pc, sn, ssc_n, i0, pn, lmx);
                    if (__builtin_amdgcn_ballot_w64(lmx[0] > m_run[0] + PF_SLACK) |
                        __builtin_amdgcn_ballot_w64(lmx[1] > m_run[1] + PF_SLACK)) {
                        rescale(lmx);
                        // the scores again from K(t + 1), still in LDS (not
                        // held through the step)
                        float sr[2][4][4];
                        if constexpr (KIND == T_REST) qk_rest_t(std::integral_constant<bool, RAW>{}, kbase[(t + 1) & 1], sr);
                        else qk_f16(kbase[(t + 1) & 1], sr);
                        float mx[2];
                        static_for<16>([&](auto PI) __attribute__((always_inline)) {
                            piece(MT, PI, sr, ssc_n, i0, pn, mx);
                        });
                    }
                };
                auto step = [&](int t, const u32x4 (&pc)[2][2], u32x4 (&pn)[2][2]) __attribute__((always_inline)) {
                    // own DMAs of K(t + 1) and V(t) landed; the barrier extends
                    // that to the workgroup and frees the buffers of K(t) and
                    // V(t - 1)
                    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                    __syncthreads();
                    const float ks1 = rfl(ks_pend);
                    if (t + 2 < nrt)
                        ks_pend = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, 0, 4 * (t + 2), 0));
                    if (t + 2 < ntiles) issue_k_any(t + 2, t & 1);
                    if (t + 1 < ntiles) issue_v_any(t + 1, (t + 1) & 1);
                    if (t + 1 < t1) {
                        const float ssc_n = scale_of(ks1);
                        if (needs_mask(first_of(KT, t + 1))) body(std::true_type{}, t, pc, ssc_n, pn);
                        else body(std::false_type{}, t, pc, ssc_n, pn);
                    } else {
                        pv16(vbase[t & 1], pc);
                    }
                };
                // the run's first tile (K(t0) has landed for the workgroup: a
                // step's or the prologue's barrier): exact maxima, then P
                u32x4 pX[2][2], pY[2][2];
                {
                    float s0[2][4][4];
                    if (needs_mask(first_of(KT, t0))) scores(std::true_type{}, t0, s0);
                    else scores(std::false_type{}, t0, s0);
                    float ssc0 = 1.0f;
                    if constexpr (KIND == T_REST) ssc0 = scale_of(rfl(sc_next));
                    const float lmx[2] = {tile_max16(s0[0]) * ssc0, tile_max16(s0[1]) * ssc0};
                    rescale(lmx);
                    exp_pack(ssc0, s0, pX);
                }
                // unrolled by two so that the two P sets keep their registers
                for (int t = t0; t < t1; t += 2) {
                    step(t, pX, pY);
                    if (t + 1 < t1) step(t + 1, pY, pX);
                }
            };
            if (ntiles > 0) {
                // prologue: K(0), V(0), K(1) and the first two k_scales
                issue_k_any(0, 0);
                issue_v_any(0, 0);
                if (ntiles > 1) issue_k_any(1, 1);
                if (nrt > 0) sc_next = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, 0, 0, 0));
                if (nrt > 1) ks_pend = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, 0, 4, 0));
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
                __syncthreads();
            }
            prun(KR{}, 0, nrt);
            // the fp16 tiles' Q operand, from Q again (through a pointer and
            // lane coordinates the compiler cannot match with the first
            // loads: it would otherwise hold those values, or addresses, in
            // registers through the rest tiles)
            {
                const uint16_t* qagain = a.q;
                asm volatile("" : "+s"(qagain));
                const int cr = static_cast<int>(opaque_v(c16)), gr = static_cast<int>(opaque_v(g));
#pragma unroll
                for (int sb = 0; sb < 2; ++sb)
#pragma unroll
                    for (int cc = 0; cc < 2; ++cc) {
                        float xv[16];
                        q_chunk(qagain, cr, gr, sb, cc, xv);
                        make_qh(sb, cc, xv);
                    }
            }
            prun(KV{}, nrt, nrt + nvt);
            prun(KW{}, nrt + nvt, ntiles);
        }
    }


    // ---- epilogue: O = acc / l (x vscale in fp8 mode) ------------------------------
    if constexpr (PV8) {
        // lane l: row l % 32 of the wavefront (row c of sub-block (l >> 4) & 1),
        // channels 32 cbk + 8 i4 + 4 (l >> 5) + 0..3
        const float l0 = quad_sum(l_run[0]), l1 = quad_sum(l_run[1]);
        const float inv = 1.0f / (((lane >> 4) & 1) ? l1 : l0);
        const int row = BM * blk + 32 * w + (lane & 31);
        if (row < a.N) {
            uint16_t* orow = a.out + b * a.o_b + h * a.o_h + static_cast<int64_t>(row) * a.o_n;
#pragma unroll
            for (int cbk = 0; cbk < 4; ++cbk)
#pragma unroll
                for (int i4 = 0; i4 < 4; ++i4) {
                    const int ch = 32 * cbk + 8 * i4 + 4 * (lane >> 5);
                    const f32x4 vs = *reinterpret_cast<const f32x4*>(a.vscale + bhk * PD + ch);
                    f32x4 o4 = {acc32[cbk][4 * i4], acc32[cbk][4 * i4 + 1], acc32[cbk][4 * i4 + 2], acc32[cbk][4 * i4 + 3]};
                    o4 = o4 * inv * vs;
                    const u32x2 o = a.f16 ? u32x2{pack_f16x2(o4[0], o4[1]), pack_f16x2(o4[2], o4[3])}
                                          : u32x2{pack_bf16x2(o4[0], o4[1]), pack_bf16x2(o4[2], o4[3])};
                    *reinterpret_cast<u32x2*>(orow + ch) = o;
                }
        }
    } else {
        // lane coordinates formed here (not hoisted into the tile loops)
        const int cr = static_cast<int>(opaque_v(c16)), gr = static_cast<int>(opaque_v(g));
#pragma unroll
        for (int sb = 0; sb < 2; ++sb) {
            const float inv = 1.0f / lsum[sb][0];
            const int row = BM * blk + 32 * w + 16 * sb + cr;
            if (row < a.N) {
                uint16_t* orow = a.out + b * a.o_b + h * a.o_h + static_cast<int64_t>(row) * a.o_n;
#pragma unroll
                for (int cb = 0; cb < 8; ++cb) {
                    const f32x4 o4 = acc[sb][cb] * inv;
                    const u32x2 o = a.f16 ? u32x2{pack_f16x2(o4[0], o4[1]), pack_f16x2(o4[2], o4[3])}
                                          : u32x2{pack_bf16x2(o4[0], o4[1]), pack_bf16x2(o4[2], o4[3])};
                    *reinterpret_cast<u32x2*>(orow + 16 * cb + 4 * gr) = o;
                }
            }
        }
    }
}

__global__ __launch_bounds__(256) void zero_counts_kernel(int32_t* __restrict__ nr, int32_t* __restrict__ nv,
                                                          int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) nr[i] = 0;
    else if (i < 2 * n) nv[i - n] = 0;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

int next_pow2(int x) {
    int p = 1;
    while (p < x) p <<= 1;
    return p;
}

// LDS a workgroup may allocate dynamically on the current device
size_t lds_budget() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    if (cache[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        cache[dev] = v;
    }
    return static_cast<size_t>(cache[dev]) - 1024;   // the kernel's static LDS
}

// ints of one row's list scratch (sorted list, bitmap, per-word prefix)
int64_t lists_row_ints(int64_t T, int64_t P) {
    return next_pow2(static_cast<int>(std::max<int64_t>(T, 1))) + 2 * ((P + 31) / 32);
}

// do one row's list arrays fit the LDS budget?
bool lists_in_lds(int64_t T, int64_t P) { return static_cast<size_t>(lists_row_ints(T, P)) * 4 <= lds_budget(); }

struct PrefillLayout {
    size_t kpart, vpart, km, vscale, k16, v16, v8, vert, rest, rcount, nr, nv, k8r, k8r_scale, vr, kv16, vv16,
        lscratch, total;
};

PrefillLayout prefill_layout(int B, int HQ, int HKV, int64_t N, int64_t T, int W, int pv_mode) {
    const int64_t P = std::max<int64_t>(0, N - W);
    const int64_t nblk = (N + BM - 1) / BM;
    const int64_t nch = (N + STAT_ROWS - 1) / STAT_ROWS;
    const int64_t nsb = (P + BN - 1) / BN;
    const int64_t BH = static_cast<int64_t>(B) * HQ, BHK = static_cast<int64_t>(B) * HKV;
    PrefillLayout L{};
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(std::max<size_t>(bytes, 1)); return o; };
    L.kpart = take(BHK * nch * PD * 8);
    L.vpart = take(BHK * nch * PD * 4);
    L.km = take(BHK * PD * 2);
    L.vscale = take(BHK * PD * 4);
    L.k16 = take(BHK * N * PD * 2);
    L.v16 = take(BHK * N * PD * 2);
    L.v8 = pv_mode ? take(BHK * N * PD) : 0;
    L.vert = take(BH * T * 4);
    L.rest = take(BH * P * 4);
    L.rcount = take(BH * 4);
    L.nr = take(BH * nblk * 4);
    L.nv = take(BH * nblk * 4);
    L.k8r = take(BH * P * PD);
    L.k8r_scale = take(BH * nsb * 4);
    L.vr = take(BH * P * PD * (pv_mode ? 1 : 2));
    L.kv16 = take(BH * T * PD * 2);
    L.vv16 = take(BH * T * PD * 2);
    L.lscratch = (P > 0 && !lists_in_lds(T, P)) ? take(BH * lists_row_ints(T, P) * 4) : 0;
    L.total = off;
    return L;
}

int launch_lists(const int64_t* vidx, int64_t vi_b, int64_t vi_h, int64_t vi_t, int BH, int H, int T, int P,
                 int nblk, int W, int32_t* vert, int32_t* rest, int32_t* rcount, int32_t* nr, int32_t* nv,
                 int* gscratch, hipStream_t stream) {
    static bool attr_set = false;
    const int n2 = next_pow2(std::max(T, 1));
    if (lists_in_lds(T, P)) {
        const size_t lds = sizeof(int) * static_cast<size_t>(lists_row_ints(T, P));
        if (!attr_set && lds > 64 * 1024) {
            if (hipFuncSetAttribute(reinterpret_cast<const void*>(&lists_kernel<false>),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds_budget())) != hipSuccess)
                return fail(HYQ_EDEVICE, "prefill lists: cannot raise the LDS limit of lists_kernel");
            attr_set = true;
        }
        hipLaunchKernelGGL(lists_kernel<false>, dim3(BH), dim3(LIST_THREADS), lds, stream, vidx, vi_b, vi_h, vi_t, H, T,
                           n2, P, nblk, W, vert, rest, rcount, nr, nv, nullptr);
    } else {
        if (!gscratch) return fail(HYQ_ENOSPC, "prefill lists: no scratch for lists larger than LDS");
        hipLaunchKernelGGL(lists_kernel<true>, dim3(BH), dim3(LIST_THREADS), 0, stream, vidx, vi_b, vi_h, vi_t, H, T,
                           n2, P, nblk, W, vert, rest, rcount, nr, nv, gscratch);
    }
    return check_launch("lists_kernel");
}

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" size_t hyq_prefill_workspace_size(int32_t b, int32_t hq, int32_t hkv, int64_t n, int64_t t,
                                             int32_t window, int32_t pv_mode) {
    if (b <= 0 || hq <= 0 || hkv <= 0 || n <= 0 || t < 0 || window < 0) return 0;
    return prefill_layout(b, hq, hkv, n, t, window, pv_mode).total;
}

extern "C" int hyq_per_block_int8(const void* x, int32_t x_is_fp16, int64_t xs_b, int64_t xs_h, int64_t xs_n,
                                  int32_t b, int32_t h, int64_t len, int32_t d, float sm, int32_t blk,
                                  const void* km, int64_t km_b, int64_t km_h, void* out, int64_t os_b, int64_t os_h,
                                  int64_t os_n, float* scale, int64_t ss_b, int64_t ss_h, void* stream_) {
    hipStream_t stream = static_cast<hipStream_t>(stream_);
    if (d != PD) return fail(HYQ_ENOTSUP, "hyq_per_block_int8: head_dim must be 128");
    if (b < 0 || h < 0 || len < 0 || blk <= 0 || blk > 4096 || len > INT32_MAX)
        return fail(HYQ_EINVAL, "hyq_per_block_int8: invalid sizes");
    if (b == 0 || h == 0 || len == 0) return HYQ_OK;
    if (!x || !out || !scale) return fail(HYQ_EINVAL, "hyq_per_block_int8: null pointer");
    if (!aligned(x, 16) || (xs_n * 2) % 16 || (xs_h * 2) % 16 || (xs_b * 2) % 16)
        return fail(HYQ_EINVAL, "hyq_per_block_int8: input rows must be 16-byte aligned");
    if (!aligned(out, 8) || os_n % 8 || os_h % 8 || os_b % 8)
        return fail(HYQ_EINVAL, "hyq_per_block_int8: output rows must be 8-byte aligned");
    const int nb = static_cast<int>((len + blk - 1) / blk);
    hipLaunchKernelGGL(per_block_int8_kernel, dim3(nb, h, b), dim3(256), 0, stream,
                       static_cast<const uint16_t*>(x), x_is_fp16, xs_b, xs_h, xs_n, static_cast<int>(len), blk, sm,
                       static_cast<const uint16_t*>(km), km_b, km_h, static_cast<int8_t*>(out), os_b, os_h, os_n,
                       scale, ss_b, ss_h);
    return check_launch("per_block_int8_kernel");
}

extern "C" size_t hyq_prefill_lists_workspace_size(int32_t b, int32_t h, int64_t n, int64_t t, int32_t window) {
    if (b <= 0 || h <= 0 || n <= 0 || t < 0 || window < 0) return 0;
    const int64_t P = std::max<int64_t>(0, n - window);
    if (P == 0 || P > MAX_P || t > MAX_T || lists_in_lds(t, P)) return 0;
    return static_cast<size_t>(b) * h * lists_row_ints(t, P) * 4;
}

extern "C" int hyq_prefill_lists(const int64_t* vidx, int64_t vi_b, int64_t vi_h, int64_t vi_t, int32_t b,
                                 int32_t h, int64_t n, int64_t t, int32_t window, int32_t* vert, int32_t* rest,
                                 int32_t* rcount, int32_t* nr, int32_t* nv, void* workspace, size_t workspace_bytes,
                                 void* stream) {
    if (b < 0 || h < 0 || n < 0 || t < 0 || window < 0 || n > INT32_MAX / 2)
        return fail(HYQ_EINVAL, "hyq_prefill_lists: invalid sizes");
    const int64_t P = std::max<int64_t>(0, n - window);
    if (P > MAX_P) return fail(HYQ_ENOTSUP, "hyq_prefill_lists: n - window exceeds 2^24");
    if (t > MAX_T) return fail(HYQ_ENOTSUP, "hyq_prefill_lists: more than 2^24 indices per head");
    if (b == 0 || h == 0 || n == 0) return HYQ_OK;
    const int nblk = static_cast<int>((n + BM - 1) / BM);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (P == 0) {
        if (!nr || !nv) return fail(HYQ_EINVAL, "hyq_prefill_lists: null pointer");
        hipLaunchKernelGGL(zero_counts_kernel, dim3((2 * b * h * nblk + 255) / 256), dim3(256), 0, s, nr, nv,
                           b * h * nblk);
        return check_launch("zero_counts_kernel");
    }
    if ((t > 0 && (!vidx || !vert)) || !rest || !rcount || !nr || !nv)
        return fail(HYQ_EINVAL, "hyq_prefill_lists: null pointer");
    const size_t need = hyq_prefill_lists_workspace_size(b, h, n, t, window);
    if (need > 0 && (!workspace || workspace_bytes < need || !aligned(workspace, 4)))
        return fail(HYQ_ENOSPC, "hyq_prefill_lists: workspace too small (need " + std::to_string(need) + " bytes)");
    return launch_lists(vidx, vi_b, vi_h, vi_t, b * h, h, static_cast<int>(t), static_cast<int>(P), nblk, window, vert,
                        rest, rcount, nr, nv, need > 0 ? static_cast<int*>(workspace) : nullptr, s);
}

namespace hyq {
namespace {
// Both prefill entry points: the hybrid partition, or with rest_causal (the
// unified kernel's window 0) every key through int8 up to the diagonal.
int prefill_run(const hyq_prefill_params* p, void* ws, size_t ws_bytes, hipStream_t stream, bool rest_causal,
                bool qk_fp8, const std::string& name) {
    if (!p) return fail(HYQ_EINVAL, name + ": null params");
    const int B = p->batch, HQ = p->hq, HKV = p->hkv, W = p->window;
    const int64_t N = p->n, T = p->t;
    if (p->head_dim != PD) return fail(HYQ_ENOTSUP, name + ": head_dim must be 128");
    if (p->pv_mode != 0 && p->pv_mode != 1) return fail(HYQ_EINVAL, name + ": pv_mode must be 0 (fp16) or 1 (fp8)");
    if (p->dtype_fp16 != 0 && p->dtype_fp16 != 1) return fail(HYQ_EINVAL, name + ": dtype_fp16 must be 0 or 1");
    const int f16 = p->dtype_fp16;
    if (B <= 0 || HQ <= 0 || HKV <= 0 || HQ % HKV || N <= 0 || N > INT32_MAX / 2 || T < 0 || W < 0)
        return fail(HYQ_EINVAL, name + ": invalid sizes (need HQ % HKV == 0, N > 0)");
    const int64_t P = std::max<int64_t>(0, N - W);
    if (N > MAX_N) return fail(HYQ_ENOTSUP, name + ": sequence length exceeds 2^24");
    if (P > MAX_P) return fail(HYQ_ENOTSUP, name + ": N - window exceeds 2^24");
    if (T > MAX_T) return fail(HYQ_ENOTSUP, name + ": more than 2^24 vertical indices per head");
    if (!p->q || !p->k || !p->v || !p->out || (P > 0 && T > 0 && !p->vidx))
        return fail(HYQ_EINVAL, name + ": null pointer");
    auto rows16 = [](const void* ptr, int64_t sb, int64_t sh, int64_t sn) {
        return aligned(ptr, 16) && (sb * 2) % 16 == 0 && (sh * 2) % 16 == 0 && (sn * 2) % 16 == 0;
    };
    if (!rows16(p->q, p->q_stride_b, p->q_stride_h, p->q_stride_n) ||
        !rows16(p->k, p->k_stride_b, p->k_stride_h, p->k_stride_n) ||
        !rows16(p->v, p->v_stride_b, p->v_stride_h, p->v_stride_n) ||
        !rows16(p->out, p->o_stride_b, p->o_stride_h, p->o_stride_n))
        return fail(HYQ_EINVAL, name + ": q/k/v/out rows must be contiguous and 16-byte aligned");
    const PrefillLayout L = prefill_layout(B, HQ, HKV, N, T, W, p->pv_mode);
    if (!ws || ws_bytes < L.total || !aligned(ws, 256))
        return fail(HYQ_ENOSPC, name + ": workspace too small or not 256-byte aligned (need " +
                                    std::to_string(L.total) + " bytes)");
    uint8_t* base = static_cast<uint8_t*>(ws);
    auto at = [&](size_t off) { return static_cast<void*>(base + off); };
    const int BH = B * HQ, BHK = B * HKV;
    const int nblk = static_cast<int>((N + BM - 1) / BM);
    const int nch = static_cast<int>((N + STAT_ROWS - 1) / STAT_ROWS);
    const int nsb = static_cast<int>((P + BN - 1) / BN);
    const int Pi = static_cast<int>(P), Ti = static_cast<int>(P > 0 ? T : 0), Ni = static_cast<int>(N);
    const uint16_t* k = static_cast<const uint16_t*>(p->k);
    const uint16_t* v = static_cast<const uint16_t*>(p->v);

    hipLaunchKernelGGL(kv_stats_kernel, dim3(nch, BHK), dim3(256), 0, stream, k, p->k_stride_b, p->k_stride_h,
                       p->k_stride_n, v, p->v_stride_b, p->v_stride_h, p->v_stride_n, HKV, Ni, nch, f16,
                       static_cast<double*>(at(L.kpart)), static_cast<float*>(at(L.vpart)));
    if (int st = check_launch("kv_stats_kernel")) return st;
    hipLaunchKernelGGL(kv_final_kernel, dim3(BHK), dim3(PD), 0, stream, static_cast<const double*>(at(L.kpart)),
                       static_cast<const float*>(at(L.vpart)), nch, Ni, p->smooth_k ? 1 : 0, f16,
                       static_cast<uint16_t*>(at(L.km)), static_cast<float*>(at(L.vscale)));
    if (int st = check_launch("kv_final_kernel")) return st;
    const int cblocks = static_cast<int>((N * 16 + 255) / 256);
    hipLaunchKernelGGL(kv_convert_kernel, dim3(cblocks, BHK), dim3(256), 0, stream, k, p->k_stride_b,
                       p->k_stride_h, p->k_stride_n, v, p->v_stride_b, p->v_stride_h, p->v_stride_n, HKV, Ni, f16,
                       static_cast<const uint16_t*>(at(L.km)), static_cast<const float*>(at(L.vscale)),
                       static_cast<uint16_t*>(at(L.k16)), static_cast<uint16_t*>(at(L.v16)),
                       p->pv_mode ? static_cast<uint8_t*>(at(L.v8)) : nullptr);
    if (int st = check_launch("kv_convert_kernel")) return st;
    if (P > 0) {
        if (int st = launch_lists(p->vidx, p->vi_stride_b, p->vi_stride_h, p->vi_stride_t, BH, HQ, Ti, Pi, nblk, W,
                                  static_cast<int32_t*>(at(L.vert)), static_cast<int32_t*>(at(L.rest)),
                                  static_cast<int32_t*>(at(L.rcount)), static_cast<int32_t*>(at(L.nr)),
                                  static_cast<int32_t*>(at(L.nv)),
                                  L.lscratch ? static_cast<int*>(at(L.lscratch)) : nullptr, stream))
            return st;
        const int nvb = (Ti + BN - 1) / BN;
        hipLaunchKernelGGL(gather_kernel, dim3(nsb + nvb, BH), dim3(256), 0, stream,
                           static_cast<const uint16_t*>(at(L.k16)), static_cast<const uint16_t*>(at(L.v16)),
                           p->pv_mode ? static_cast<const uint8_t*>(at(L.v8)) : nullptr, HQ, HQ / HKV, HKV, Ni, Pi, Ti,
                           nsb, static_cast<const int32_t*>(at(L.rest)), static_cast<const int32_t*>(at(L.rcount)),
                           static_cast<const int32_t*>(at(L.vert)), static_cast<int8_t*>(at(L.k8r)),
                           static_cast<float*>(at(L.k8r_scale)), static_cast<uint8_t*>(at(L.vr)),
                           static_cast<uint16_t*>(at(L.kv16)), static_cast<uint16_t*>(at(L.vv16)), qk_fp8 ? 1 : 0);
        if (int st = check_launch("gather_kernel")) return st;
    } else {
        // no prefix: every block reads zero rest / vertical entries
        hipLaunchKernelGGL(zero_counts_kernel, dim3((2 * BH * nblk + 255) / 256), dim3(256), 0, stream,
                           static_cast<int32_t*>(at(L.nr)), static_cast<int32_t*>(at(L.nv)), BH * nblk);
        if (int st = check_launch("zero_counts_kernel")) return st;
    }
    PfArgs a{};
    a.q = static_cast<const uint16_t*>(p->q); a.q_b = p->q_stride_b; a.q_h = p->q_stride_h; a.q_n = p->q_stride_n;
    a.out = static_cast<uint16_t*>(p->out); a.o_b = p->o_stride_b; a.o_h = p->o_stride_h; a.o_n = p->o_stride_n;
    a.k8r = static_cast<const int8_t*>(at(L.k8r));
    a.k8r_scale = static_cast<const float*>(at(L.k8r_scale));
    a.vr = static_cast<const uint16_t*>(at(L.vr));
    a.kv16 = static_cast<const uint16_t*>(at(L.kv16));
    a.vv16 = static_cast<const uint16_t*>(at(L.vv16));
    a.k16 = static_cast<const uint16_t*>(at(L.k16));
    a.v16 = static_cast<const uint16_t*>(at(L.v16));
    a.nr = static_cast<const int32_t*>(at(L.nr));
    a.nv = static_cast<const int32_t*>(at(L.nv));
    a.B = B; a.HQ = HQ; a.HKV = HKV; a.N = Ni; a.nblk = nblk; a.W = W; a.P = Pi; a.T = Ti; a.nsb = nsb;
    const double sm = p->sm_scale > 0.0 ? p->sm_scale : std::pow(static_cast<double>(PD), -0.5);
    a.c = static_cast<float>(sm * 1.44269504);
    a.total = BH * nblk;
    a.per_xcd = (a.total + 7) / 8;
    a.vscale = static_cast<const float*>(at(L.vscale));
    a.rest_causal = rest_causal ? 1 : 0;
    a.f16 = f16;
    if (qk_fp8)
        hipLaunchKernelGGL((prefill_main_kernel<false, true>), dim3(8 * a.per_xcd), dim3(PF_THREADS), 0, stream, a);
    else if (p->pv_mode)
        hipLaunchKernelGGL((prefill_main_kernel<true, false>), dim3(8 * a.per_xcd), dim3(PF_THREADS), 0, stream, a);
    else
        hipLaunchKernelGGL((prefill_main_kernel<false, false>), dim3(8 * a.per_xcd), dim3(PF_THREADS), 0, stream, a);
    return check_launch("prefill_main_kernel");
}
}  // namespace
}  // namespace hyq

extern "C" int hyq_prefill_hybrid(const hyq_prefill_params* p, void* ws, size_t ws_bytes, void* stream) {
    return hyq::prefill_run(p, ws, ws_bytes, static_cast<hipStream_t>(stream), false, false, "hyq_prefill_hybrid");
}

extern "C" int hyq_prefill_hybrid_fp8qk(const hyq_prefill_params* p, void* ws, size_t ws_bytes, void* stream) {
    if (!p) return hyq::fail(HYQ_EINVAL, "hyq_prefill_hybrid_fp8qk: null params");
    if (p->pv_mode != 0) return hyq::fail(HYQ_EINVAL, "hyq_prefill_hybrid_fp8qk: pv_mode must be 0 (fp16 P.V)");
    return hyq::prefill_run(p, ws, ws_bytes, static_cast<hipStream_t>(stream), false, true,
                            "hyq_prefill_hybrid_fp8qk");
}

extern "C" int hyq_prefill_unified(const hyq_prefill_params* p, void* ws, size_t ws_bytes, void* stream) {
    if (!p) return hyq::fail(HYQ_EINVAL, "hyq_prefill_unified: null params");
    if (p->t != 0) return hyq::fail(HYQ_EINVAL, "hyq_prefill_unified: t must be 0 (no vertical indices)");
    return hyq::prefill_run(p, ws, ws_bytes, static_cast<hipStream_t>(stream), p->window == 0, false,
                            "hyq_prefill_unified");
}
