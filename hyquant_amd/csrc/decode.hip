// Fused four-segment hybrid decode attention for gfx950 (MI355X).
//
// Math (fused_d_stage_decode, src/ops/decode_d_stage.py:916-1005, split-K
// kernels :481-782): for each query head, one online softmax (log2 domain,
// scale sm_scale*log2e) over [int4 prefix | top-k | staging | window].  On the
// int4 prefix the per-token K scale is factored out of the dot product,
// s = (q . k_code) * s_k, and P is rounded to bf16 after multiplying by the
// per-token V scale, P' = bf16(p * s_v), before P' . v_code (F8).
//
// Two launches per step, no fences inside either:
//   decode_partial_kernel — a workgroup of 4 wavefronts owns one chunk of one
//     KV head (all G query heads of the GQA group ride along as MFMA
//     columns).  int4 chunks hold `split` tokens walked in 32-token groups
//     (wavefront w takes groups w, w+4, ...) through a three-deep register
//     ring, so two groups' loads are in flight while one is computed; bf16
//     chunks hold 128 tokens of one segment (two 16-token tiles per
//     wavefront, both loaded up front).  bf16 chunks are numbered first so
//     they start first.  The four wavefronts' (m, l, acc) are merged in LDS
//     and the workgroup writes one partial.
//   decode_merge_kernel — one workgroup per (KV head, 8-channel slice) reads
//     every partial of its head (its partial loads are issued before the
//     (m, l) table is built, so the merge is about one memory round trip) and
//     writes the bf16 output.  The kernel boundary orders the partials; a device-scope
//     release/acquire per workgroup inside one kernel costs an L2 writeback
//     each, which measured 3 us (B=1) to 47 us (B=16) per step.
//
// Per wavefront, lane l = 16*kb + c (c = l & 15, kb = l >> 4):
//   QK  S^T[token][g] = K_tile . Q^T with v_mfma_f32_16x16x32_{f16,bf16}:
//       A = 16 tokens x 32 channels (lane = token c, 8 channels), B = Q^T
//       (lane = head c).  Output lane (g=c, r=kb) holds tokens 4r..4r+3.
//   PV  O^T[channel][g] = V^T . P'^T with v_mfma_f32_16x16x32_bf16:
//       A = 16 channels x 32 token slots, B = P'^T; the 32-token group is
//       permuted so that slot e of lane-row kb is token
//       tau(kb,e) = e<4 ? 4kb+e : 16+4kb+(e-4), exactly the tokens whose
//       scores the QK output left in that lane: no cross-lane shuffle of P.
//   Channel 8*j+nb of V sits in row j of PV MFMA nb (lane j loads the dword /
//   16 bytes holding channels 8j..8j+7).  bf16 tiles use the K=16 form
//   (v_mfma_f32_16x16x16_bf16) whose slot e of lane-row kb is token 4kb+e.
// int4 -> MFMA operand conversion is done in registers without any lookup:
//   K: nibble ^ 8 -> fp16(1024 + u) by OR-ing a magic exponent, then one
//      packed fp16 add of -1032 gives the exact code (Q is fed as fp16,
//      pre-scaled by a power of two so every bf16 query value is exact).
//   V: nibble ^ 8 -> bf16(128 + u); the constant 136 is removed after the
//      product with a ninth MFMA against an all-ones operand, which yields
//      sum_t P'[g][t] rounded exactly as the main product.
#include "hyq_common.h"

#include <algorithm>
#include <string>

namespace hyq {
namespace {

constexpr int D = 128;
constexpr int WAVES = 4;                 // wavefronts per partial workgroup
constexpr int THREADS = 64 * WAVES;
constexpr int GROUP = 32;                // int4 tokens per wavefront iteration
constexpr int TILE = 16;                 // bf16 tokens per wavefront iteration
constexpr int CHUNK4_MIN = WAVES * GROUP;   // int4 split granularity
constexpr int CHUNK16 = WAVES * 2 * TILE;   // bf16 tokens per workgroup chunk
constexpr int MSLICE = 8;                // channels per merge workgroup
constexpr int MERGE_THREADS = 256;
constexpr float LOG2E = 1.44269504f;     // src/ops/decode_d_stage.py:17
constexpr float RESCALE_SLACK = 8.0f;    // lazy max update threshold (log2 units)
constexpr float M_INIT = -1.0e30f;
constexpr int MAX_PARTIALS = 4096;       // nwg * G bound of the merge tables

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct DecArgs {
    const uint16_t* q; int64_t q_stride;
    uint16_t* out; int64_t out_stride;
    const uint8_t* kp; int64_t kp_bh, kp_n;
    const uint8_t* vp; int64_t vp_bh, vp_n;
    const uint16_t* ks; int64_t ks_bh;
    const uint16_t* vs; int64_t vs_bh;
    int32_t n_quant;
    const uint16_t* sk[3]; const uint16_t* sv[3];
    int64_t sk_bh[3], sk_n[3], sv_bh[3], sv_n[3];
    int32_t sn[3];
    int32_t G;
    int32_t bh_kv;
    float qk_scale;        // sm_scale * log2(e)
    int32_t split;         // int4 tokens per chunk (multiple of CHUNK4_MIN)
    int32_t n4;            // int4 chunks per head
    int32_t nseg[3];       // bf16 chunks per segment
    int32_t n16;           // bf16 chunks per head
    int32_t nwg;           // chunks per head
    float* part;           // [bh_kv][nwg][G][D]
    float* ml;             // [bh_kv][nwg][G][2] = (m, l)
};

struct WaveState {
    float m;               // running reference max of column g (same in the 4 lanes of g)
    float l;               // this lane's partial softmax denominator
    f32x4 acc[8];          // O^T tiles: acc[nb][i] = O[g][32*kb + 8*i + nb]
    f32x4 ones;            // sum of P' per column (int4 V offset correction)
};

__device__ __forceinline__ f32x4 mfma_f16(const f16x8& a, const f16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma_bf16_k16(const bf16x4& a, const bf16x4& b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}

__device__ __forceinline__ uint32_t f16x2_add(uint32_t a, f16x2 b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) + b);
}

// NB: operand vectors are always assembled from scalars with a brace list;
// element-wise stores into an ext_vector inside unrolled loops were
// miscompiled (every element received element 0).

// nibble pair (s, s+16) of x, offset to u = code + 8 and tagged with a magic
// exponent: ((x >> s) & 0x000f000f) ^ (0x00080008 | magic).
__device__ __forceinline__ uint32_t nib2(uint32_t x, int s, uint32_t magic_xor) {
    return ((x >> s) & 0x000f000fu) ^ magic_xor;
}

// 8 int4 codes (one dword, nibble i = channel i, two's complement) -> 8 exact
// fp16 values in slot order [c0,c4,c1,c5,c2,c6,c3,c7]: fp16(1024 + u) - 1032.
__device__ __forceinline__ f16x8 int4_to_f16x8(uint32_t x) {
    const f16x2 bias = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const u32x4 o = {f16x2_add(nib2(x, 0, 0x64086408u), bias), f16x2_add(nib2(x, 4, 0x64086408u), bias),
                     f16x2_add(nib2(x, 8, 0x64086408u), bias), f16x2_add(nib2(x, 12, 0x64086408u), bias)};
    return __builtin_bit_cast(f16x8, o);
}

// v_exp_f32: 2^x without the denormal range fix-up of exp2f (results below
// 2^-126 flush to zero, which is harmless for softmax weights).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Cross-lane max / sum over the 4 lanes {c, c+16, c+32, c+48} of a column,
// with the gfx950 row-swap instructions: v_permlane16_swap leaves lane l
// holding {v[l], v[l^16]} in its two results and v_permlane32_swap
// {v[l], v[l^32]}, so two VALU swaps replace two LDS-routed shuffles.
__device__ __forceinline__ float xor16_pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_pair_max(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float col_max(float v) { return xor32_pair_max(xor16_pair_max(v)); }
__device__ __forceinline__ float col_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// token slot e of lane-row kb within a 32-token group
__device__ __forceinline__ constexpr int tau(int kb, int e) { return e < 4 ? 4 * kb + e : 16 + 4 * kb + (e - 4); }

// Online-softmax update with this lane's N log2-domain scores; on return s
// holds p = exp2(s - m) relative to the (possibly raised) running max.
template <int N>
__device__ __forceinline__ void softmax_step(WaveState& st, float (&s)[N], bool has_ones) {
    float mx = s[0];
#pragma unroll
    for (int e = 1; e < N; ++e) mx = fmaxf(mx, s[e]);
    mx = col_max(mx);
    const bool need = mx > st.m + RESCALE_SLACK;
    if (__builtin_amdgcn_ballot_w64(need)) {             // rare after the first group
        const float mnew = fmaxf(st.m, mx);
        const float alpha = fast_exp2(st.m - mnew);
        st.l *= alpha;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) st.acc[nb] *= alpha;
        if (has_ones) st.ones *= alpha;
        st.m = mnew;
    }
    float lsum = 0.f;
#pragma unroll
    for (int e = 0; e < N; ++e) {
        s[e] = fast_exp2(s[e] - st.m);
        lsum += s[e];
    }
    st.l += lsum;
}

// ---------------------------------------------------------------------------
// int4 prefix
// ---------------------------------------------------------------------------
struct Int4Raw {
    uint4 k[2];            // tile t: token 16t + c, bytes 16kb..16kb+15 (channels 32kb..32kb+31)
    uint32_t v[8];         // slot e: token tau(kb, e), bytes 4c..4c+3 (channels 8c..8c+7)
    uint32_t scl;          // lane < 32: k scale of token lane; else v scale of token lane-32
};

// Packed rows are contiguous (64 bytes per token), so every load of a group is
// one per-lane base plus a compile-time offset (immediate in the instruction).
constexpr int PROW = D / 2;
constexpr int BROW = D;                   // bf16 row stride in elements

struct Int4Ctx {
    const uint8_t* kbase;  // this head's packed K / V rows
    const uint8_t* vbase;
    const uint16_t* sbase; // this lane's scale array (k for lanes < 32, v otherwise)
    uint32_t klane;        // lane offset of tile 0: c * 64 + 16 * kb
    uint32_t vlane;        // lane offset of slot 0: 4kb * 64 + 4c
    int hi;                // end of the chunk
};

__device__ __forceinline__ void int4_load_full(Int4Raw& r, const Int4Ctx& x, int t0, int lane) {
    const uint8_t* kl = x.kbase + static_cast<int64_t>(t0) * PROW + x.klane;
    const uint8_t* vl = x.vbase + static_cast<int64_t>(t0) * PROW + x.vlane;
    r.k[0] = *reinterpret_cast<const uint4*>(kl);
    r.k[1] = *reinterpret_cast<const uint4*>(kl + 16 * PROW);
#pragma unroll
    for (int e = 0; e < 8; ++e) r.v[e] = *reinterpret_cast<const uint32_t*>(vl + tau(0, e) * PROW);
    r.scl = x.sbase[t0 + (lane & 31)];
}

// partial last group: every token index clamped to the last valid one
__device__ __forceinline__ void int4_load_tail(Int4Raw& r, const Int4Ctx& x, int t0, int nv, int lane) {
    const int c = lane & 15, kb = lane >> 4;
    const uint8_t* kg = x.kbase + static_cast<int64_t>(t0) * PROW;
    const uint8_t* vg = x.vbase + static_cast<int64_t>(t0) * PROW;
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
        r.k[tile] = *reinterpret_cast<const uint4*>(kg + min(16 * tile + c, nv - 1) * PROW + 16 * kb);
#pragma unroll
    for (int e = 0; e < 8; ++e)
        r.v[e] = *reinterpret_cast<const uint32_t*>(vg + min(tau(kb, e), nv - 1) * PROW + 4 * c);
    r.scl = x.sbase[t0 + min(lane & 31, nv - 1)];
}

template <bool MASK>
__device__ __forceinline__ void int4_compute(WaveState& st, const Int4Raw& r, const f16x8 (&qop)[4],
                                             uint16_t* scl, int nv, int lane, float qk) {
    const int kb = lane >> 4;
    // scales through this wavefront's LDS slot: 32 k scales then 32 v scales
    scl[lane] = static_cast<uint16_t>(r.scl);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    float sk[8], sv[8];
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        const u32x2 k4 = *reinterpret_cast<const u32x2*>(scl + 16 * half + 4 * kb);
        const u32x2 v4 = *reinterpret_cast<const u32x2*>(scl + 32 + 16 * half + 4 * kb);
        sk[4 * half + 0] = f16_bits_to_f32(k4[0] & 0xffff); sk[4 * half + 1] = f16_bits_to_f32(k4[0] >> 16);
        sk[4 * half + 2] = f16_bits_to_f32(k4[1] & 0xffff); sk[4 * half + 3] = f16_bits_to_f32(k4[1] >> 16);
        sv[4 * half + 0] = f16_bits_to_f32(v4[0] & 0xffff); sv[4 * half + 1] = f16_bits_to_f32(v4[0] >> 16);
        sv[4 * half + 2] = f16_bits_to_f32(v4[1] & 0xffff); sv[4 * half + 3] = f16_bits_to_f32(v4[1] >> 16);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // QK: S^T tile = K_tile . Q^T (exact fp16 codes x fp16 q)
    float s[8];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        acc = mfma_f16(int4_to_f16x8(r.k[tile].x), qop[0], acc);
        acc = mfma_f16(int4_to_f16x8(r.k[tile].y), qop[1], acc);
        acc = mfma_f16(int4_to_f16x8(r.k[tile].z), qop[2], acc);
        acc = mfma_f16(int4_to_f16x8(r.k[tile].w), qop[3], acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) s[4 * tile + i] = acc[i] * (sk[4 * tile + i] * qk);
    }
    if (MASK) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (tau(kb, e) >= nv) s[e] = -INFINITY;
    }
    softmax_step<8>(st, s, true);
    // P' = bf16(p * s_v): B operand of the PV MFMAs (slot e = token tau(kb, e))
    const u32x4 pw = {pack_bf16x2(s[0] * sv[0], s[1] * sv[1]), pack_bf16x2(s[2] * sv[2], s[3] * sv[3]),
                      pack_bf16x2(s[4] * sv[4], s[5] * sv[5]), pack_bf16x2(s[6] * sv[6], s[7] * sv[7])};
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);
    // V^T operands: bf16(128 + u) = code + 136, token pairs merged by perm
    uint32_t lo[4], hi[4];
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
        lo[pr] = perm(r.v[2 * pr + 1], r.v[2 * pr], 0x05040100u);  // nibbles 0-3 of both tokens
        hi[pr] = perm(r.v[2 * pr + 1], r.v[2 * pr], 0x07060302u);  // nibbles 4-7
    }
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const uint32_t* src = nb < 4 ? lo : hi;
        const int sh = 4 * (nb & 3);
        const u32x4 w = {nib2(src[0], sh, 0x43084308u), nib2(src[1], sh, 0x43084308u),
                         nib2(src[2], sh, 0x43084308u), nib2(src[3], sh, 0x43084308u)};
        st.acc[nb] = mfma_bf16(__builtin_bit_cast(bf16x8, w), pop, st.acc[nb]);
    }
    const u32x4 onesw = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    st.ones = mfma_bf16(__builtin_bit_cast(bf16x8, onesw), pop, st.ones);
}

// ---------------------------------------------------------------------------
// bf16 segments: 16-token tiles
// ---------------------------------------------------------------------------
struct Bf16Raw {
    uint4 k[4];            // token c, channels 32kb..32kb+31
    uint4 v[4];            // slot e: token 4kb+e, channels 8c..8c+7
};

__device__ __forceinline__ void bf16_load(Bf16Raw& r, const uint16_t* kg, const uint16_t* vg, int nv, int lane) {
    const int c = lane & 15, kb = lane >> 4;
    if (nv == TILE) {
        const uint4* krow = reinterpret_cast<const uint4*>(kg + c * BROW + 32 * kb);
        const uint16_t* vl = vg + 4 * kb * BROW + 8 * c;
#pragma unroll
        for (int i = 0; i < 4; ++i) r.k[i] = krow[i];
#pragma unroll
        for (int e = 0; e < 4; ++e) r.v[e] = *reinterpret_cast<const uint4*>(vl + e * BROW);
    } else {
        const uint4* krow = reinterpret_cast<const uint4*>(kg + min(c, nv - 1) * BROW + 32 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.k[i] = krow[i];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            r.v[e] = *reinterpret_cast<const uint4*>(vg + min(4 * kb + e, nv - 1) * BROW + 8 * c);
    }
}

__device__ __forceinline__ void bf16_compute(WaveState& st, const Bf16Raw& r, const bf16x8 (&qop)[4], int nv,
                                             int lane, float qk) {
    const int kb = lane >> 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc = mfma_bf16(__builtin_bit_cast(bf16x8, r.k[i]), qop[i], acc);
    float s[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = (4 * kb + i < nv) ? acc[i] * qk : -INFINITY;
    softmax_step<4>(st, s, false);
    const u32x2 pw = {pack_bf16x2(s[0], s[1]), pack_bf16x2(s[2], s[3])};
    const bf16x4 pop = __builtin_bit_cast(bf16x4, pw);
    const uint32_t vd[4][4] = {{r.v[0].x, r.v[0].y, r.v[0].z, r.v[0].w}, {r.v[1].x, r.v[1].y, r.v[1].z, r.v[1].w},
                               {r.v[2].x, r.v[2].y, r.v[2].z, r.v[2].w}, {r.v[3].x, r.v[3].y, r.v[3].z, r.v[3].w}};
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
        const int dw = nb >> 1;
        const u32x2 w = {perm(vd[1][dw], vd[0][dw], sel), perm(vd[3][dw], vd[2][dw], sel)};
        st.acc[nb] = mfma_bf16_k16(__builtin_bit_cast(bf16x4, w), pop, st.acc[nb]);
    }
}

__global__ __launch_bounds__(THREADS, 2) void decode_partial_kernel(DecArgs a) {
    const int nh = a.bh_kv;
    const int head = blockIdx.x % nh;
    const int wg = blockIdx.x / nh;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, kb = lane >> 4;
    const int G = a.G;

    extern __shared__ float s_acc[];               // [WAVES][G][D+1]
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ __align__(16) uint16_t s_scl[WAVES][64];

    WaveState st;
    st.m = M_INIT;
    st.l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.ones = f32x4{0.f, 0.f, 0.f, 0.f};

    // Q row of head c (zero for padding columns): channels 32kb..32kb+31
    uint4 qraw[4] = {};
    if (c < G) {
        const uint4* qrow = reinterpret_cast<const uint4*>(a.q + static_cast<int64_t>(head * G + c) * a.q_stride + 32 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) qraw[i] = qrow[i];
    }

    if (wg < a.n16) {
        // ---------------- bf16 chunk: tiles wave, wave+WAVES ----------------
        int w = wg, seg = 0;
        while (seg < 2 && w >= a.nseg[seg]) { w -= a.nseg[seg]; ++seg; }
        const int lo = w * CHUNK16;
        const int hi = min(lo + CHUNK16, a.sn[seg]);
        const bf16x8 qop[4] = {__builtin_bit_cast(bf16x8, qraw[0]), __builtin_bit_cast(bf16x8, qraw[1]),
                               __builtin_bit_cast(bf16x8, qraw[2]), __builtin_bit_cast(bf16x8, qraw[3])};
        const uint16_t* kbase = a.sk[seg] + static_cast<int64_t>(head) * a.sk_bh[seg];
        const uint16_t* vbase = a.sv[seg] + static_cast<int64_t>(head) * a.sv_bh[seg];
        const int t0 = lo + wave * TILE;
        const int t1 = t0 + WAVES * TILE;
        Bf16Raw r0, r1;
        if (t0 < hi) bf16_load(r0, kbase + static_cast<int64_t>(t0) * BROW, vbase + static_cast<int64_t>(t0) * BROW,
                               min(TILE, hi - t0), lane);
        if (t1 < hi) bf16_load(r1, kbase + static_cast<int64_t>(t1) * BROW, vbase + static_cast<int64_t>(t1) * BROW,
                               min(TILE, hi - t1), lane);
        if (t0 < hi) bf16_compute(st, r0, qop, min(TILE, hi - t0), lane, a.qk_scale);
        if (t1 < hi) bf16_compute(st, r1, qop, min(TILE, hi - t1), lane, a.qk_scale);
    } else {
        // ---------------- int4 chunk: groups wave, wave+WAVES, ... ----------------
        const int lo = (wg - a.n16) * a.split;
        Int4Ctx x;
        x.hi = min(lo + a.split, a.n_quant);
        x.kbase = a.kp + static_cast<int64_t>(head) * a.kp_bh;
        x.vbase = a.vp + static_cast<int64_t>(head) * a.vp_bh;
        x.sbase = lane < 32 ? a.ks + static_cast<int64_t>(head) * a.ks_bh : a.vs + static_cast<int64_t>(head) * a.vs_bh;
        x.klane = static_cast<uint32_t>(c * PROW + 16 * kb);
        x.vlane = static_cast<uint32_t>(4 * kb * PROW + 4 * c);
        // full groups g = wave, wave+WAVES, ... < nfull go through a three-deep
        // register ring (two groups' loads in flight while one is computed);
        // the one partial group of a chunk, if any, is done last with clamping.
        constexpr int STRIDE = WAVES * GROUP;
        const int ntok = max(0, x.hi - lo);
        const int nfull = ntok / GROUP;
        const int tail = ntok - nfull * GROUP;
        const int nmine = nfull > wave ? (nfull - wave + WAVES - 1) / WAVES : 0;
        const int t0 = lo + wave * GROUP;
        // issue the first two groups' loads before anything waits on Q
        Int4Raw b0, b1, b2;
        if (nmine > 0) int4_load_full(b0, x, t0, lane);
        if (nmine > 1) int4_load_full(b1, x, t0 + STRIDE, lane);

        // Q -> fp16 in int4 slot order, pre-scaled by 2^-ex so |q| < 2^15
        float qf[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ww[4] = {qraw[i].x, qraw[i].y, qraw[i].z, qraw[i].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                qf[8 * i + 2 * j] = __uint_as_float(ww[j] << 16);
                qf[8 * i + 2 * j + 1] = __uint_as_float(ww[j] & 0xffff0000u);
            }
        }
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(qf[i]));
        amax = col_max(amax);
        const int ex = amax >= 16384.f ? ilogbf(amax) - 13 : 0;
        const float qscale = ldexpf(1.0f, -ex);
        f16x8 qop[4];
#pragma unroll
        for (int sidx = 0; sidx < 4; ++sidx) {
            const float* f = qf + 8 * sidx;
            const f16x8 v = {static_cast<_Float16>(f[0] * qscale), static_cast<_Float16>(f[4] * qscale),
                             static_cast<_Float16>(f[1] * qscale), static_cast<_Float16>(f[5] * qscale),
                             static_cast<_Float16>(f[2] * qscale), static_cast<_Float16>(f[6] * qscale),
                             static_cast<_Float16>(f[3] * qscale), static_cast<_Float16>(f[7] * qscale)};
            qop[sidx] = v;
        }
        const float qk = a.qk_scale * ldexpf(1.0f, ex);
        uint16_t* scl = s_scl[wave];
        for (int i = 0; i < nmine; i += 3) {
            const int t = t0 + i * STRIDE;
            if (i + 2 < nmine) int4_load_full(b2, x, t + 2 * STRIDE, lane);
            int4_compute<false>(st, b0, qop, scl, GROUP, lane, qk);
            if (i + 1 >= nmine) break;
            if (i + 3 < nmine) int4_load_full(b0, x, t + 3 * STRIDE, lane);
            int4_compute<false>(st, b1, qop, scl, GROUP, lane, qk);
            if (i + 2 >= nmine) break;
            if (i + 4 < nmine) int4_load_full(b1, x, t + 4 * STRIDE, lane);
            int4_compute<false>(st, b2, qop, scl, GROUP, lane, qk);
        }
        if (tail > 0 && wave == nfull % WAVES) {
            int4_load_tail(b0, x, lo + nfull * GROUP, tail, lane);
            int4_compute<true>(st, b0, qop, scl, tail, lane, qk);
        }
        // remove the +136 offset of the V codes: acc -= 136 * sum_t P'
        const float corr = 136.0f * st.ones[0];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) st.acc[nb] -= corr;
    }

    // ---- wave -> LDS ----------------------------------------------------------
    st.l = col_sum(st.l);
    if (kb == 0) {
        s_m[wave][c] = st.m;
        s_l[wave][c] = st.l;
    }
    if (c < G) {
        float* row = s_acc + (wave * G + c) * (D + 1);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) row[32 * kb + 8 * i + nb] = st.acc[nb][i];
    }
    __syncthreads();

    // ---- workgroup merge -> partial acc[G][D] and (m, l)[G] ---------------------
    const int64_t slot = static_cast<int64_t>(head) * a.nwg + wg;
    float* part = a.part + slot * G * D;
    for (int idx = threadIdx.x; idx < G * D; idx += THREADS) {
        const int g = idx / D, ch = idx % D;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
        float accv = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) accv += fast_exp2(s_m[w][g] - M) * s_acc[(w * G + g) * (D + 1) + ch];
        part[idx] = accv;
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
        float lv = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) lv += fast_exp2(s_m[w][g] - M) * s_l[w][g];
        a.ml[(slot * G + g) * 2] = M;
        a.ml[(slot * G + g) * 2 + 1] = lv;
    }
}

// ---------------------------------------------------------------------------
// merge: one workgroup per (KV head, MSLICE-channel slice)
// ---------------------------------------------------------------------------
constexpr int MERGE_PREFETCH = 8;        // partials per thread loaded before the first barrier

__global__ __launch_bounds__(MERGE_THREADS) void decode_merge_kernel(DecArgs a) {
    const int head = blockIdx.x / (D / MSLICE);
    const int ch0 = (blockIdx.x % (D / MSLICE)) * MSLICE;
    const int G = a.G;
    const int nwg = a.nwg;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    extern __shared__ float sm[];
    float* t_m = sm;                               // [nwg][G]
    float* t_l = sm + nwg * G;                     // [nwg][G]
    float* red = sm + 2 * nwg * G;                 // [slices][G][MSLICE]
    __shared__ float s_M[16], s_den[16];
    // thread -> (output o = g*MSLICE + channel, slice sl of the partials)
    const int outs = G * MSLICE;
    const int slices = max(1, MERGE_THREADS / outs);
    const int o = tid % outs, sl = tid / outs;
    const bool active = tid < outs * slices;
    const int g = o / MSLICE, ch = ch0 + o % MSLICE;
    const float* hp = a.part + (static_cast<int64_t>(head) * nwg * G + g) * D + ch;   // + w*G*D
    // the first MERGE_PREFETCH partials of this thread, issued before any wait
    float x[MERGE_PREFETCH];
#pragma unroll
    for (int j = 0; j < MERGE_PREFETCH; ++j) {
        const int w = sl + j * slices;
        x[j] = (active && w < nwg) ? hp[static_cast<int64_t>(w) * G * D] : 0.f;
    }
    const float* ml = a.ml + static_cast<int64_t>(head) * nwg * G * 2;
    for (int idx = tid; idx < nwg * G; idx += MERGE_THREADS) {
        t_m[idx] = ml[2 * idx];
        t_l[idx] = ml[2 * idx + 1];
    }
    __syncthreads();
    for (int gg = wave; gg < G; gg += MERGE_THREADS / 64) {
        float M = M_INIT;
        for (int w = lane; w < nwg; w += 64) M = fmaxf(M, t_m[w * G + gg]);
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) M = fmaxf(M, __shfl_xor(M, off, 64));
        float den = 0.f;
        for (int w = lane; w < nwg; w += 64) den += fast_exp2(t_m[w * G + gg] - M) * t_l[w * G + gg];
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) den += __shfl_xor(den, off, 64);
        if (lane == 0) {
            s_M[gg] = M;
            s_den[gg] = den;
        }
    }
    __syncthreads();
    if (active) {
        const float M = s_M[g];
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < MERGE_PREFETCH; ++j) {
            const int w = sl + j * slices;
            if (w < nwg) acc += fast_exp2(t_m[w * G + g] - M) * x[j];
        }
        for (int w = sl + MERGE_PREFETCH * slices; w < nwg; w += slices)
            acc += fast_exp2(t_m[w * G + g] - M) * hp[static_cast<int64_t>(w) * G * D];
        red[sl * outs + o] = acc;
    }
    __syncthreads();
    if (tid < outs) {
        float num = 0.f;
        for (int k = 0; k < slices; ++k) num += red[k * outs + tid];
        const float den = s_den[g];
        const float r = den > 0.f ? num / den : 0.f;
        a.out[static_cast<int64_t>(head * G + g) * a.out_stride + ch] = f32_to_bf16_rne(r);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct Plan {
    int split, n4, nseg[3], n16, nwg;
};

// int4 tokens per workgroup: at least one 32-token group per wavefront, at
// most ~32 partials per head (bounded merge traffic), and enough workgroups
// (~2048) to cover the 256 CUs several times when the batch is small.
int choose_split(int64_t n_quant, int bh_kv, int requested) {
    auto round_up = [](int64_t x, int64_t m) { return ((x + m - 1) / m) * m; };
    if (requested > 0) return static_cast<int>(round_up(requested, CHUNK4_MIN));
    int64_t split = CHUNK4_MIN;
    split = std::max<int64_t>(split, round_up((n_quant + 31) / 32, CHUNK4_MIN));
    split = std::max<int64_t>(split, round_up((n_quant * bh_kv + 2047) / 2048, CHUNK4_MIN));
    return static_cast<int>(std::min<int64_t>(split, 1 << 30));
}

Plan make_plan(int64_t n_quant, const int64_t seg_n[3], int bh_kv, int G, int requested) {
    Plan p;
    p.split = choose_split(n_quant, bh_kv, requested);
    p.n16 = 0;
    for (int s = 0; s < 3; ++s) {
        p.nseg[s] = static_cast<int>((seg_n[s] + CHUNK16 - 1) / CHUNK16);
        p.n16 += p.nseg[s];
    }
    // keep nwg * G within the merge tables
    while (true) {
        p.n4 = static_cast<int>((n_quant + p.split - 1) / p.split);
        p.nwg = p.n4 + p.n16;
        if (static_cast<int64_t>(p.nwg) * G <= MAX_PARTIALS || p.n4 <= 1) break;
        p.split *= 2;
    }
    return p;
}

size_t partial_lds_bytes(int G) { return static_cast<size_t>(WAVES) * G * (D + 1) * sizeof(float); }

size_t merge_lds_bytes(const Plan& pl, int G) {
    const int outs = G * MSLICE;
    const int slices = std::max(1, MERGE_THREADS / outs);
    return (2 * static_cast<size_t>(pl.nwg) * G + static_cast<size_t>(slices) * outs) * sizeof(float);
}

size_t workspace_bytes(const Plan& pl, int bh_kv, int G) {
    const size_t slots = static_cast<size_t>(bh_kv) * std::max(pl.nwg, 1) * G;
    const size_t part = ((slots * D * sizeof(float) + 255) / 256) * 256;
    return part + slots * 2 * sizeof(float);
}

int validate(const hyq_decode_params* p) {
    if (!p) return fail(HYQ_EINVAL, "null params");
    if (p->head_dim != D) return fail(HYQ_ENOTSUP, "head_dim must be 128, got " + std::to_string(p->head_dim));
    if (p->k_bits != 4 || p->v_bits != 4)
        return fail(HYQ_ENOTSUP, "only K4V4 is implemented (k_bits=" + std::to_string(p->k_bits) +
                                     ", v_bits=" + std::to_string(p->v_bits) + ")");
    if (p->kv_repeat < 1 || p->kv_repeat > 16)
        return fail(HYQ_ENOTSUP, "kv_repeat must be in [1, 16], got " + std::to_string(p->kv_repeat));
    if (p->bh_kv < 0) return fail(HYQ_EINVAL, "bh_kv < 0");
    if (p->bh_kv > (1 << 24)) return fail(HYQ_ENOTSUP, "bh_kv too large");
    if (p->n_quant < 0 || p->n_quant > (1 << 30)) return fail(HYQ_EINVAL, "bad n_quant");
    if (p->bh_kv == 0) return HYQ_OK;
    if (!p->q || !p->out) return fail(HYQ_EINVAL, "null q/out");
    if (!aligned(p->q, 16) || p->q_stride % 8) return fail(HYQ_EINVAL, "q must be 16-byte aligned, row stride % 8 == 0");
    if (!aligned(p->out, 2)) return fail(HYQ_EINVAL, "out misaligned");
    if (p->n_quant > 0) {
        if (!p->k_packed || !p->v_packed || !p->k_scale || !p->v_scale) return fail(HYQ_EINVAL, "null prefix tensor");
        if (p->kp_stride_n != PROW || p->vp_stride_n != PROW)
            return fail(HYQ_EINVAL, "packed K/V rows must be contiguous (token stride 64 bytes)");
        if (!aligned(p->k_packed, 16) || p->kp_stride_bh % 16)
            return fail(HYQ_EINVAL, "k_packed must be 16-byte aligned with a 16-byte head stride");
        if (!aligned(p->v_packed, 4) || p->vp_stride_bh % 4)
            return fail(HYQ_EINVAL, "v_packed must be 4-byte aligned with a 4-byte head stride");
        if (!aligned(p->k_scale, 2) || !aligned(p->v_scale, 2))
            return fail(HYQ_EINVAL, "scales must be 2-byte aligned");
    }
    for (int s = 0; s < 3; ++s) {
        if (p->seg_n[s] < 0 || p->seg_n[s] > (1 << 30)) return fail(HYQ_EINVAL, "bad segment length");
        if (p->seg_n[s] == 0) continue;
        if (!p->seg_k[s] || !p->seg_v[s]) return fail(HYQ_EINVAL, "null bf16 segment");
        if (p->seg_k_stride_n[s] != BROW || p->seg_v_stride_n[s] != BROW)
            return fail(HYQ_EINVAL, "bf16 segment rows must be contiguous (token stride = head_dim)");
        if (!aligned(p->seg_k[s], 16) || !aligned(p->seg_v[s], 16) || p->seg_k_stride_bh[s] % 8 ||
            p->seg_v_stride_bh[s] % 8)
            return fail(HYQ_EINVAL, "bf16 segments must be 16-byte aligned with head strides % 8 == 0");
    }
    return HYQ_OK;
}

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" size_t hyq_decode_workspace_size(const hyq_decode_params* p) {
    if (validate(p) != HYQ_OK) return 0;
    const Plan pl = make_plan(p->n_quant, p->seg_n, p->bh_kv, p->kv_repeat, p->split_tokens);
    return workspace_bytes(pl, p->bh_kv, p->kv_repeat);
}

extern "C" int hyq_decode_hybrid(const hyq_decode_params* p, void* workspace, size_t ws_bytes, void* stream) {
    int rc = validate(p);
    if (rc != HYQ_OK) return rc;
    if (p->bh_kv == 0) return HYQ_OK;
    const Plan pl = make_plan(p->n_quant, p->seg_n, p->bh_kv, p->kv_repeat, p->split_tokens);
    if (pl.nwg == 0) return fail(HYQ_EINVAL, "decode with zero key tokens");
    if (static_cast<int64_t>(pl.nwg) * p->kv_repeat > MAX_PARTIALS)
        return fail(HYQ_ENOTSUP, "too many bf16 chunks per head for the merge tables");
    const size_t need = workspace_bytes(pl, p->bh_kv, p->kv_repeat);
    if (!workspace || ws_bytes < need || !aligned(workspace, 256))
        return fail(HYQ_ENOSPC, "decode workspace too small or misaligned: need " + std::to_string(need) + " bytes");
    DecArgs a{};
    a.q = p->q; a.q_stride = p->q_stride;
    a.out = p->out; a.out_stride = p->out_stride;
    a.kp = reinterpret_cast<const uint8_t*>(p->k_packed); a.kp_bh = p->kp_stride_bh; a.kp_n = p->kp_stride_n;
    a.vp = reinterpret_cast<const uint8_t*>(p->v_packed); a.vp_bh = p->vp_stride_bh; a.vp_n = p->vp_stride_n;
    a.ks = p->k_scale; a.ks_bh = p->ks_stride_bh;
    a.vs = p->v_scale; a.vs_bh = p->vs_stride_bh;
    a.n_quant = static_cast<int32_t>(p->n_quant);
    for (int s = 0; s < 3; ++s) {
        a.sk[s] = p->seg_k[s]; a.sv[s] = p->seg_v[s];
        a.sk_bh[s] = p->seg_k_stride_bh[s]; a.sk_n[s] = p->seg_k_stride_n[s];
        a.sv_bh[s] = p->seg_v_stride_bh[s]; a.sv_n[s] = p->seg_v_stride_n[s];
        a.sn[s] = static_cast<int32_t>(p->seg_n[s]);
        a.nseg[s] = pl.nseg[s];
    }
    a.G = p->kv_repeat;
    a.bh_kv = p->bh_kv;
    a.qk_scale = p->sm_scale * LOG2E;
    a.split = pl.split; a.n4 = pl.n4; a.n16 = pl.n16; a.nwg = pl.nwg;
    const size_t slots = static_cast<size_t>(p->bh_kv) * pl.nwg * p->kv_repeat;
    const size_t part_bytes = ((slots * D * sizeof(float) + 255) / 256) * 256;
    a.part = static_cast<float*>(workspace);
    a.ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + part_bytes);
    const int64_t blocks = static_cast<int64_t>(pl.nwg) * p->bh_kv;
    if (blocks > 0x7fffffffLL) return fail(HYQ_ENOTSUP, "grid too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    decode_partial_kernel<<<dim3(static_cast<unsigned>(blocks)), dim3(THREADS), partial_lds_bytes(p->kv_repeat), s>>>(a);
    rc = check_launch("hyq_decode_hybrid (partial)");
    if (rc != HYQ_OK) return rc;
    decode_merge_kernel<<<dim3(static_cast<unsigned>(p->bh_kv * (D / MSLICE))), dim3(MERGE_THREADS),
                          merge_lds_bytes(pl, p->kv_repeat), s>>>(a);
    return check_launch("hyq_decode_hybrid (merge)");
}

extern "C" size_t hyq_decode_bf16_workspace_size(int32_t bh_kv, int32_t kv_repeat, int64_t n, int32_t d) {
    if (bh_kv < 0 || kv_repeat < 1 || kv_repeat > 16 || d != D || n < 0) return 0;
    const int64_t seg_n[3] = {n, 0, 0};
    const Plan pl = make_plan(0, seg_n, bh_kv, kv_repeat, 0);
    return workspace_bytes(pl, bh_kv, kv_repeat);
}

extern "C" int hyq_decode_bf16(const uint16_t* q, int64_t q_stride, uint16_t* out, int64_t out_stride,
                               const uint16_t* k, int64_t k_stride_bh, int64_t k_stride_n,
                               const uint16_t* v, int64_t v_stride_bh, int64_t v_stride_n,
                               int64_t n, int32_t bh_kv, int32_t kv_repeat, int32_t d, float sm_scale,
                               void* workspace, size_t workspace_bytes, void* stream) {
    hyq_decode_params p{};
    p.q = q; p.q_stride = q_stride; p.out = out; p.out_stride = out_stride;
    p.seg_k[0] = k; p.seg_k_stride_bh[0] = k_stride_bh; p.seg_k_stride_n[0] = k_stride_n;
    p.seg_v[0] = v; p.seg_v_stride_bh[0] = v_stride_bh; p.seg_v_stride_n[0] = v_stride_n;
    p.seg_n[0] = n;
    p.bh_kv = bh_kv; p.kv_repeat = kv_repeat; p.head_dim = d; p.k_bits = 4; p.v_bits = 4;
    p.sm_scale = sm_scale;
    return hyq_decode_hybrid(&p, workspace, workspace_bytes, stream);
}
