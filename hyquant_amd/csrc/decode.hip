// Fused four-segment hybrid decode attention for gfx950 (MI355X).
//
// Math (fused_d_stage_decode, src/ops/decode_d_stage.py:916-1005, split-K
// kernels :481-782): for each query head, one online softmax (log2 domain,
// scale sm_scale*log2e) over [int4 prefix | top-k | staging | window].  On the
// int4 prefix the per-token K scale is factored out of the dot product,
// s = (q . k_code) * s_k, and P is rounded to bf16 after multiplying by the
// per-token V scale, P' = bf16(p * s_v), before P' . v_code (F8).
//
// One launch per step.  A workgroup of 4 wavefronts owns one piece of one KV
// head (all G query heads of the GQA group ride along as MFMA columns); the
// grid is (KV heads, pieces per head).  A head's keys are laid end to end as
// schedule units, int4 groups of 32 tokens and then bf16 units of 8 tokens
// of each segment, and the host cuts them into `nwg` pieces, each inside one
// segment and of about equal bytes within it (make_plan); the cut points
// travel in the kernel arguments.  With many KV heads the pieces are sized
// so that the grid is about 1.25 rounds of the resident workgroup slots.  In
// a piece:
//   its int4 tokens are walked in 32-token groups (wavefront w takes groups
//     w, w+4, ...) through a three-deep register ring, so two groups' loads
//     are in flight while one is computed;
//   the tokens of each bf16 segment it reaches are walked in 16-token tiles
//     (wavefront w takes tiles w, w+4, ...) through a two-deep register ring.
// Every load goes through a buffer descriptor whose range is the piece's part
// of the segment (past the end reads zeros), so the rings' loads are
// unconditional and their wait counts exact; the loop position travels in the
// scalar offset.
//
// The four wavefronts' (m, l, acc) are merged in LDS and the workgroup writes
// one partial with device-scope stores (write-through to the device coherence
// point), waits for them, and counts itself in on its head's arrival counter.
// The workgroup that arrives last merges the head's partials (one wavefront
// per query head; see merge_head_waves) and resets the counter to zero, so the
// counters are zero again when the launch ends.  No fence is needed: the
// partials never sit dirty in a per-XCD L2, and the merge reads them with
// device-scope loads.
//
// Per wavefront, lane l = 16*kb + c (c = l & 15, kb = l >> 4):
//   PV  O^T[channel][g] = V^T . P'^T with v_mfma_f32_16x16x32_bf16:
//       A = 16 channels x 32 token slots, B = P'^T.  Slot e of lane-row kb
//       is token 4e + kb of the 32-token group, so V load e of the wavefront
//       reads four consecutive packed rows 4e..4e+3 (whole 128-byte lines).
//   QK  S^T[token][g] = K_tile . Q^T with v_mfma_f32_16x16x32_{f16,bf16}:
//       A = 16 tokens x 32 channels, B = Q^T (lane = head c).  Row i of tile
//       t is token 16t + 4(i & 3) + (i >> 2), so output lane (g = c, kb),
//       which holds rows 4kb..4kb+3, holds tokens 16t + 4i + kb: exactly the
//       P' slots 4t + i of its lane-row.  No cross-lane shuffle of P.
//   Channel 8*j+nb of V sits in row j of PV MFMA nb (lane j loads the dword /
//   16 bytes holding channels 8j..8j+7).  bf16 tiles use the K=16 form
//   (v_mfma_f32_16x16x16_bf16) whose slot e of lane-row kb is token 4kb+e.
//   Lane i of a quad loads the K and V scales of token 16t + 4i + kb of a
//   tile and quad-broadcast DPP moves hand every lane all four.
//   Loads whose instructions cover whole 128-byte lines are non-temporal:
//   the quantised prefix's packed rows and the bf16 tiles' V rows.  This
//   raised a loads-only copy of the prefix schedule from 75% to 82% of HBM
//   peak, the kernel at B=16, 32K from 66% to 81% and the bf16-only
//   comparator from 72% to 80%.  Loads that read a line in pieces from
//   several instructions (the scales, the bf16 tiles' K rows) were slower
//   non-temporal and keep the default policy.
// int4 -> MFMA operand conversion is done in registers without any lookup:
//   K: u = nibble ^ 8 placed in the mantissa of an fp16 subnormal (value
//      u * 2^-24, one shift and one bitop3 per pair of codes); Q is fed as
//      fp16, pre-scaled by a power of two so every bf16 query value is
//      exact, every product is exact in fp32, and the QK accumulators start
//      at -2^-24 * 8 * sum(q) so that they end at 2^-24 * q . code.
//   V: nibble ^ 8 -> bf16(128 + u); the constant 136 is removed after the
//      product with a ninth MFMA against an all-ones operand, which yields
//      sum_t P'[g][t] rounded exactly as the main product.
#include "hyq_common.h"

#include <algorithm>
#include <atomic>
#include <mutex>
#include <string>

namespace hyq {
namespace {

constexpr int D = 128;
constexpr int WAVES = 4;                 // wavefronts per workgroup
constexpr int THREADS = 64 * WAVES;
constexpr int GROUP = 32;                // int4 tokens per wavefront iteration
constexpr int TILE = 16;                 // bf16 tokens per wavefront iteration
constexpr int BUNIT = 8;                 // bf16 tokens per schedule unit (an int4 unit is a GROUP)
constexpr float LOG2E = 1.44269504f;     // src/ops/decode_d_stage.py:17
constexpr float RESCALE_SLACK = 8.0f;    // lazy max update threshold (log2 units)
constexpr float M_INIT = -1.0e30f;
constexpr int MAX_PARTIALS = 1024;       // nwg * G bound
constexpr int MAX_NWG = 256;             // chunks per head (merge weight table)
constexpr int CNT_PAD = 32;              // arrival counters 128 bytes apart
constexpr int CNT_CAP = 16384;           // counter slots at the head of every workspace (bh_kv bound)

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Kernel arguments.  The first PRO_DWORDS dwords are everything the
// prologue needs before its first loads; decode_kernel reads them, with its
// piece's two entries of bnd, in one batch of scalar loads (kernel_args), so
// their layout is fixed: pointers on 8-byte boundaries, the rest 32-bit (row
// and head strides fit 31 bits, checked on the host).
struct DecArgs {
    const uint16_t* q;     // dwords 0-1
    const uint8_t* kp;     // 2-3
    const uint8_t* vp;     // 4-5
    const uint16_t* ks;    // 6-7
    const uint16_t* vs;    // 8-9
    const uint16_t* sk[3]; // 10-15
    const uint16_t* sv[3]; // 16-21
    const int32_t* len_q;  // 22-23  optional per-head valid prefix tokens
    const int32_t* len_s0; // 24-25  optional per-head valid tokens of segment 0
    int32_t q_stride;      // 26
    int32_t kp_bh, vp_bh, ks_bh, vs_bh;   // 27-30
    int32_t sk_bh[3];      // 31-33
    int32_t sv_bh[3];      // 34-36
    int32_t n_quant;       // 37
    int32_t sn[3];         // 38-40
    int32_t G;             // 41
    int32_t nqg;           // 42     int4 schedule units (GROUP tokens) per head
    int32_t segu[2];       // 43-44  bf16 schedule units (BUNIT tokens) of segments 0 and 1
    float qk_scale;        // 45     sm_scale * log2(e)
    int32_t io;            // 46     HYQ_DT_* flags: fp16 q / fp16 segments / fp16 out
    int32_t pad0;          // 47
    // used once the stream is done (loaded with the prologue block, waited
    // for after the stream)
    uint16_t* out;         // 48-49
    float* part;           // 50-51  [bh_kv][nwg][G][D] partial numerators
    float* ml;             // 52-53  [bh_kv][nwg][G][2] = (m, l)
    uint32_t* cnt;         // 54-55  arrival counter of head h at cnt[h * CNT_PAD]
    int32_t out_stride;    // 56
    int32_t nwg;           // 57     pieces (workgroups) per head
    int32_t mj;            // 58     merge batch: partial columns per merging thread and load batch
    int32_t bh_kv;         // 59
    int32_t bnd[MAX_NWG + 1];  // piece p: schedule units [bnd[p], bnd[p+1]) of its head
};
constexpr int PRO_DWORDS = 48;
static_assert(offsetof(DecArgs, pad0) == 4 * (PRO_DWORDS - 1), "prologue block layout");
static_assert(offsetof(DecArgs, bh_kv) == 4 * 59, "epilogue block layout");

typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x8 __attribute__((ext_vector_type(8)));

// The prologue block of the kernel arguments and this piece's bounds
// (bnd[wg], bnd[wg + 1]) in one batch of scalar loads with one wait: left to
// the compiler, they came in two batches (two round trips) before the first
// vector load.  The epilogue block's loads are issued right after, into
// registers of their own, and waited for by epilogue_args once the stream is
// done (the compiler does not see these loads: its own lgkmcnt waits only
// over-wait for them).
struct KArgs {
    u32x16 a, b, c;
    u32x2 bnd;
    u32x8 e0;              // dwords 48-55
    u32x4 e1;              // dwords 56-59
};
__device__ __forceinline__ KArgs kernel_args(int wg) {
    const char* const base = (const char*)__builtin_amdgcn_kernarg_segment_ptr();
    const char* const bp = base + offsetof(DecArgs, bnd) + 4 * wg;
    KArgs k;
    asm volatile(
        "s_load_dwordx16 %0, %4, 0x0\n\t"
        "s_load_dwordx16 %1, %4, 0x40\n\t"
        "s_load_dwordx16 %2, %4, 0x80\n\t"
        "s_load_dwordx2 %3, %5, 0x0\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&s"(k.a), "=&s"(k.b), "=&s"(k.c), "=&s"(k.bnd)
        : "s"(base), "s"(bp)
        : "memory");
    asm volatile(
        "s_load_dwordx8 %0, %2, 0xc0\n\t"
        "s_load_dwordx4 %1, %2, 0xe0"
        : "=&s"(k.e0), "=&s"(k.e1)
        : "s"(base));
    return k;
}
__device__ __forceinline__ void epilogue_args(KArgs& k) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+s"(k.e0), "+s"(k.e1)::"memory");
}
// dword i of the prologue block
__device__ __forceinline__ uint32_t kdw(const KArgs& k, int i) {
    return i < 16 ? k.a[i] : i < 32 ? k.b[i - 16] : k.c[i - 32];
}
template <typename T>
__device__ __forceinline__ T* kptr(const KArgs& k, int i) {
    return reinterpret_cast<T*>(static_cast<uintptr_t>(kdw(k, i)) | (static_cast<uintptr_t>(kdw(k, i + 1)) << 32));
}
template <typename T>
__device__ __forceinline__ T* eptr(const KArgs& k, int i) {
    return reinterpret_cast<T*>(static_cast<uintptr_t>(k.e0[i]) | (static_cast<uintptr_t>(k.e0[i + 1]) << 32));
}

// ---------------------------------------------------------------------------
// Phase trace (built only with -DHYQ_PHASE_TRACE, into a separate library:
// `python -m hyquant_amd.build --trace`).  Every wavefront reads
// s_memrealtime (a 100 MHz clock common to every XCD) at the phase points
// below, keeps the stamps in SGPRs and stores them once at its end, into a
// ring of the last TRACE_SLOTS launches (one record per wavefront).  The
// workgroup that finishes a launch last advances the ring.
// ---------------------------------------------------------------------------
#ifdef HYQ_PHASE_TRACE
constexpr int TRACE_SLOTS = 32;
constexpr int TRACE_MAX_WG = 4096;
constexpr int TRACE_PH = 14;
//  0 entry                       7 arrival counter returned
//  1 kernel arguments loaded
//  2 Q arrived                   8 merge: (m, l) arrived       (merging
//  3 first K/V group arrived     9 merge: partials summed       wavefronts of
//  4 own stream done            10 merge: output acked          G <= 4 heads;
//  5 all four wavefronts in LDS 11 merge: entered               else 0)
//  6 partial stored, acknowledged 12 merge: loads issued
//                               13 launch index (not a time)
__device__ uint64_t g_trace[TRACE_SLOTS][TRACE_MAX_WG * 4][TRACE_PH];
__device__ uint32_t g_trace_launch;
__device__ uint32_t g_trace_done;
#define HYQ_STAMP(i) (ph[i] = __builtin_amdgcn_s_memrealtime())
#define TRACE_PARAM , uint64_t (&ph)[TRACE_PH]
#define TRACE_ARG , ph
#else
#define HYQ_STAMP(i) ((void)0)
#define TRACE_PARAM
#define TRACE_ARG
#endif

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


// NB: operand vectors are always assembled from scalars with a brace list;
// element-wise stores into an ext_vector inside unrolled loops were
// miscompiled (every element received element 0).

// nibble pair (s, s+16) of x, offset to u = code + 8 and tagged with a magic
// exponent: ((x >> s) & 0x000f000f) ^ (0x00080008 | magic).
__device__ __forceinline__ uint32_t nib2(uint32_t x, int s, uint32_t magic_xor) {
    return ((x >> s) & 0x000f000fu) ^ magic_xor;
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

// q.to(bf16) of an fp16 query (mask all ones) or the bf16 query unchanged
// (mask zero), without a branch: a branch here made the compiler wait for the
// Q loads at its join, before the first K/V loads were issued, which put the
// whole Q round trip in front of the K/V stream.  Called after those loads;
// the empty asm statements keep the compiler from hoisting the conversion
// (and so the wait for Q) above them.
__device__ __forceinline__ void q_to_bf16(u32x4 (&q)[4], uint32_t mask) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t w[4] = {q[i][0], q[i][1], q[i][2], q[i][3]};
        asm volatile("" : "+v"(w[0]), "+v"(w[1]), "+v"(w[2]), "+v"(w[3]));
        q[i] = u32x4{(f16x2_to_bf16x2(w[0]) & mask) | (w[0] & ~mask), (f16x2_to_bf16x2(w[1]) & mask) | (w[1] & ~mask),
                     (f16x2_to_bf16x2(w[2]) & mask) | (w[2] & ~mask), (f16x2_to_bf16x2(w[3]) & mask) | (w[3] & ~mask)};
    }
}

// One int32 through the scalar cache (a wave-uniform address written before
// the launch): a vector load there would be waited for with vmcnt(0), which
// also waits for the Q loads already in flight.
__device__ __forceinline__ int sload_i32(const int32_t* p) {
    int v;
    asm volatile("s_load_dword %0, %1, 0x0\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
    return v;
}
__device__ __forceinline__ float col_sum(float v) {
    auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// token slot e of lane-row kb within a 32-token group
__device__ __forceinline__ constexpr int slot_token(int kb, int e) { return 4 * e + kb; }
// token of row i of a 16-token QK tile (relative to the tile)
__device__ __forceinline__ constexpr int krow_token(int i) { return 4 * (i & 3) + (i >> 2); }

// Online-softmax update with this lane's N log2-domain scores; on return s
// holds p = exp2(s - m) relative to the (possibly raised) running max.
template <int N>
__device__ __forceinline__ void softmax_step(WaveState& st, float (&s)[N], bool has_ones) {
    // this lane's max (plain v_max3 steps), tested against the running max
    // on its own: st.m is the same on the four lanes of a column, so some
    // lane passes exactly when the column max does, and the column max (two
    // row swaps) is formed only when the running max moves
    float mx = s[0];
    int e = 1;
#pragma unroll
    for (; e + 1 < N; e += 2) mx = vmax3(mx, s[e], s[e + 1]);
    if (e < N) mx = vmax2(mx, s[e]);
    if (__builtin_amdgcn_ballot_w64(mx > st.m + RESCALE_SLACK)) {   // rare after the first group
        mx = col_max(mx);
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
// Every load goes through a buffer descriptor whose range is the chunk, so a
// token past the chunk end reads zeros without touching memory: the loads of
// the ring are unconditional, which keeps the compiler's wait counts exact
// (a load under a branch makes every later wait a full drain).
typedef __amdgpu_buffer_rsrc_t Rsrc;
constexpr int RSRC_W3 = 0x00020000;      // raw buffer, 32-bit data format

__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, RSRC_W3);
}
// voff: per-lane byte offset (constant across a loop), soff: wave-uniform
// byte offset (the loop position, kept in an SGPR); POL: cache policy bits
// (NT: non-temporal, for data read once)
constexpr int NT = 2;
template <int POL = 0>
__device__ __forceinline__ u32x4 bld128(Rsrc r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, POL));
}
template <int POL = 0>
__device__ __forceinline__ uint32_t bld32(Rsrc r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, POL);
}
template <int POL = 0>
__device__ __forceinline__ u32x2 bld64(Rsrc r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, POL));
}
template <int POL = 0>
__device__ __forceinline__ uint32_t bld16(Rsrc r, uint32_t voff, uint32_t soff = 0) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, POL);
}

template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(v), CTRL, 0xf, 0xf, false));
}

// Quantised prefix with KB-bit K codes and VB-bit V codes (2, 4 or 8; packed
// rows of 16*bits bytes, src/ops/decode_d_stage.py:104-133).  Per lane:
//   k[t][*]  tile t: token 16t + krow_token(c), channels 32kb..32kb+31 (KB dwords)
//   v[e][*]  slot e: token slot_token(kb, e) = 4e + kb, channels 8c..8c+7 (VB
//            bytes; 2-byte loads are zero-extended)
//   sk, sv   tile t: fp16 scale bits of token 16t + 4(c & 3) + kb
template <int KB, int VB>
struct QRaw {
    uint32_t k[2][KB];
    uint32_t v[8][VB == 8 ? 2 : 1];
    uint32_t sk[2], sv[2];
};

constexpr int prow(int bits) { return 16 * bits; }   // packed bytes per token (D = 128)
constexpr int BROW = D;                   // bf16 row stride in elements

struct QCtx {
    Rsrc k, v, ks, vs;     // this chunk's packed K / V rows and scales
    uint32_t klane;        // lane offset of tile 0: krow_token(c) * prow(KB) + 4 KB kb
    uint32_t vlane;        // lane offset of slot 0: kb * prow(VB) + VB c
    uint32_t slane;        // lane offset of the scale of tile 0: (4 (c & 3) + kb) * 2
};

// t0 is wave-uniform: it only enters the scalar offsets
template <int KB, int VB>
__device__ __forceinline__ void qload(QRaw<KB, VB>& r, const QCtx& x, int t0) {
    const uint32_t sok = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t0) * prow(KB));
    const uint32_t sov = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t0) * prow(VB));
    const uint32_t ss = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t0) * 2);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t ko = x.klane + t * 16 * prow(KB);
        if constexpr (KB == 2) {
            const u32x2 w = bld64<NT>(x.k, ko, sok);
            r.k[t][0] = w[0]; r.k[t][1] = w[1];
        } else {
#pragma unroll
            for (int h = 0; h < KB / 4; ++h) {
                const u32x4 w = bld128<NT>(x.k, ko + 16 * h, sok);
                r.k[t][4 * h] = w[0]; r.k[t][4 * h + 1] = w[1]; r.k[t][4 * h + 2] = w[2]; r.k[t][4 * h + 3] = w[3];
            }
        }
    }
    // scales (in the order qcompute uses them: after the K tiles, before the
    // V rows): a 128-byte line of them is read by several instructions, so
    // they keep the default cache policy
    r.sk[0] = bld16(x.ks, x.slane, ss);
    r.sk[1] = bld16(x.ks, x.slane + 32, ss);
    r.sv[0] = bld16(x.vs, x.slane, ss);
    r.sv[1] = bld16(x.vs, x.slane + 32, ss);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const uint32_t vo = x.vlane + slot_token(0, e) * prow(VB);
        if constexpr (VB == 2) {
            r.v[e][0] = bld16<NT>(x.v, vo, sov);
        } else if constexpr (VB == 4) {
            r.v[e][0] = bld32<NT>(x.v, vo, sov);
        } else {
            const u32x2 w = bld64<NT>(x.v, vo, sov);
            r.v[e][0] = w[0]; r.v[e][1] = w[1];
        }
    }
}

// QK A operand of MFMA m (channels 32kb + 8m + [0..7]) in slot order
// [c0,c4,c1,c5,c2,c6,c3,c7], the order of the Q operands, as fp16
// subnormals whose bits are the offset-binary code u = code + 2^(KB-1):
// the value is u * 2^-24 exactly, so every product with the fp16 query is
// exact in fp32 and the MFMA yields 2^-24 (q . code + 2^(KB-1) sum(q)).  The
// second term is the same for every token of a query column: the QK
// accumulators start at minus that bias (kbias, one MFMA product per piece),
// which leaves 2^-24 q . code.
//   4 bits: (nibble ^ 8) pairs (s, s + 16) of one dword
//   8 bits: byte j of the two dwords paired by one perm, ^ 0x80
//   2 bits: the two bytes of the 16-bit half spread to the two fp16 halves by
//           one perm, crumbs ^ 2
template <int KB>
__device__ __forceinline__ f16x8 k_operand(const uint32_t (&k)[KB], int m) {
    if constexpr (KB == 4) {
        const uint32_t x = k[m];
        const u32x4 o = {nib2(x, 0, 0x00080008u), nib2(x, 4, 0x00080008u), nib2(x, 8, 0x00080008u),
                         nib2(x, 12, 0x00080008u)};
        return __builtin_bit_cast(f16x8, o);
    } else if constexpr (KB == 8) {
        const uint32_t lo = k[2 * m], hi = k[2 * m + 1];
        const u32x4 o = {perm(hi, lo, 0x0c040c00u) ^ 0x00800080u, perm(hi, lo, 0x0c050c01u) ^ 0x00800080u,
                         perm(hi, lo, 0x0c060c02u) ^ 0x00800080u, perm(hi, lo, 0x0c070c03u) ^ 0x00800080u};
        return __builtin_bit_cast(f16x8, o);
    } else {
        const uint32_t w = k[m >> 1];
        const uint32_t y = (m & 1) ? perm(w, w, 0x0c030c02u) : perm(w, w, 0x0c010c00u);
        const u32x4 o = {((y >> 0) & 0x00030003u) ^ 0x00020002u, ((y >> 2) & 0x00030003u) ^ 0x00020002u,
                         ((y >> 4) & 0x00030003u) ^ 0x00020002u, ((y >> 6) & 0x00030003u) ^ 0x00020002u};
        return __builtin_bit_cast(f16x8, o);
    }
}

// Minus the K operand's offset term of each query column, -2^-24 2^(KB-1)
// sum_d q_d, as the MFMA forms it: the product of an all-offset K tile (every
// slot the subnormal 2^(KB-1) * 2^-24) with the Q operands.  Lane (c, kb)
// gets column c in all four entries.
template <int KB>
__device__ __forceinline__ f32x4 k_bias(const f16x8 (&qop)[4]) {
    constexpr uint32_t half = 1u << (KB - 1);
    const u32x4 w = {half | half << 16, half | half << 16, half | half << 16, half | half << 16};
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = mfma_f16(__builtin_bit_cast(f16x8, w), qop[m], acc);
    return -acc;
}

// The constant the PV operands add to every V code (removed at the end with
// the all-ones product): bf16(128 + u) operands, u = code + 8 (4 bits),
// code + 2 (2 bits); 8-bit codes are split into their nibbles,
// bf16(128 + lo) + bf16(16 (128 + (hi ^ 8))) = code + 2304.
template <int VB>
constexpr float v_offset() { return VB == 4 ? 136.0f : VB == 2 ? 130.0f : 2304.0f; }

// x of lane i of this lane's quad (a DPP quad broadcast, which the compiler
// folds into the VOP2 instruction that consumes it)
template <int I>
__device__ __forceinline__ float quad_bcast(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), I * 0x55, 0xf, 0xf, true));
}

template <int KB, int VB>
__device__ __forceinline__ void qcompute(WaveState& st, const QRaw<KB, VB>& r, const f16x8 (&qop)[4],
                                         const f32x4& kbias, int nv, int lane, float qk) {
    const int kb = lane >> 4;
    // each lane converts the scales of its own token of each tile (lane i of
    // a quad holds token 16t + 4i + kb, the token of score slot 4t + i); the
    // scores and P' take them with quad broadcasts
    const float skq[2] = {f16_bits_to_f32(static_cast<uint16_t>(r.sk[0])) * qk,
                          f16_bits_to_f32(static_cast<uint16_t>(r.sk[1])) * qk};
    const float svo[2] = {f16_bits_to_f32(static_cast<uint16_t>(r.sv[0])),
                          f16_bits_to_f32(static_cast<uint16_t>(r.sv[1]))};
    // QK: S^T tile = K_tile . Q^T (exact fp16 codes x fp16 q)
    float s[8];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile) {
        f32x4 acc = kbias;
#pragma unroll
        for (int m = 0; m < 4; ++m) acc = mfma_f16(k_operand<KB>(r.k[tile], m), qop[m], acc);
        s[4 * tile + 0] = acc[0] * quad_bcast<0>(skq[tile]);
        s[4 * tile + 1] = acc[1] * quad_bcast<1>(skq[tile]);
        s[4 * tile + 2] = acc[2] * quad_bcast<2>(skq[tile]);
        s[4 * tile + 3] = acc[3] * quad_bcast<3>(skq[tile]);
    }
    if (nv < GROUP) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (slot_token(kb, e) >= nv) s[e] = -INFINITY;
    }
    softmax_step<8>(st, s, true);
    // P' = bf16(p * s_v): B operand of the PV MFMAs (slot e = token slot_token(kb, e))
    const u32x4 pw = {pack_bf16x2(s[0] * quad_bcast<0>(svo[0]), s[1] * quad_bcast<1>(svo[0])),
                      pack_bf16x2(s[2] * quad_bcast<2>(svo[0]), s[3] * quad_bcast<3>(svo[0])),
                      pack_bf16x2(s[4] * quad_bcast<0>(svo[1]), s[5] * quad_bcast<1>(svo[1])),
                      pack_bf16x2(s[6] * quad_bcast<2>(svo[1]), s[7] * quad_bcast<3>(svo[1]))};
    const bf16x8 pop = __builtin_bit_cast(bf16x8, pw);
    // V^T operands (A of PV MFMA nb: channel 8c + nb of the 8 token slots),
    // token pairs (2pr, 2pr + 1) merged into one dword per operand register
    if constexpr (VB == 4) {
        // bf16(128 + u) = code + 136
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) {
            lo[pr] = perm(r.v[2 * pr + 1][0], r.v[2 * pr][0], 0x05040100u);  // nibbles 0-3 of both tokens
            hi[pr] = perm(r.v[2 * pr + 1][0], r.v[2 * pr][0], 0x07060302u);  // nibbles 4-7
        }
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const uint32_t* src = nb < 4 ? lo : hi;
            const int sh = 4 * (nb & 3);
            const u32x4 w = {nib2(src[0], sh, 0x43084308u), nib2(src[1], sh, 0x43084308u),
                             nib2(src[2], sh, 0x43084308u), nib2(src[3], sh, 0x43084308u)};
            st.acc[nb] = mfma_bf16(__builtin_bit_cast(bf16x8, w), pop, st.acc[nb]);
        }
    } else if constexpr (VB == 2) {
        // bf16(128 + (crumb ^ 2)) = code + 130
        uint32_t x[4];
#pragma unroll
        for (int pr = 0; pr < 4; ++pr) x[pr] = perm(r.v[2 * pr + 1][0], r.v[2 * pr][0], 0x05040100u);
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const int sh = 2 * nb;
            const u32x4 w = {((x[0] >> sh) & 0x00030003u) ^ 0x43024302u, ((x[1] >> sh) & 0x00030003u) ^ 0x43024302u,
                             ((x[2] >> sh) & 0x00030003u) ^ 0x43024302u, ((x[3] >> sh) & 0x00030003u) ^ 0x43024302u};
            st.acc[nb] = mfma_bf16(__builtin_bit_cast(bf16x8, w), pop, st.acc[nb]);
        }
    } else {
        // code = 16 hi + lo (hi signed, lo unsigned): two products per channel
        // into one accumulator, bf16(128 + lo) and bf16(16 (128 + (hi ^ 8)))
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
            const int dw = nb >> 2;
            const uint32_t sel = 0x0c040c00u + 0x00010001u * (nb & 3);
            uint32_t x[4];
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) x[pr] = perm(r.v[2 * pr + 1][dw], r.v[2 * pr][dw], sel);
            const u32x4 wl = {(x[0] & 0x000f000fu) | 0x43004300u, (x[1] & 0x000f000fu) | 0x43004300u,
                              (x[2] & 0x000f000fu) | 0x43004300u, (x[3] & 0x000f000fu) | 0x43004300u};
            const u32x4 wh = {nib2(x[0], 4, 0x45084508u), nib2(x[1], 4, 0x45084508u),
                              nib2(x[2], 4, 0x45084508u), nib2(x[3], 4, 0x45084508u)};
            st.acc[nb] = mfma_bf16(__builtin_bit_cast(bf16x8, wl), pop, st.acc[nb]);
            st.acc[nb] = mfma_bf16(__builtin_bit_cast(bf16x8, wh), pop, st.acc[nb]);
        }
    }
    const u32x4 onesw = {0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u};
    st.ones = mfma_bf16(__builtin_bit_cast(bf16x8, onesw), pop, st.ones);
}

// ---------------------------------------------------------------------------
// bf16 segments: 16-token tiles
// ---------------------------------------------------------------------------
struct Bf16Raw {
    u32x4 k[4];            // token c, channels 32kb..32kb+31
    u32x4 v[4];            // slot e: token 4kb+e, channels 8c..8c+7
};

__device__ __forceinline__ void f16_to_bf16(Bf16Raw& r) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.k[i][j] = f16x2_to_bf16x2(r.k[i][j]);
            r.v[i][j] = f16x2_to_bf16x2(r.v[i][j]);
        }
}

// rk / rv cover this chunk's rows; tokens past the chunk read zeros
__device__ __forceinline__ void bf16_load(Bf16Raw& r, Rsrc rk, Rsrc rv, int t0, int lane) {
    const int c = lane & 15, kb = lane >> 4;
    const uint32_t so = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(t0) * (BROW * 2));
    const uint32_t ko = static_cast<uint32_t>(c) * (BROW * 2) + 64 * kb;
    const uint32_t vo = static_cast<uint32_t>(4 * kb) * (BROW * 2) + 16 * c;
#pragma unroll
    for (int i = 0; i < 4; ++i) r.k[i] = bld128(rk, ko + 16 * i, so);
#pragma unroll
    for (int e = 0; e < 4; ++e) r.v[e] = bld128<NT>(rv, vo + e * (BROW * 2), so);
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
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
        const uint32_t sel = (nb & 1) ? 0x07060302u : 0x05040100u;
        const int dw = nb >> 1;
        const u32x2 w = {perm(r.v[1][dw], r.v[0][dw], sel), perm(r.v[3][dw], r.v[2][dw], sel)};
        st.acc[nb] = mfma_bf16_k16(__builtin_bit_cast(bf16x4, w), pop, st.acc[nb]);
    }
}

// ---------------------------------------------------------------------------
// merge of a head's partials by its last workgroup
// ---------------------------------------------------------------------------
__device__ __forceinline__ u32x2 ld2_dev(Rsrc r, uint32_t off) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 16));    // sc1: device scope
}
__device__ __forceinline__ f32x4 ld4_dev(Rsrc r, uint32_t off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 16));
}

template <int CTRL>
__device__ __forceinline__ float dppf(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
// full-wavefront max / sum: DPP within each row of 16 (quad swaps, half-row
// and row mirrors), then the gfx950 row swaps across rows
__device__ __forceinline__ float wave_max64(float v) {
    v = fmaxf(v, dppf<0xb1>(v));
    v = fmaxf(v, dppf<0x4e>(v));
    v = fmaxf(v, dppf<0x141>(v));
    v = fmaxf(v, dppf<0x140>(v));
    return col_max(v);
}
__device__ __forceinline__ float wave_sum64(float v) {
    v += dppf<0xb1>(v);
    v += dppf<0x4e>(v);
    v += dppf<0x141>(v);
    v += dppf<0x140>(v);
    return col_sum(v);
}

// The merge of a head's partials, by all THREADS threads of its last
// workgroup.  The partials of query head g are rows of D floats, so the head
// has NC = 32 G float4 columns.  For G <= 8 thread t owns column t % NC of
// the partials s, s + TPC, ... (s = t / NC, TPC = THREADS / NC threads per
// column); for G > 8 it owns columns t and t + THREADS of every partial.  A
// thread's items alternate between two accumulators: item e goes to acc[e & 1]
// (its two columns for G > 8, the even and odd partials of its column
// otherwise).
//   1. every (m, l) pair of the head is loaded (two float4 per thread), then
//      the thread's first MJ items, all before any wait: the weights are
//      built while the partial loads are in flight;
//   2. (m, l) go to LDS; wavefront w takes query heads w, w + 4, ...: lane p
//      holds partial p (p + 64, ...), the wavefront max / sum give M_g and
//      den_g = sum_p exp2(m_p - M_g) l_p, and the weight exp2(m_p - M_g)
//      replaces m_p in LDS;
//   3. each thread sums weight * partial over its items in order (further
//      batches of MJ loads when it owns more), the TPC threads of a column
//      add their sums in subset order through LDS, and the column is divided
//      by den_g and stored.
// Items past a thread's share load from an offset outside the buffer range
// (zeros) and take their weight from an LDS slot holding zero, so the loops
// have no branches.  The summation order depends on nothing but (G, nwg):
// every call gives the same result.
struct MergeArgs {
    int G, nwg;
    const float* part;
    const float* ml;
    uint16_t* out;
    int64_t out_stride;
    int out16;             // store fp16 instead of bf16
};

constexpr int ML_LDS = 2 * MAX_PARTIALS;               // (m, l) per partial; the weights overwrite m
constexpr int ZERO_SLOT = ML_LDS + 16;                  // holds 0.0f (weight of an empty item)
constexpr int COMB_LDS = ML_LDS + 32;                   // one float4 per thread (column sums)
constexpr int MERGE_LDS = COMB_LDS + 4 * THREADS;
constexpr uint32_t OUT_OF_RANGE = 0xfffffff0u;          // a buffer offset past every range: reads zero

// Column q (channels 4q..4q+3) of query head g: acc / den rounded once to
// the output dtype (out.to(q.dtype) of the fp32 result), 0 when den == 0.
__device__ __forceinline__ void store_out(const MergeArgs& a, int head, int g, int q, const f32x4& acc, float den) {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = den > 0.f ? acc[i] / den : 0.f;
    const u32x2 o = a.out16 ? u32x2{static_cast<uint32_t>(f32_to_f16_bits(r[0])) |
                                        (static_cast<uint32_t>(f32_to_f16_bits(r[1])) << 16),
                                    static_cast<uint32_t>(f32_to_f16_bits(r[2])) |
                                        (static_cast<uint32_t>(f32_to_f16_bits(r[3])) << 16)}
                            : u32x2{static_cast<uint32_t>(f32_to_bf16_rne(r[0])) |
                                        (static_cast<uint32_t>(f32_to_bf16_rne(r[1])) << 16),
                                    static_cast<uint32_t>(f32_to_bf16_rne(r[2])) |
                                        (static_cast<uint32_t>(f32_to_bf16_rne(r[3])) << 16)};
    *reinterpret_cast<u32x2*>(a.out + static_cast<int64_t>(head * a.G + g) * a.out_stride + 4 * q) = o;
}

// G <= 4: one wavefront per query head g, no workgroup barrier.  Lane
// (h, q) = (lane >> 5, lane & 31) sums channels 4q..4q+3 of g over the
// partials 2j + h; lane p holds (m, l) of partial p (p + 64, ...).  The (m, l)
// loads go first, then the first MJ partial loads (MJ >= half the partials
// when the host can pick it), so the weights are built while the partials
// are in flight; they reach the lanes through a per-wavefront LDS table
// (same-address reads broadcast), whose entries past nwg hold zero, and a
// row swap adds the two halves.
template <int MJ>
__device__ __forceinline__ void merge_head_waves(const MergeArgs& a, int head, float* lds TRACE_PARAM) {
    const int G = a.G, P = a.nwg;
    const int lane = threadIdx.x & 63;
    const int g = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (g >= G) return;
    HYQ_STAMP(11);
    const int h = lane >> 5, q = lane & 31;
    const int npair = P * G;
    const Rsrc rp = make_rsrc(a.part + static_cast<int64_t>(head) * npair * D, static_cast<uint32_t>(npair) * D * 4);
    const Rsrc rm = make_rsrc(a.ml + static_cast<int64_t>(head) * npair * 2, static_cast<uint32_t>(npair) * 8);
    float* wt = lds + g * MAX_NWG;
    // (m, l) of partials lane, lane + 64, ... (past nwg: out of range, zeros);
    // the host's choice of MJ covers every partial in one batch when nwg <=
    // 48, so only the blocks of 64 that 2 MJ partials reach are loaded (a load
    // past the range still takes the CU's address path, which bounds the merge)
    constexpr int NML = MJ < 24 ? (2 * MJ + 63) / 64 : MAX_NWG / 64;
    u32x2 mlr[NML];
#pragma unroll
    for (int k = 0; k < NML; ++k) mlr[k] = ld2_dev(rm, static_cast<uint32_t>(((lane + 64 * k) * G + g) * 8));
    const uint32_t pbase = static_cast<uint32_t>(((h * G + g) * D + 4 * q) * 4);
    const uint32_t pstep = static_cast<uint32_t>(2 * G * D * 4);
    f32x4 px[MJ];
#pragma unroll
    for (int j = 0; j < MJ; ++j) px[j] = ld4_dev(rp, pbase + j * pstep);
    HYQ_STAMP(12);
    float M = M_INIT;
#pragma unroll
    for (int k = 0; k < NML; ++k)
        if (lane + 64 * k < P) M = fmaxf(M, __uint_as_float(mlr[k][0]));
    M = wave_max64(M);
    HYQ_STAMP(8);
    float den = 0.f;
#pragma unroll
    for (int k = 0; k < NML; ++k) {
        const bool ok = lane + 64 * k < P;
        const float w = ok ? fast_exp2(__uint_as_float(mlr[k][0]) - M) : 0.f;
        den += ok ? w * __uint_as_float(mlr[k][1]) : 0.f;
        wt[lane + 64 * k] = w;
    }
#pragma unroll
    for (int k = NML; k < MAX_NWG / 64; ++k) wt[lane + 64 * k] = 0.f;
    den = wave_sum64(den);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    static_assert(2 * MJ <= MAX_NWG, "a batch lies inside the weight table");
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc += wt[2 * j + h] * px[j];
    const int npr = (P + 1) / 2;                          // partial pairs
    for (int j0 = MJ; j0 < npr; j0 += MJ) {              // more than MJ pairs: one round trip per batch
#pragma unroll
        for (int j = 0; j < MJ; ++j) px[j] = ld4_dev(rp, pbase + (j0 + j) * pstep);
#pragma unroll
        for (int j = 0; j < MJ; ++j)
            if (2 * (j0 + j) + h < P) acc += wt[2 * (j0 + j) + h] * px[j];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[i]), __float_as_uint(acc[i]), false, false);
        acc[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    HYQ_STAMP(9);
    if (h == 0) store_out(a, head, g, q, acc, den);
#ifdef HYQ_PHASE_TRACE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    HYQ_STAMP(10);
#endif
}

// MJ: items loaded per thread per batch (even; the host picks the smallest
// instance that covers a thread's items, merge_batch)
template <int MJ>
__device__ __forceinline__ void merge_head_cols(const MergeArgs& a, int head, float* lds) {
    static_assert(MJ % 2 == 0, "items come in (even, odd) pairs");
    const int G = a.G, P = a.nwg;
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int npair = P * G;
    const Rsrc rp = make_rsrc(a.part + static_cast<int64_t>(head) * npair * D, static_cast<uint32_t>(npair) * D * 4);
    const Rsrc rm = make_rsrc(a.ml + static_cast<int64_t>(head) * npair * 2, static_cast<uint32_t>(npair) * 8);
    const int NC = G * (D / 4);
    const bool two = NC > THREADS;                       // G > 8
    const int TPC = two ? 1 : THREADS / NC;
    const int s = two ? 0 : t / NC;                      // partial subset (s >= TPC: idle thread)
    const int col0 = two ? t : t - s * NC;
    // item e = 2k + b: partial pb[b] + pstep * k, column col[b]
    const int pstep = two ? 1 : 2 * TPC;
    int pb[2], vb[2], wb[2];
    bool ok[2];
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        pb[b] = two ? 0 : s + TPC * b;
        const int col = two ? col0 + THREADS * b : col0;
        ok[b] = col < NC && s < TPC;
        vb[b] = (pb[b] * G * D + 4 * col) * 4;           // byte offset in the head's partials
        wb[b] = (pb[b] * G + (col >> 5)) * 2;            // LDS index of the weight
    }
    const int vstep = pstep * G * D * 4, wstep = pstep * G * 2;
    auto voff = [&](int e) -> uint32_t {
        const int b = e & 1, k = e >> 1;
        return ok[b] && pb[b] + pstep * k < P ? static_cast<uint32_t>(vb[b] + k * vstep) : OUT_OF_RANGE;
    };
    auto widx = [&](int e) -> int {
        const int b = e & 1, k = e >> 1;
        return ok[b] && pb[b] + pstep * k < P ? wb[b] + k * wstep : ZERO_SLOT;
    };
    // 1. (m, l) table, then the first batch of items
    static_assert(2 * MAX_PARTIALS <= 2 * 4 * THREADS, "two float4 (m, l) loads per thread cover the table");
    f32x4 mlv[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) mlv[k] = ld4_dev(rm, static_cast<uint32_t>((t + THREADS * k) * 16));
    f32x4 px[MJ];
#pragma unroll
    for (int j = 0; j < MJ; ++j) px[j] = ld4_dev(rp, voff(j));
    // 2. weights
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int u = t + THREADS * k;                   // float4 unit: pairs 2u, 2u + 1
        if (4 * u < 2 * npair) *reinterpret_cast<f32x4*>(lds + 4 * u) = mlv[k];
    }
    if (t == 0) lds[ZERO_SLOT] = 0.f;
    __syncthreads();
    // one 16-lane row per query head (heads 4 w .. 4 w + 3 on wavefront w,
    // then 16 more per pass), lane j of the row taking partials j, j + 16, ...:
    // every head's max and denominator at once, by 16-lane DPP reductions
    const int seg = lane >> 4, jl = lane & 15;
    for (int g0 = 4 * wave; g0 < G; g0 += 4 * WAVES) {
        const int g = g0 + seg;
        const bool gv = g < G;
        float M = M_INIT;
        if (gv)
            for (int p = jl; p < P; p += 16) M = fmaxf(M, lds[(p * G + g) * 2]);
        M = max16_dpp(M);
        float den = 0.f;
        if (gv)
            for (int p = jl; p < P; p += 16) {
                const float w = fast_exp2(lds[(p * G + g) * 2] - M);
                den += w * lds[(p * G + g) * 2 + 1];
                lds[(p * G + g) * 2] = w;
            }
        den = sum16_dpp(den);
        if (gv && jl == 0) lds[ML_LDS + g] = den;
    }
    __syncthreads();
    // 3. weighted sums in item order
    f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int j = 0; j < MJ; ++j) acc[j & 1] += lds[widx(j)] * px[j];
    const int nitems = s < TPC ? (two ? 2 * P : (P - s + TPC - 1) / TPC) : 0;
    for (int j0 = MJ; j0 < nitems; j0 += MJ) {           // a thread with more than MJ items
#pragma unroll
        for (int j = 0; j < MJ; ++j) px[j] = ld4_dev(rp, voff(j0 + j));
#pragma unroll
        for (int j = 0; j < MJ; ++j) acc[j & 1] += lds[widx(j0 + j)] * px[j];
    }
    if (!two) acc[0] += acc[1];
    f32x4* comb = reinterpret_cast<f32x4*>(lds + COMB_LDS);
    if (TPC > 1) {
        if (s >= 1 && s < TPC) comb[t] = acc[0];
        __syncthreads();
        if (s == 0)
            for (int k = 1; k < TPC; ++k) acc[0] += comb[t + k * NC];
    }
    if (s == 0) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const int col = col0 + THREADS * b;
            if ((b == 0 || two) && col < NC) {
                store_out(a, head, col >> 5, col & 31, acc[b], lds[ML_LDS + (col >> 5)]);
            }
        }
    }
}

// Largest number of items one merging thread loads (the host's choice of
// the MJ instance).
constexpr int merge_items(int G, int nwg) {
    return 32 * G > THREADS ? 2 * nwg : (nwg + THREADS / (32 * G) - 1) / (THREADS / (32 * G));
}

// ---------------------------------------------------------------------------
// the kernel
// ---------------------------------------------------------------------------
template <int KB, int VB>
__global__ __launch_bounds__(THREADS, 2) void decode_kernel(DecArgs a) {
#ifdef HYQ_PHASE_TRACE
    uint64_t ph[TRACE_PH] = {};
    HYQ_STAMP(0);
    const uint32_t launch = __hip_atomic_load(&g_trace_launch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
    const int head = blockIdx.x;
    const int wg = blockIdx.y;                       // piece of the head
    KArgs K = kernel_args(wg);
    const int u0 = static_cast<int>(K.bnd[0]), u1 = static_cast<int>(K.bnd[1]);   // its schedule units
    const uint16_t* const qp = kptr<const uint16_t>(K, 0);
    const uint8_t* const kp = kptr<const uint8_t>(K, 2);
    const uint8_t* const vp = kptr<const uint8_t>(K, 4);
    const uint16_t* const ksp = kptr<const uint16_t>(K, 6);
    const uint16_t* const vsp = kptr<const uint16_t>(K, 8);
    const uint16_t* const sk0 = kptr<const uint16_t>(K, 10);
    const uint16_t* const sk1 = kptr<const uint16_t>(K, 12);
    const uint16_t* const sk2 = kptr<const uint16_t>(K, 14);
    const uint16_t* const sv0 = kptr<const uint16_t>(K, 16);
    const uint16_t* const sv1 = kptr<const uint16_t>(K, 18);
    const uint16_t* const sv2 = kptr<const uint16_t>(K, 20);
    const int32_t* const len_q = kptr<const int32_t>(K, 22);
    const int32_t* const len_s0 = kptr<const int32_t>(K, 24);
    const int32_t q_stride = static_cast<int32_t>(kdw(K, 26));
    // head strides fit 32 bits (the host checks); products are formed in 64
    const int32_t kp_bh = static_cast<int32_t>(kdw(K, 27)), vp_bh = static_cast<int32_t>(kdw(K, 28));
    const int32_t ks_bh = static_cast<int32_t>(kdw(K, 29)), vs_bh = static_cast<int32_t>(kdw(K, 30));
    const int32_t skb0 = static_cast<int32_t>(kdw(K, 31)), skb1 = static_cast<int32_t>(kdw(K, 32));
    const int32_t skb2 = static_cast<int32_t>(kdw(K, 33)), svb0 = static_cast<int32_t>(kdw(K, 34));
    const int32_t svb1 = static_cast<int32_t>(kdw(K, 35)), svb2 = static_cast<int32_t>(kdw(K, 36));
    const int nquant = static_cast<int>(kdw(K, 37));
    const int sn0 = static_cast<int>(kdw(K, 38)), sn1 = static_cast<int>(kdw(K, 39)), sn2 = static_cast<int>(kdw(K, 40));
    const int G = static_cast<int>(kdw(K, 41));
    const int nqg = static_cast<int>(kdw(K, 42));
    const int su0 = static_cast<int>(kdw(K, 43)), su1 = static_cast<int>(kdw(K, 44));
    const float qk_scale = __uint_as_float(kdw(K, 45));
    const int io = static_cast<int>(kdw(K, 46));
    HYQ_STAMP(1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, kb = lane >> 4;

    extern __shared__ float s_acc[];               // [WAVES][G][D+1]; later the merge weights
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ int s_last;

    WaveState st;
    st.m = M_INIT;
    st.l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.ones = f32x4{0.f, 0.f, 0.f, 0.f};

    // Q row of head c (zero for padding columns c >= G): channels 32kb..32kb+31
    u32x4 qraw[4];
    {
        const Rsrc rq = make_rsrc(qp + static_cast<int64_t>(head) * G * q_stride,
                                  static_cast<uint32_t>(G * q_stride * 2));
        const uint32_t qo = static_cast<uint32_t>(c * q_stride * 2 + 64 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) qraw[i] = bld128(rq, qo + 16 * i);
    }
    // an fp16 query is rounded to bf16 (as the reference's Q loads) once the
    // first K/V loads are in flight
    uint32_t q16 = (io & HYQ_DT_Q_FP16) ? ~0u : 0u;
    asm volatile("" : "+s"(q16));

    if (u0 < nqg) {
        // ---------------- int4 part: groups wave, wave+WAVES, ... ----------------
        const int lo = u0 * GROUP;
        int nq = nquant;
        if (len_q != nullptr) nq = min(nq, max(0, sload_i32(len_q + head)));
        const int ntok = max(0, min((min(u1, nqg) - u0) * GROUP, nq - lo));   // 0: past a ragged head's end
        QCtx x;
        x.k = make_rsrc(kp + static_cast<int64_t>(head) * kp_bh + static_cast<int64_t>(lo) * prow(KB),
                        static_cast<uint32_t>(ntok) * prow(KB));
        x.v = make_rsrc(vp + static_cast<int64_t>(head) * vp_bh + static_cast<int64_t>(lo) * prow(VB),
                        static_cast<uint32_t>(ntok) * prow(VB));
        x.ks = make_rsrc(ksp + static_cast<int64_t>(head) * ks_bh + lo, static_cast<uint32_t>(ntok) * 2);
        x.vs = make_rsrc(vsp + static_cast<int64_t>(head) * vs_bh + lo, static_cast<uint32_t>(ntok) * 2);
        x.klane = static_cast<uint32_t>(krow_token(c) * prow(KB) + 4 * KB * kb);
        x.vlane = static_cast<uint32_t>(kb * prow(VB) + VB * c);
        x.slane = static_cast<uint32_t>((4 * (c & 3) + kb) * 2);
        // groups wave, wave+WAVES, ... of the piece through a three-deep
        // register ring: two groups' loads in flight while one is computed
        constexpr int STRIDE = WAVES * GROUP;
        const int ngrp = (ntok + GROUP - 1) / GROUP;
        const int nmine = ngrp > wave ? (ngrp - wave + WAVES - 1) / WAVES : 0;
        const int t0 = wave * GROUP;
        QRaw<KB, VB> b0, b1, b2;
        // in issue order (the scheduler would otherwise group the three
        // groups' loads by kind, which puts the first group's last load near
        // the end and its wait near a full drain)
        qload(b0, x, t0);
        __builtin_amdgcn_sched_barrier(0);
        qload(b1, x, t0 + STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        qload(b2, x, t0 + 2 * STRIDE);
        __builtin_amdgcn_sched_barrier(0);
        q_to_bf16(qraw, q16);
        HYQ_STAMP(2);
#ifdef HYQ_PHASE_TRACE
        asm volatile("" ::"v"(b0.sv[1]));   // the last load of the first group
        HYQ_STAMP(3);
#endif

        // Q -> fp16 in int4 slot order, pre-scaled by 2^-ex so |q| < 2^15
        float qf[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t ww[4] = {qraw[i][0], qraw[i][1], qraw[i][2], qraw[i][3]};
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
        // the K operands are u * 2^-24 (k_operand): 2^24 goes into the score scale
        const float qk = qk_scale * ldexpf(1.0f, ex + 24);
        const f32x4 kbias = k_bias<KB>(qop);
        // First round peeled (its three groups' loads were all issued before
        // the wait for Q; straight-line code keeps the compiler's waits exact),
        // then the ring: each round issues a group's loads before computing
        // the oldest, two groups in flight while one is computed.
        do {
            qcompute(st, b0, qop, kbias, ntok - t0, lane, qk);
            if (nmine <= 1) break;
            qload(b0, x, t0 + 3 * STRIDE);
            qcompute(st, b1, qop, kbias, ntok - t0 - STRIDE, lane, qk);
            if (nmine <= 2) break;
            qload(b1, x, t0 + 4 * STRIDE);
            qcompute(st, b2, qop, kbias, ntok - t0 - 2 * STRIDE, lane, qk);
            for (int i = 3; i < nmine; i += 3) {
                const int t = t0 + i * STRIDE;
                qload(b2, x, t + 2 * STRIDE);
                __builtin_amdgcn_sched_barrier(0);
                qcompute(st, b0, qop, kbias, ntok - t, lane, qk);
                if (i + 1 >= nmine) break;
                qload(b0, x, t + 3 * STRIDE);
                __builtin_amdgcn_sched_barrier(0);
                qcompute(st, b1, qop, kbias, ntok - t - STRIDE, lane, qk);
                if (i + 2 >= nmine) break;
                qload(b1, x, t + 4 * STRIDE);
                __builtin_amdgcn_sched_barrier(0);
                qcompute(st, b2, qop, kbias, ntok - t - 2 * STRIDE, lane, qk);
            }
        } while (false);
        // remove the offset of the V operands: acc -= offset * sum_t P'
        const float corr = v_offset<VB>() * st.ones[0];
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) st.acc[nb] -= corr;
    } else {
        // ------------- bf16 parts: tiles wave, wave+WAVES, ... of each segment -------------
        // (a piece never holds both int4 and bf16 tokens: make_plan cuts at
        // the segment boundaries, so the Q copies of one part are dead
        // during the other's loop)
        // fp16 segments (an fp16 model's cache) are rounded to bf16 after
        // their loads, as the reference's .to(tl.bfloat16) of each tile
        const bool seg16 = io & HYQ_DT_SEG_FP16;
        // segment bounds in units: [nqg, b1), [b1, b2), [b2, end of head)
        const int b1 = nqg + su0, b2 = b1 + su1;
        for (int seg = 0; seg < 3; ++seg) {
            const int sb = seg == 0 ? nqg : seg == 1 ? b1 : b2;
            const int ua = max(u0, sb), ub = min(u1, seg == 0 ? b1 : seg == 1 ? b2 : u1);
            if (ua >= ub) continue;
            const int lo = (ua - sb) * BUNIT;
            int seg_len = seg == 0 ? sn0 : seg == 1 ? sn1 : sn2;
            if (seg == 0 && len_s0 != nullptr) seg_len = min(seg_len, max(0, sload_i32(len_s0 + head)));
            const int n = max(0, min((ub - ua) * BUNIT, seg_len - lo));     // 0: past a ragged head's end
            const uint16_t* const skp = seg == 0 ? sk0 : seg == 1 ? sk1 : sk2;
            const uint16_t* const svp = seg == 0 ? sv0 : seg == 1 ? sv1 : sv2;
            const int32_t skb = seg == 0 ? skb0 : seg == 1 ? skb1 : skb2;
            const int32_t svb = seg == 0 ? svb0 : seg == 1 ? svb1 : svb2;
            const uint16_t* kbase = skp + static_cast<int64_t>(head) * skb + static_cast<int64_t>(lo) * BROW;
            const uint16_t* vbase = svp + static_cast<int64_t>(head) * svb + static_cast<int64_t>(lo) * BROW;
            const uint32_t nbytes = static_cast<uint32_t>(n) * (BROW * 2);
            const Rsrc rk = make_rsrc(kbase, nbytes), rv = make_rsrc(vbase, nbytes);
            // tiles wave, wave+WAVES, ... through a two-deep register ring
            constexpr int TSTRIDE = WAVES * TILE;
            const int ntile = (n + TILE - 1) / TILE;
            const int nmine = ntile > wave ? (ntile - wave + WAVES - 1) / WAVES : 0;
            const int t0 = wave * TILE;
            Bf16Raw r0, r1;
            bf16_load(r0, rk, rv, t0, lane);
            bf16_load(r1, rk, rv, t0 + TSTRIDE, lane);
            u32x4 qs[4] = {qraw[0], qraw[1], qraw[2], qraw[3]};
            q_to_bf16(qs, q16);
#ifdef HYQ_PHASE_TRACE
            if (ph[2] == 0) {
                HYQ_STAMP(2);
                asm volatile("" ::"v"(r0.v[3][3]));   // the last load of the first tile
                HYQ_STAMP(3);
            }
#endif
            const bf16x8 qb[4] = {__builtin_bit_cast(bf16x8, qs[0]), __builtin_bit_cast(bf16x8, qs[1]),
                                  __builtin_bit_cast(bf16x8, qs[2]), __builtin_bit_cast(bf16x8, qs[3])};
            // the ring: the tile two ahead is loaded into the slot just computed
            for (int i = 0; i < nmine; i += 2) {
                const int t = t0 + i * TSTRIDE;
                if (seg16) f16_to_bf16(r0);
                bf16_compute(st, r0, qb, n - t, lane, qk_scale);
                if (i + 1 >= nmine) break;
                bf16_load(r0, rk, rv, t + 2 * TSTRIDE, lane);
                if (seg16) f16_to_bf16(r1);
                bf16_compute(st, r1, qb, n - t - TSTRIDE, lane, qk_scale);
                if (i + 2 >= nmine) break;
                bf16_load(r1, rk, rv, t + 3 * TSTRIDE, lane);
            }
        }
    }

    // ---- wave -> LDS ----------------------------------------------------------
    HYQ_STAMP(4);
    epilogue_args(K);
    const int mj = static_cast<int>(K.e1[2]);
    const MergeArgs ma{G, static_cast<int>(K.e1[1]), eptr<const float>(K, 2), eptr<const float>(K, 4),
                       eptr<uint16_t>(K, 0), static_cast<int64_t>(static_cast<int32_t>(K.e1[0])),
                       io & HYQ_DT_OUT_FP16};
    uint32_t* const cnt = eptr<uint32_t>(K, 6);
    // The rings' last loads (past the piece's end: zeros, no memory access)
    // are drained here, with a wait the compiler sees, so that it has no
    // stale loads to wait for among the stores below.
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0)
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
    HYQ_STAMP(5);

    // ---- workgroup merge -> partial acc[G][D] and (m, l)[G] ----------------------
    const int64_t slot = static_cast<int64_t>(head) * ma.nwg + wg;
    {
        const Rsrc rpart = make_rsrc(ma.part + slot * G * D, static_cast<uint32_t>(G * D * 4));
        for (int o = threadIdx.x; o < G * (D / 4); o += THREADS) {
            const int g = o / (D / 4), ch = 4 * (o % (D / 4));
            float M = s_m[0][g];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
            f32x4 accv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float wt = fast_exp2(s_m[w][g] - M);
                const float* row = s_acc + (w * G + g) * (D + 1) + ch;
                accv += wt * f32x4{row[0], row[1], row[2], row[3]};
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, accv), rpart, o * 16, 0, 16);   // sc1
        }
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
        float lv = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) lv += fast_exp2(s_m[w][g] - M) * s_l[w][g];
        float* const mlw = const_cast<float*>(ma.ml);
        __hip_atomic_store(mlw + (slot * G + g) * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(mlw + (slot * G + g) * 2 + 1, lv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every store of this workgroup acknowledged before its arrival is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    HYQ_STAMP(6);
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(cnt + head * CNT_PAD, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == static_cast<uint32_t>(ma.nwg - 1));
    }
    __syncthreads();
    HYQ_STAMP(7);
    if (s_last) {
        if (threadIdx.x == 0) __hip_atomic_store(cnt + head * CNT_PAD, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        switch (mj) {      // G <= 4: merge_head_waves, pairs per lane; G > 4: merge_head_cols, items per thread
            case 4: merge_head_waves<4>(ma, head, s_acc TRACE_ARG); break;
            case 8: merge_head_waves<8>(ma, head, s_acc TRACE_ARG); break;
            case 12: merge_head_waves<12>(ma, head, s_acc TRACE_ARG); break;
            case 16: merge_head_waves<16>(ma, head, s_acc TRACE_ARG); break;
            case 20: merge_head_waves<20>(ma, head, s_acc TRACE_ARG); break;
            case 24: merge_head_waves<24>(ma, head, s_acc TRACE_ARG); break;
            case 108: merge_head_cols<8>(ma, head, s_acc); break;
            case 116: merge_head_cols<16>(ma, head, s_acc); break;
            default: merge_head_cols<24>(ma, head, s_acc); break;
        }
    }
#ifdef HYQ_PHASE_TRACE
    const uint32_t lwg = blockIdx.y * gridDim.x + blockIdx.x;
    if (lane == 0 && lwg < TRACE_MAX_WG) {
        ph[13] = launch;
        uint64_t* dst = g_trace[launch % TRACE_SLOTS][lwg * 4 + wave];
        for (int i = 0; i < TRACE_PH; ++i) dst[i] = ph[i];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t total = gridDim.x * gridDim.y;
        if (__hip_atomic_fetch_add(&g_trace_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == total - 1) {
            __hip_atomic_store(&g_trace_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_add(&g_trace_launch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
#endif
}

// ---------------------------------------------------------------------------
// legacy-format decode
// ---------------------------------------------------------------------------
// The legacy decode format of src/ops/d_stage_cache.py (fused_decode_
// attention_k4v4 :504-591, splitk_decode_attention_k4v4 :825-951 and its MMA
// variant :1247-1366 with K_BITS / V_BITS of 4 or 2, :977-1092): a prefix of
// offset-encoded codes (int4: channel 2j in the high nibble of byte j, value
// u - 8; int2: channel 4j + i in bits 7-2i..6-2i of byte j, value u - 1.5)
// with one fp16 scale per (group of tokens, channel), then the top-k,
// staging and window bf16 rows.  The prefix tiles are dequantised in
// registers to the bf16 values of legacy_dequant_kernel (legacy_twice_to_bf16)
// scaled by an exact power of two, and computed by the bf16 tile path
// (bf16_compute): the result of dequantising the prefix and decoding bf16
// rows, without the bf16 copy in HBM.  One workgroup per piece
// (LEG_PIECE prefix tokens or BF_PIECE rows of one segment, the same number
// of bytes; halved together, down to LEG_PIECE_MIN tokens, while the grid
// would leave a CU without a workgroup; doubled together while the prefix
// still gives every resident workgroup slot a piece, up to LEG_PIECE_MAX
// tokens, and for long caches until the pieces fit the merge tables), merged
// by the head's last arriving workgroup with decode_kernel's protocol and
// merge.
constexpr int LEG_PIECE = 512;
constexpr int LEG_PIECE_MIN = 128;
constexpr int LEG_PIECE_MAX = 4096;
constexpr int BF_PIECE = 128;

struct LegArgs {
    const uint16_t* q;
    int64_t q_stride;
    const uint8_t* kc;             // prefix codes [bh][n][16 * bits] (byte strides)
    const uint8_t* vc;
    int64_t kc_bh, kc_n, vc_bh, vc_n;
    const uint16_t* ks;            // prefix scales [bh][groups][D] (element strides)
    const uint16_t* vs;
    int64_t ks_bh, ks_g, vs_bh, vs_g;
    int64_t ks_rows, vs_rows;      // scale rows per head (the descriptors' ranges)
    int n_leg, group;
    const uint16_t* sk[3];         // top-k, staging, window rows [bh][n][D]
    const uint16_t* sv[3];
    int64_t sk_bh[3], sv_bh[3];
    int sn[3];
    int G;
    float qk_scale;                // sm_scale * log2(e)
    float* part;
    float* ml;
    uint32_t* cnt;
    uint16_t* out;
    int64_t out_stride;
    int nwg, mj;
    int pfirst[5];                 // pieces of segment s (0: the prefix): [pfirst[s], pfirst[s + 1])
    int plen[4];                   // tokens per piece of segment s
};

// the raw loads of one 16-token prefix tile, for the layout of Bf16Raw (the
// group is a multiple of 16 and tiles start at multiples of 16 tokens, so a
// tile's tokens share one scale row)
template <int KB, int VB>
struct LegRaw {
    uint32_t kc[KB];               // token c: codes of channels 32kb .. 32kb + 31 (4 KB bytes)
    u32x4 ksc[4];                  // their fp16 scales, 8 channels per vector
    uint32_t vc[4];                // slot e (token 4kb + e): codes of channels 8c .. 8c + 7 (VB bytes, zero-extended)
    u32x4 vsc;                     // their fp16 scales
};

// Loads of the tile at token t of a piece starting at prefix token lo: the
// lane's offsets (kco: token c, vco: token 4kb) are fixed, the tile's
// position goes in the scalar offsets.  The code descriptors cover the piece
// and the scale descriptors the head's scale rows (the range check covers
// the scalar offset too): tokens past either read zeros.
template <int KB, int VB>
__device__ __forceinline__ void legacy_fetch(LegRaw<KB, VB>& r, const LegArgs& a, Rsrc rkc, Rsrc rvc, Rsrc rks,
                                             Rsrc rvs, uint32_t kco, uint32_t vco, int lo, int t, int lane) {
    const int c = lane & 15, kb = lane >> 4;
    // wave-uniform scalar offsets (left to the compiler, some became vector
    // values and their loads were wrapped in waterfall loops)
    const int tu = __builtin_amdgcn_readfirstlane(t);
    const int g = (lo + tu) / a.group;                     // the tile's scale row
    const uint32_t skc = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tu * a.kc_n));
    const uint32_t sks = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(g * a.ks_g * 2));
    const uint32_t svc = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(tu * a.vc_n));
    const uint32_t svs = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(g * a.vs_g * 2));
    // codes are read once: non-temporal, as the fused decode's packed rows
    // (with inputs rotated over 1 GiB: 128 KV heads at 62000 tokens 300-307
    // -> 290 us, 32 heads 50.5-51.0 -> 49.0-49.5 us); the scale rows, read by
    // every tile of their group, keep the default policy
    if constexpr (KB == 4) {
        const u32x4 w = bld128<NT>(rkc, kco, skc);
        r.kc[0] = w[0]; r.kc[1] = w[1]; r.kc[2] = w[2]; r.kc[3] = w[3];
    } else {
        const u32x2 w = bld64<NT>(rkc, kco, skc);
        r.kc[0] = w[0]; r.kc[1] = w[1];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) r.ksc[i] = bld128(rks, static_cast<uint32_t>(64 * kb + 16 * i), sks);
#pragma unroll
    for (int e = 0; e < 4; ++e)
        r.vc[e] = VB == 4 ? bld32<NT>(rvc, vco + static_cast<uint32_t>(e * a.vc_n), svc)
                          : bld16<NT>(rvc, vco + static_cast<uint32_t>(e * a.vc_n), svc);
    r.vsc = bld128(rvs, static_cast<uint32_t>(16 * c), svs);
}

// Codes -> bf16 operands at a power-of-two fraction of the dequantised
// values.  v_cvt_off_f32_i4 turns the low 4 bits of its operand (byte B of
// the word, picked by SDWA) into that signed 4-bit field divided by 16, so
// one instruction replaces a bit-field extract and a conversion.
//   int4: the code word w has every nibble XOR 8, so a nibble read as a
//     signed field is u - 8; channel 2j sits in the high nibble of byte j
//     (read from w >> 4), 2j + 1 in the low one (read from w): (u - 8) / 16.
//   int2: crumb m of every byte (bits 7-2m..6-2m, channel 4j + m) goes to
//     the low bits of its byte, and 2u + 13 makes a nibble whose signed value
//     is 2u - 3: (u - 1.5) / 8.
// The value times an fp16 scale is exact in fp32 and is rounded once by the
// packed bf16 conversion, which gives exactly 1/16 (int4) or 1/8 (int2) of
// legacy_twice_to_bf16's bits (every such product is a normal float or zero,
// so the power-of-two factor commutes with the rounding; the zeros keep their
// signs).  The kernel multiplies the score scale by 16 (8) for the prefix and
// its P.V accumulators by 16 (8) after it, both exact.
template <int B>
__device__ __forceinline__ float off4_byte(uint32_t w) {
    float r;
    if constexpr (B == 0)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(w));
    else if constexpr (B == 1)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(w));
    else if constexpr (B == 2)
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(w));
    else
        asm("v_cvt_off_f32_i4_sdwa %0, %1 dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(w));
    return r;
}
// x times the fp16 in the low (HI = false) or high half of sw, converted
// inside v_fma_mix_f32; the addend is neg(0) = -0 so that x * s + a is the
// product itself, zeros with their signs
template <bool HI>
__device__ __forceinline__ float mul_f16_half(float x, uint32_t sw) {
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(sw));
    else
        asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[0,0,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(x), "v"(sw));
    return r;
}
// K: byte B's two channels, each with its own fp16 scale (the halves of sw)
template <int B>
__device__ __forceinline__ uint32_t leg4_pair_k(uint32_t w, uint32_t wsh, uint32_t sw) {
    return pack_bf16x2(mul_f16_half<false>(off4_byte<B>(wsh), sw), mul_f16_half<true>(off4_byte<B>(w), sw));
}
// V: the lane's eight channel scales are shared by its four code words, so
// they are converted once and multiplied in fp32
template <int B>
__device__ __forceinline__ uint32_t leg4_pair_v(uint32_t w, uint32_t wsh, const float (&s)[8]) {
    return pack_bf16x2(off4_byte<B>(wsh) * s[2 * B], off4_byte<B>(w) * s[2 * B + 1]);
}

// int2: crumb m of every byte of w as a nibble of value 2u - 3 in its byte
template <int M>
__device__ __forceinline__ uint32_t crumb_nibbles(uint32_t w) {
    return (((w >> (6 - 2 * M)) & 0x03030303u) << 1) + 0x0d0d0d0du;
}
// K, int2: the pair (channels 4j + M, 4j + M + 1) of byte J, with the two
// halves of the scale word sw
template <int J, int M>
__device__ __forceinline__ uint32_t leg2_pair_k(const uint32_t (&n)[4], uint32_t sw) {
    return pack_bf16x2(mul_f16_half<false>(off4_byte<J>(n[M]), sw), mul_f16_half<true>(off4_byte<J>(n[M + 1]), sw));
}
template <int J, int M>
__device__ __forceinline__ uint32_t leg2_pair_v(const uint32_t (&n)[4], const float (&s)[8]) {
    return pack_bf16x2(off4_byte<J>(n[M]) * s[4 * J + M], off4_byte<J>(n[M + 1]) * s[4 * J + M + 1]);
}

template <int KB, int VB>
__device__ __forceinline__ void legacy_dequant(Bf16Raw& b, const LegRaw<KB, VB>& r) {
    if constexpr (KB == 4) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = r.kc[i] ^ 0x88888888u, wsh = w >> 4;
            b.k[i] = u32x4{leg4_pair_k<0>(w, wsh, r.ksc[i][0]), leg4_pair_k<1>(w, wsh, r.ksc[i][1]),
                           leg4_pair_k<2>(w, wsh, r.ksc[i][2]), leg4_pair_k<3>(w, wsh, r.ksc[i][3])};
        }
    } else {
        // word h holds channels 32kb + 16h .. + 15: operand 2h + 0 takes its
        // bytes 0 and 1, operand 2h + 1 its bytes 2 and 3
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t n[4] = {crumb_nibbles<0>(r.kc[h]), crumb_nibbles<1>(r.kc[h]), crumb_nibbles<2>(r.kc[h]),
                                   crumb_nibbles<3>(r.kc[h])};
            const u32x4& s0 = r.ksc[2 * h];
            const u32x4& s1 = r.ksc[2 * h + 1];
            b.k[2 * h] = u32x4{leg2_pair_k<0, 0>(n, s0[0]), leg2_pair_k<0, 2>(n, s0[1]), leg2_pair_k<1, 0>(n, s0[2]),
                               leg2_pair_k<1, 2>(n, s0[3])};
            b.k[2 * h + 1] = u32x4{leg2_pair_k<2, 0>(n, s1[0]), leg2_pair_k<2, 2>(n, s1[1]),
                                   leg2_pair_k<3, 0>(n, s1[2]), leg2_pair_k<3, 2>(n, s1[3])};
        }
    }
    float vs[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        vs[2 * j] = f16_bits_to_f32(static_cast<uint16_t>(r.vsc[j]));
        vs[2 * j + 1] = f16_bits_to_f32(static_cast<uint16_t>(r.vsc[j] >> 16));
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (VB == 4) {
            const uint32_t w = r.vc[e] ^ 0x88888888u, wsh = w >> 4;
            b.v[e] = u32x4{leg4_pair_v<0>(w, wsh, vs), leg4_pair_v<1>(w, wsh, vs), leg4_pair_v<2>(w, wsh, vs),
                           leg4_pair_v<3>(w, wsh, vs)};
        } else {
            const uint32_t n[4] = {crumb_nibbles<0>(r.vc[e]), crumb_nibbles<1>(r.vc[e]), crumb_nibbles<2>(r.vc[e]),
                                   crumb_nibbles<3>(r.vc[e])};
            b.v[e] = u32x4{leg2_pair_v<0, 0>(n, vs), leg2_pair_v<0, 2>(n, vs), leg2_pair_v<1, 0>(n, vs),
                           leg2_pair_v<1, 2>(n, vs)};
        }
    }
}

// Three workgroups per CU (168 VGPRs): the tile loop keeps its registers and
// the merge at the end spills 236 bytes per lane.  Against two per CU (213
// VGPRs, no spill), same box, 128 KV heads: 31000 tokens K4V4 171.5 ->
// 167-169 us, K2V2 184 -> 167-169 us; 62000 tokens 322 -> 294-297 us (waves
// that wait on memory leave the VALU to the others: 59-67% VALU-busy at two).
template <int KB, int VB>
__global__ __launch_bounds__(THREADS, 3) void legacy_decode_kernel(LegArgs a) {
#ifdef HYQ_PHASE_TRACE
    uint64_t ph[TRACE_PH] = {};    // (the merge stamps; not stored by this kernel)
#endif
    const int head = blockIdx.x;
    const int wg = blockIdx.y;
    const int G = a.G;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, kb = lane >> 4;

    extern __shared__ float s_acc[];               // [WAVES][G][D+1]; later the merge weights
    __shared__ float s_m[WAVES][16];
    __shared__ float s_l[WAVES][16];
    __shared__ int s_last;

    WaveState st;
    st.m = M_INIT;
    st.l = 0.f;
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) st.acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    st.ones = f32x4{0.f, 0.f, 0.f, 0.f};

    // Q row of head c (zero for c >= G): channels 32kb..32kb+31
    u32x4 qs[4];
    {
        const Rsrc rq = make_rsrc(a.q + static_cast<int64_t>(head) * G * a.q_stride,
                                  static_cast<uint32_t>(G * a.q_stride * 2));
        const uint32_t qo = static_cast<uint32_t>(c * a.q_stride * 2 + 64 * kb);
#pragma unroll
        for (int i = 0; i < 4; ++i) qs[i] = bld128(rq, qo + 16 * i);
    }
    const bf16x8 qb[4] = {__builtin_bit_cast(bf16x8, qs[0]), __builtin_bit_cast(bf16x8, qs[1]),
                          __builtin_bit_cast(bf16x8, qs[2]), __builtin_bit_cast(bf16x8, qs[3])};

    // this piece: segment sg (0: the prefix), tokens [lo, lo + n) of it
    int sg = 0;
    while (sg < 3 && wg >= a.pfirst[sg + 1]) ++sg;
    const int lo = (wg - a.pfirst[sg]) * a.plen[sg];
    const int seg_n = sg == 0 ? a.n_leg : a.sn[sg - 1];
    const int n = max(0, min(a.plen[sg], seg_n - lo));
    constexpr int TSTRIDE = WAVES * TILE;
    const int ntile = (n + TILE - 1) / TILE;
    const int nmine = ntile > wave ? (ntile - wave + WAVES - 1) / WAVES : 0;
    const int t0 = wave * TILE;
    if (sg == 0) {
        const Rsrc rkc = make_rsrc(a.kc + head * a.kc_bh + lo * a.kc_n, static_cast<uint32_t>(n * a.kc_n));
        const Rsrc rvc = make_rsrc(a.vc + head * a.vc_bh + lo * a.vc_n, static_cast<uint32_t>(n * a.vc_n));
        const Rsrc rks = make_rsrc(a.ks + head * a.ks_bh, static_cast<uint32_t>(a.ks_rows * a.ks_g * 2));
        const Rsrc rvs = make_rsrc(a.vs + head * a.vs_bh, static_cast<uint32_t>(a.vs_rows * a.vs_g * 2));
        // tiles wave, wave+WAVES, ... through a two-deep register ring
        const uint32_t kco = static_cast<uint32_t>(c * a.kc_n + 4 * KB * kb);
        const uint32_t vco = static_cast<uint32_t>(4 * kb * a.vc_n + VB * c);
        LegRaw<KB, VB> r0, r1;
        Bf16Raw b;
        constexpr float KF = KB == 4 ? 16.f : 8.f, VF = VB == 4 ? 16.f : 8.f;   // the operands are 1/KF, 1/VF of the values
        const float qk16 = KF * a.qk_scale;
        legacy_fetch(r0, a, rkc, rvc, rks, rvs, kco, vco, lo, t0, lane);
        legacy_fetch(r1, a, rkc, rvc, rks, rvs, kco, vco, lo, t0 + TSTRIDE, lane);
        for (int i = 0; i < nmine; i += 2) {
            const int t = t0 + i * TSTRIDE;
            legacy_dequant(b, r0);
            bf16_compute(st, b, qb, n - t, lane, qk16);
            if (i + 1 >= nmine) break;
            legacy_fetch(r0, a, rkc, rvc, rks, rvs, kco, vco, lo, t + 2 * TSTRIDE, lane);
            legacy_dequant(b, r1);
            bf16_compute(st, b, qb, n - t - TSTRIDE, lane, qk16);
            if (i + 2 >= nmine) break;
            legacy_fetch(r1, a, rkc, rvc, rks, rvs, kco, vco, lo, t + 3 * TSTRIDE, lane);
        }
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) st.acc[nb] *= VF;
    } else {
        const int s3 = sg - 1;
        const uint16_t* kbase = a.sk[s3] + head * a.sk_bh[s3] + static_cast<int64_t>(lo) * BROW;
        const uint16_t* vbase = a.sv[s3] + head * a.sv_bh[s3] + static_cast<int64_t>(lo) * BROW;
        const uint32_t nbytes = static_cast<uint32_t>(n) * (BROW * 2);
        const Rsrc rk = make_rsrc(kbase, nbytes), rv = make_rsrc(vbase, nbytes);
        Bf16Raw r0, r1;
        bf16_load(r0, rk, rv, t0, lane);
        bf16_load(r1, rk, rv, t0 + TSTRIDE, lane);
        for (int i = 0; i < nmine; i += 2) {
            const int t = t0 + i * TSTRIDE;
            bf16_compute(st, r0, qb, n - t, lane, a.qk_scale);
            if (i + 1 >= nmine) break;
            bf16_load(r0, rk, rv, t + 2 * TSTRIDE, lane);
            bf16_compute(st, r1, qb, n - t - TSTRIDE, lane, a.qk_scale);
            if (i + 2 >= nmine) break;
            bf16_load(r1, rk, rv, t + 3 * TSTRIDE, lane);
        }
    }

    // ---- wave -> LDS -> this piece's partial, then decode_kernel's arrival protocol ----
    const MergeArgs ma{G, a.nwg, a.part, a.ml, a.out, a.out_stride, 0};
    __builtin_amdgcn_s_waitcnt(0x0f70);   // vmcnt(0): the rings' last (empty) loads
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
    const int64_t slot = static_cast<int64_t>(head) * ma.nwg + wg;
    {
        const Rsrc rpart = make_rsrc(ma.part + slot * G * D, static_cast<uint32_t>(G * D * 4));
        for (int o = threadIdx.x; o < G * (D / 4); o += THREADS) {
            const int g = o / (D / 4), ch = 4 * (o % (D / 4));
            float M = s_m[0][g];
#pragma unroll
            for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
            f32x4 accv = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const float wt = fast_exp2(s_m[w][g] - M);
                const float* row = s_acc + (w * G + g) * (D + 1) + ch;
                accv += wt * f32x4{row[0], row[1], row[2], row[3]};
            }
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, accv), rpart, o * 16, 0, 16);   // sc1
        }
    }
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        float M = s_m[0][g];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) M = fmaxf(M, s_m[w][g]);
        float lv = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) lv += fast_exp2(s_m[w][g] - M) * s_l[w][g];
        __hip_atomic_store(a.ml + (slot * G + g) * 2, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.ml + (slot * G + g) * 2 + 1, lv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // every store of this workgroup acknowledged before its arrival is counted
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t old = __hip_atomic_fetch_add(a.cnt + head * CNT_PAD, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (old == static_cast<uint32_t>(ma.nwg - 1));
    }
    __syncthreads();
    if (s_last) {
        if (threadIdx.x == 0) __hip_atomic_store(a.cnt + head * CNT_PAD, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        switch (a.mj) {
            case 4: merge_head_waves<4>(ma, head, s_acc TRACE_ARG); break;
            case 8: merge_head_waves<8>(ma, head, s_acc TRACE_ARG); break;
            case 12: merge_head_waves<12>(ma, head, s_acc TRACE_ARG); break;
            case 16: merge_head_waves<16>(ma, head, s_acc TRACE_ARG); break;
            case 20: merge_head_waves<20>(ma, head, s_acc TRACE_ARG); break;
            case 24: merge_head_waves<24>(ma, head, s_acc TRACE_ARG); break;
            case 108: merge_head_cols<8>(ma, head, s_acc); break;
            case 116: merge_head_cols<16>(ma, head, s_acc); break;
            default: merge_head_cols<24>(ma, head, s_acc); break;
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

struct Slots {
    int slots, cus;        // workgroups resident at once, compute units (0: unknown)
};

struct Plan {
    int nwg;               // pieces per head
    int nqg, segu[3];      // schedule units: int4 groups, bf16 units per segment
    int bnd[MAX_NWG + 1];  // piece p covers units [bnd[p], bnd[p+1])
};

size_t round256(size_t x) { return (x + 255) / 256 * 256; }

// Cut a head into pieces, each inside one segment (a piece spanning segments
// would walk their rings one after the other; decode_kernel relies on no
// piece holding both int4 and bf16 units), the int4 pieces first so that the
// short segment pieces fill the end of the grid.
//   requested > 0: pieces of about that many int4 tokens' bytes.
//   few KV heads (bh_kv < 32, a step of a few microseconds, bound by the
//     per-piece round trips), G <= 4: every segment cut into pieces of
//     equal bytes, total / (0.8 CUs) (measured best at B=1 from 2K to 32K
//     prefixes), at most 48 per head.
//   few KV heads, G > 4 (each partial is G rows, so the merge weighs more):
//     int4 pieces of the smallest power-of-two token count >= 128 that gives
//     at most 32 pieces (2048 at most), bf16 pieces of 128 tokens (without
//     a prefix, like the prefix: a power of two from 128 to 512).
//   many KV heads: pieces of about total / (1.25 * slots) bytes, `slots`
//     being the workgroups the device holds at once: the first round fills
//     every slot and the remaining quarter, with the short segment pieces,
//     evens out the workgroups that ran slow.  Pieces stay >= 96 KiB: below
//     that the per-piece round trips cost more than the balance gains.  From
//     a 384 KiB target the bf16 segments (the top-k rows above all, which
//     run in the last round) are cut at half the target: B=16, 32K went
//     from 100.9 to 98.2 us and B=8, 32K from 54.4 to 52.7 us (same box),
//     while with smaller targets the extra partials cost more than the
//     shorter round gains (GLM-4-9B shape, 248 KiB: 37.4 -> 40.1 us).
// Each segment gets its bytes / target pieces (rounded, at least one); the
// target grows until the pieces fit the merge tables.
Plan make_plan(int64_t n_quant, const int64_t seg_n[3], int bh_kv, int G, int requested, int kb, int vb,
               Slots sl_) {
    const int slots = sl_.slots;
    Plan p{};
    p.nqg = static_cast<int>((n_quant + GROUP - 1) / GROUP);
    for (int s = 0; s < 3; ++s) p.segu[s] = static_cast<int>((seg_n[s] + BUNIT - 1) / BUNIT);
    const int64_t cq = static_cast<int64_t>(GROUP) * (16 * kb + 16 * vb + 4);   // bytes of an int4 group
    const int64_t cb = static_cast<int64_t>(BUNIT) * 4 * D;                     // bytes of a bf16 unit (K and V)
    const int64_t su[4] = {p.nqg, p.segu[0], p.segu[1], p.segu[2]};             // units per segment
    const int64_t sc[4] = {cq, cb, cb, cb};
    int64_t head_bytes = 0;
    int nonempty = 0;
    for (int s = 0; s < 4; ++s) {
        head_bytes += su[s] * sc[s];
        nonempty += su[s] > 0;
    }
    p.nwg = 0;
    if (nonempty == 0) return p;
    const int kmax = std::max(nonempty, std::min(MAX_NWG, MAX_PARTIALS / G));
    int ks[4];
    int bdiv = 1;                      // the bf16 segments' pieces: target / bdiv bytes
    auto counts_for = [&](int64_t target) {
        int total = 0;
        for (int s = 0; s < 4; ++s) {
            const int64_t tg = s == 0 ? target : std::max<int64_t>(1, target / bdiv);
            ks[s] = su[s] > 0 ? static_cast<int>(std::min<int64_t>(
                                    su[s], std::max<int64_t>(1, (su[s] * sc[s] + tg / 2) / tg)))
                              : 0;
            total += ks[s];
        }
        return total;
    };
    int total;
    int64_t target;
    if (requested > 0) {
        target = std::max<int64_t>(1, (requested + GROUP - 1) / GROUP) * cq;
        total = counts_for(target);
    } else if (bh_kv < 32 && G <= WAVES) {
        // few heads, G <= 4: pieces of equal bytes, about 0.8 per CU (a
        // workgroup per CU streams faster than two sharing one, and the
        // merge grows with the piece count), at least 8 KiB and at most 48
        // per head
        const int64_t cus = sl_.cus > 0 ? sl_.cus : 256;
        target = std::max<int64_t>(8 << 10, head_bytes * bh_kv * 5 / (4 * cus));
        target = std::max<int64_t>(target, (head_bytes + 47) / 48);
        total = counts_for(target);
    } else if (bh_kv < 32) {
        int64_t split = 4 * GROUP, bsplit = 128;
        while (split < 2048 && split * 32 < n_quant) split *= 2;
        if (n_quant == 0) {       // bf16 alone (the full-precision comparator): split like a prefix
            const int64_t nb = seg_n[0] + seg_n[1] + seg_n[2];
            while (bsplit < 512 && bsplit * 32 < nb) bsplit *= 2;
        }
        const int64_t gsplit = split / GROUP;
        bsplit /= BUNIT;
        ks[0] = static_cast<int>((su[0] + gsplit - 1) / gsplit);
        total = ks[0];
        for (int s = 1; s < 4; ++s) {
            ks[s] = static_cast<int>((su[s] + bsplit - 1) / bsplit);
            total += ks[s];
        }
        target = (head_bytes + total - 1) / total;
    } else {
        const int64_t sl = slots > 0 ? slots : 512;
        target = std::max<int64_t>(96 << 10, head_bytes * bh_kv * 4 / (5 * sl));
        bdiv = target >= (384 << 10) ? 2 : 1;
        total = counts_for(target);
    }
    while (total > kmax) {
        target += target / 8 + 1;
        total = counts_for(target);
    }
    int64_t base = 0;
    for (int s = 0; s < 4; ++s) {
        for (int i = 0; i < ks[s]; ++i) p.bnd[p.nwg++] = static_cast<int>(base + su[s] * i / ks[s]);
        base += su[s];
    }
    p.bnd[p.nwg] = static_cast<int>(base);
    return p;
}

size_t lds_bytes(int G) {
    return std::max(static_cast<size_t>(WAVES) * G * (D + 1), static_cast<size_t>(MERGE_LDS)) * sizeof(float);
}

// The merge instance: for G <= 4 merge_head_waves with the smallest batch
// covering a lane's partial pairs (else batches of 24); for G > 4
// merge_head_cols (100 + batch) with the smallest batch covering a thread's
// items (else batches of 24).
int merge_batch(int G, int nwg) {
    if (G <= WAVES) {
        const int pairs = (nwg + 1) / 2;
        for (int mj : {4, 8, 12, 16, 20})
            if (pairs <= mj) return mj;
        return 24;
    }
    const int items = merge_items(G, nwg);
    for (int mj : {8, 16})
        if (items <= mj) return 100 + mj;
    return 124;
}

// Workgroups of one decode_kernel instance the device holds at once (and
// the device's CU count), cached per device and GQA width (the LDS size).
template <int KB, int VB>
Slots resident_slots_of(int G) {
    static std::atomic<int> cache[64][17][2];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || G < 1 || G > 16) return {0, 0};
    const int known = cache[dev][G][0].load(std::memory_order_relaxed);
    if (known > 0) return {known, cache[dev][G][1].load(std::memory_order_relaxed)};
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, reinterpret_cast<const void*>(&decode_kernel<KB, VB>),
                                                     THREADS, lds_bytes(G)) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return {0, 0};
    cache[dev][G][1].store(cus, std::memory_order_relaxed);
    cache[dev][G][0].store(per_cu * cus, std::memory_order_relaxed);
    return {per_cu * cus, cus};
}

Slots resident_slots(int kb, int vb, int G) {
    switch (10 * kb + vb) {
        case 44: return resident_slots_of<4, 4>(G);
        case 42: return resident_slots_of<4, 2>(G);
        case 48: return resident_slots_of<4, 8>(G);
        case 24: return resident_slots_of<2, 4>(G);
        case 22: return resident_slots_of<2, 2>(G);
        case 28: return resident_slots_of<2, 8>(G);
        case 84: return resident_slots_of<8, 4>(G);
        case 82: return resident_slots_of<8, 2>(G);
        default: return resident_slots_of<8, 8>(G);
    }
}

Plan plan_for(const hyq_decode_params* p) {
    const int kb = p->n_quant > 0 ? p->k_bits : 4, vb = p->n_quant > 0 ? p->v_bits : 4;
    return make_plan(p->n_quant, p->seg_n, p->bh_kv, p->kv_repeat, p->split_tokens, kb, vb,
                     resident_slots(kb, vb, p->kv_repeat));
}

// workspace: [arrival counters: CNT_CAP slots, 128 B apart][(m, l) table][partials].
// The counter area has the same size and place for every call, so the data of
// one call never lands on the counters of another call of a different shape.
struct Layout {
    size_t cnt, ml, part, total;
};
Layout layout(const Plan& pl, int bh_kv, int G) {
    const size_t slots = static_cast<size_t>(bh_kv) * std::max(pl.nwg, 1) * G;
    Layout L;
    L.cnt = 0;
    L.ml = static_cast<size_t>(CNT_CAP) * CNT_PAD * sizeof(uint32_t);
    L.part = L.ml + round256(slots * 2 * sizeof(float));
    L.total = L.part + round256(slots * D * sizeof(float));
    return L;
}

bool fits31(int64_t x) { return x >= 0 && x <= 0x7fffffffLL; }

int validate(const hyq_decode_params* p) {
    if (!p) return fail(HYQ_EINVAL, "null params");
    if (p->head_dim != D) return fail(HYQ_ENOTSUP, "head_dim must be 128, got " + std::to_string(p->head_dim));
    auto okbits = [](int b) { return b == 2 || b == 4 || b == 8; };
    if (!okbits(p->k_bits) || !okbits(p->v_bits))
        return fail(HYQ_EINVAL, "k_bits and v_bits must be 2, 4 or 8 (k_bits=" + std::to_string(p->k_bits) +
                                    ", v_bits=" + std::to_string(p->v_bits) + ")");
    if (p->kv_repeat < 1 || p->kv_repeat > 16)
        return fail(HYQ_ENOTSUP, "kv_repeat must be in [1, 16], got " + std::to_string(p->kv_repeat));
    if (p->bh_kv < 0) return fail(HYQ_EINVAL, "bh_kv < 0");
    if (p->bh_kv > CNT_CAP) return fail(HYQ_ENOTSUP, "bh_kv (batch * kv heads) above " + std::to_string(CNT_CAP));
    if (p->n_quant < 0 || p->n_quant > (1 << 24)) return fail(HYQ_EINVAL, "bad n_quant");
    if (p->dtype_flags & ~(HYQ_DT_Q_FP16 | HYQ_DT_SEG_FP16 | HYQ_DT_OUT_FP16))
        return fail(HYQ_EINVAL, "unknown dtype_flags bits " + std::to_string(p->dtype_flags));
    if (p->bh_kv == 0) return HYQ_OK;
    if (!p->q || !p->out) return fail(HYQ_EINVAL, "null q/out");
    if (!aligned(p->q, 16) || p->q_stride % 8 || p->q_stride < D)
        return fail(HYQ_EINVAL, "q must be 16-byte aligned with row stride % 8 == 0 and >= head_dim");
    if (static_cast<int64_t>(p->kv_repeat) * p->q_stride * 2 > 0x7fffffffLL) return fail(HYQ_ENOTSUP, "q row stride too large");
    if (!aligned(p->out, 8) || p->out_stride % 4 || p->out_stride < D)
        return fail(HYQ_EINVAL, "out must be 8-byte aligned with row stride % 4 == 0 and >= head_dim");
    if (!fits31(p->out_stride)) return fail(HYQ_ENOTSUP, "out row stride must lie in [0, 2^31)");
    if (p->n_quant > 0) {
        if (!p->k_packed || !p->v_packed || !p->k_scale || !p->v_scale) return fail(HYQ_EINVAL, "null prefix tensor");
        if (p->kp_stride_n != prow(p->k_bits) || p->vp_stride_n != prow(p->v_bits))
            return fail(HYQ_EINVAL, "packed K/V rows must be contiguous (token stride 16 * bits bytes)");
        const int ka = p->k_bits == 2 ? 8 : 16, va = p->v_bits;      // load sizes in bytes
        if (!aligned(p->k_packed, ka) || p->kp_stride_bh % ka)
            return fail(HYQ_EINVAL, "k_packed must be " + std::to_string(ka) + "-byte aligned, head stride included");
        if (!aligned(p->v_packed, va) || p->vp_stride_bh % va)
            return fail(HYQ_EINVAL, "v_packed must be " + std::to_string(va) + "-byte aligned, head stride included");
        if (!aligned(p->k_scale, 2) || !aligned(p->v_scale, 2))
            return fail(HYQ_EINVAL, "scales must be 2-byte aligned");
        if (!fits31(p->kp_stride_bh) || !fits31(p->vp_stride_bh) || !fits31(p->ks_stride_bh) || !fits31(p->vs_stride_bh))
            return fail(HYQ_ENOTSUP, "prefix head strides must lie in [0, 2^31)");
    }
    for (int s = 0; s < 3; ++s) {
        if (p->seg_n[s] < 0 || p->seg_n[s] > (1 << 23)) return fail(HYQ_EINVAL, "bad segment length");
        if (p->seg_n[s] == 0) continue;
        if (!p->seg_k[s] || !p->seg_v[s]) return fail(HYQ_EINVAL, "null bf16 segment");
        if (p->seg_k_stride_n[s] != BROW || p->seg_v_stride_n[s] != BROW)
            return fail(HYQ_EINVAL, "bf16 segment rows must be contiguous (token stride = head_dim)");
        if (!aligned(p->seg_k[s], 16) || !aligned(p->seg_v[s], 16) || p->seg_k_stride_bh[s] % 8 ||
            p->seg_v_stride_bh[s] % 8)
            return fail(HYQ_EINVAL, "bf16 segments must be 16-byte aligned with head strides % 8 == 0");
        if (!fits31(p->seg_k_stride_bh[s]) || !fits31(p->seg_v_stride_bh[s]))
            return fail(HYQ_ENOTSUP, "bf16 segment head strides must lie in [0, 2^31)");
    }
    return HYQ_OK;
}

// ---- legacy-format decode: plan and checks ----
struct LegPlan {
    int nwg = 0;
    int pfirst[5] = {0, 0, 0, 0, 0};
    int plen[4] = {LEG_PIECE, BF_PIECE, BF_PIECE, BF_PIECE};
};
// Workgroups of legacy_decode_kernel<KB, VB> the device holds at once (0:
// unknown), cached per device, variant and GQA width (the LDS size).
template <int KB, int VB>
int legacy_slots_of(int G) {
    static std::atomic<int> cache[64][17];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || G < 1 || G > 16) return 0;
    const int known = cache[dev][G].load(std::memory_order_relaxed);
    if (known > 0) return known;
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &per_cu, reinterpret_cast<const void*>(&legacy_decode_kernel<KB, VB>), THREADS, lds_bytes(G)) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return 0;
    cache[dev][G].store(per_cu * cus, std::memory_order_relaxed);
    return per_cu * cus;
}
int legacy_slots(int kb, int vb, int G) {
    switch (10 * kb + vb) {
        case 44: return legacy_slots_of<4, 4>(G);
        case 42: return legacy_slots_of<4, 2>(G);
        case 24: return legacy_slots_of<2, 4>(G);
        default: return legacy_slots_of<2, 2>(G);
    }
}

// Pieces grow while the prefix alone would still hand every resident slot a
// piece after the doubling: a piece carries a fixed cost (the Q load, the
// partial store, the arrival and merge), and a 512-token piece is only four
// two-tile iterations per wave.  Measured on one MI355X (128 key heads,
// 31000 tokens): 209 us with 512-token pieces, 187 us with 1024, 176 us with
// 2048; with 8 key heads 2048-token pieces left most CUs idle (33 us against
// 23 us).
LegPlan legacy_plan(const hyq_legacy_params* p) {
    LegPlan pl;
    const int64_t n[4] = {p->n, p->seg_n[0], p->seg_n[1], p->seg_n[2]};
    const int sl = legacy_slots(p->k_bits, p->v_bits, p->kv_repeat);
    const int64_t slots = sl > 0 ? sl : 768;
    // few heads: halve the pieces (down to 128 prefix tokens) while the grid
    // would leave CUs without a workgroup (slots / 3: one per CU)
    auto pieces = [&]() {
        int64_t t = 0;
        for (int s = 0; s < 4; ++s) t += (n[s] + pl.plen[s] - 1) / pl.plen[s];
        return t * p->bh_kv;
    };
    while (pl.plen[0] > LEG_PIECE_MIN && pieces() < slots / 3)
        for (int s = 0; s < 4; ++s) pl.plen[s] /= 2;
    while (pl.plen[0] < LEG_PIECE_MAX &&
           static_cast<int64_t>(p->bh_kv) * ((n[0] + 2 * pl.plen[0] - 1) / (2 * pl.plen[0])) >= slots)
        for (int s = 0; s < 4; ++s) pl.plen[s] *= 2;
    for (;;) {
        int64_t total = 0;
        for (int s = 0; s < 4; ++s) total += (n[s] + pl.plen[s] - 1) / pl.plen[s];
        if (total <= MAX_NWG && total * p->kv_repeat <= MAX_PARTIALS) break;
        for (int s = 0; s < 4; ++s) pl.plen[s] *= 2;
    }
    for (int s = 0; s < 4; ++s)
        pl.pfirst[s + 1] = pl.pfirst[s] + static_cast<int>((n[s] + pl.plen[s] - 1) / pl.plen[s]);
    pl.nwg = pl.pfirst[4];
    return pl;
}

int validate_legacy(const hyq_legacy_params* p) {
    const char* w = "hyq_decode_legacy: ";
    if (!p) return fail(HYQ_EINVAL, std::string(w) + "null params");
    if (p->head_dim != D) return fail(HYQ_ENOTSUP, std::string(w) + "head_dim must be 128");
    if ((p->k_bits != 2 && p->k_bits != 4) || (p->v_bits != 2 && p->v_bits != 4))
        return fail(HYQ_ENOTSUP, std::string(w) + "k_bits and v_bits must be 2 or 4");
    if (p->kv_repeat < 1 || p->kv_repeat > 16) return fail(HYQ_ENOTSUP, std::string(w) + "kv_repeat must be in [1, 16]");
    if (p->bh_kv < 0 || p->bh_kv > CNT_CAP) return fail(HYQ_ENOTSUP, std::string(w) + "bh_kv out of range");
    if (p->bh_kv == 0) return HYQ_OK;
    constexpr int64_t NMAX = int64_t{1} << 24;
    if (p->n < 0 || p->n > NMAX) return fail(HYQ_ENOTSUP, std::string(w) + "prefix length out of [0, 2^24]");
    int64_t total = p->n;
    for (int s = 0; s < 3; ++s) {
        if (p->seg_n[s] < 0 || p->seg_n[s] > NMAX) return fail(HYQ_ENOTSUP, std::string(w) + "segment length out of [0, 2^24]");
        total += p->seg_n[s];
        if (p->seg_n[s] == 0) continue;
        if (!p->seg_k[s] || !p->seg_v[s]) return fail(HYQ_EINVAL, std::string(w) + "null segment");
        if (!aligned(p->seg_k[s], 16) || !aligned(p->seg_v[s], 16) || p->seg_k_stride_bh[s] % 8 ||
            p->seg_v_stride_bh[s] % 8 || p->seg_k_stride_bh[s] < 0 || p->seg_v_stride_bh[s] < 0)
            return fail(HYQ_EINVAL, std::string(w) + "segments must be 16-byte aligned (head strides % 8 == 0)");
    }
    if (total == 0) return fail(HYQ_EINVAL, std::string(w) + "decode with zero key tokens");
    if (!p->q || !p->out) return fail(HYQ_EINVAL, std::string(w) + "null q or out");
    if (!aligned(p->q, 16) || p->q_stride % 8 || p->q_stride < D || p->q_stride > NMAX)
        return fail(HYQ_EINVAL, std::string(w) + "q rows must be 16-byte aligned, stride in [128, 2^24]");
    if (!aligned(p->out, 8) || p->out_stride % 4 || p->out_stride < D)
        return fail(HYQ_EINVAL, std::string(w) + "out rows must be 8-byte aligned");
    if (p->n > 0) {
        if (p->group <= 0 || p->group % 16) return fail(HYQ_EINVAL, std::string(w) + "group must be a positive multiple of 16");
        if (!p->k_codes || !p->v_codes || !p->k_scale || !p->v_scale) return fail(HYQ_EINVAL, std::string(w) + "null prefix");
        // a K row is read as one 4*k_bits-byte load per lane, a V row as
        // v_bits-byte loads: rows aligned to those sizes, at least 16*bits bytes
        const int ka = 4 * p->k_bits, va = p->v_bits, krow = 16 * p->k_bits, vrow = 16 * p->v_bits;
        if (!aligned(p->k_codes, ka) || p->kc_stride_n % ka || p->kc_stride_bh % ka || p->kc_stride_n < krow ||
            p->kc_stride_n > 4096 || p->kc_stride_bh < 0)
            return fail(HYQ_EINVAL, std::string(w) + "k_codes rows must be " + std::to_string(ka) +
                                        "-byte aligned, row stride in [" + std::to_string(krow) + ", 4096]");
        if (!aligned(p->v_codes, va) || p->vc_stride_n % va || p->vc_stride_bh % va || p->vc_stride_n < vrow ||
            p->vc_stride_n > 4096 || p->vc_stride_bh < 0)
            return fail(HYQ_EINVAL, std::string(w) + "v_codes rows must be " + std::to_string(va) +
                                        "-byte aligned, row stride in [" + std::to_string(vrow) + ", 4096]");
        if (!aligned(p->k_scale, 16) || !aligned(p->v_scale, 16) || p->ks_stride_g % 8 || p->vs_stride_g % 8 ||
            p->ks_stride_bh % 8 || p->vs_stride_bh % 8 || p->ks_stride_g < D || p->vs_stride_g < D ||
            p->ks_stride_bh < 0 || p->vs_stride_bh < 0)
            return fail(HYQ_EINVAL, std::string(w) + "scale rows must be 16-byte aligned (strides % 8 == 0)");
        const int64_t rows = (p->n + p->group - 1) / p->group;
        if (rows * std::max(p->ks_stride_g, p->vs_stride_g) * 2 > 0xffffffffLL)
            return fail(HYQ_ENOTSUP, std::string(w) + "a head's scale rows span 4 GiB or more");
    }
    return HYQ_OK;
}

int launch_legacy(const hyq_legacy_params* p, const LegPlan& pl, const Layout& L, void* workspace, void* stream) {
    LegArgs a{};
    a.q = p->q; a.q_stride = p->q_stride;
    a.kc = p->k_codes; a.vc = p->v_codes;
    a.kc_bh = p->kc_stride_bh; a.kc_n = p->kc_stride_n; a.vc_bh = p->vc_stride_bh; a.vc_n = p->vc_stride_n;
    a.ks = p->k_scale; a.vs = p->v_scale;
    a.ks_bh = p->ks_stride_bh; a.ks_g = p->ks_stride_g; a.vs_bh = p->vs_stride_bh; a.vs_g = p->vs_stride_g;
    a.group = p->n > 0 ? p->group : 1;
    a.ks_rows = a.vs_rows = (p->n + a.group - 1) / a.group;
    a.n_leg = static_cast<int>(p->n);
    for (int s = 0; s < 3; ++s) {
        a.sk[s] = p->seg_k[s]; a.sv[s] = p->seg_v[s];
        a.sk_bh[s] = p->seg_k_stride_bh[s]; a.sv_bh[s] = p->seg_v_stride_bh[s];
        a.sn[s] = static_cast<int>(p->seg_n[s]);
    }
    a.G = p->kv_repeat;
    a.qk_scale = p->sm_scale * LOG2E;
    char* ws = static_cast<char*>(workspace);
    a.cnt = reinterpret_cast<uint32_t*>(ws + L.cnt);
    a.ml = reinterpret_cast<float*>(ws + L.ml);
    a.part = reinterpret_cast<float*>(ws + L.part);
    a.out = p->out; a.out_stride = p->out_stride;
    a.nwg = pl.nwg;
    a.mj = merge_batch(a.G, pl.nwg);
    for (int s = 0; s < 5; ++s) a.pfirst[s] = pl.pfirst[s];
    for (int s = 0; s < 4; ++s) a.plen[s] = pl.plen[s];
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid(static_cast<unsigned>(p->bh_kv), static_cast<unsigned>(pl.nwg));
    const size_t lds = lds_bytes(a.G);
    switch (10 * p->k_bits + p->v_bits) {
        case 44: legacy_decode_kernel<4, 4><<<grid, dim3(THREADS), lds, st>>>(a); break;
        case 42: legacy_decode_kernel<4, 2><<<grid, dim3(THREADS), lds, st>>>(a); break;
        case 24: legacy_decode_kernel<2, 4><<<grid, dim3(THREADS), lds, st>>>(a); break;
        default: legacy_decode_kernel<2, 2><<<grid, dim3(THREADS), lds, st>>>(a); break;
    }
    return check_launch("hyq_decode_legacy");
}

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" size_t hyq_decode_workspace_size(const hyq_decode_params* p) {
    if (validate(p) != HYQ_OK) return 0;
    const Plan pl = plan_for(p);
    return layout(pl, p->bh_kv, p->kv_repeat).total;
}

namespace hyq {
namespace {

// The launch of hyq_decode_hybrid once the workspace is settled (p validated,
// the plan checked against the merge tables, the workspace L.total bytes,
// 256-byte aligned, its counter area zero).
int launch_decode(const hyq_decode_params* p, const Plan& pl, const Layout& L, void* workspace, void* stream) {
    DecArgs a{};
    a.q = p->q; a.q_stride = static_cast<int32_t>(p->q_stride);
    a.out = p->out; a.out_stride = static_cast<int32_t>(p->out_stride);
    a.io = p->dtype_flags;
    a.kp = reinterpret_cast<const uint8_t*>(p->k_packed); a.kp_bh = static_cast<int32_t>(p->kp_stride_bh);
    a.vp = reinterpret_cast<const uint8_t*>(p->v_packed); a.vp_bh = static_cast<int32_t>(p->vp_stride_bh);
    a.ks = p->k_scale; a.ks_bh = static_cast<int32_t>(p->ks_stride_bh);
    a.vs = p->v_scale; a.vs_bh = static_cast<int32_t>(p->vs_stride_bh);
    a.n_quant = static_cast<int32_t>(p->n_quant);
    for (int s = 0; s < 3; ++s) {
        a.sk[s] = p->seg_k[s]; a.sv[s] = p->seg_v[s];
        a.sk_bh[s] = static_cast<int32_t>(p->seg_k_stride_bh[s]);
        a.sv_bh[s] = static_cast<int32_t>(p->seg_v_stride_bh[s]);
        a.sn[s] = static_cast<int32_t>(p->seg_n[s]);
    }
    a.segu[0] = pl.segu[0]; a.segu[1] = pl.segu[1];
    a.G = p->kv_repeat;
    a.bh_kv = p->bh_kv;
    a.qk_scale = p->sm_scale * LOG2E;
    a.nqg = pl.nqg; a.nwg = pl.nwg;
    a.mj = merge_batch(p->kv_repeat, pl.nwg);
    for (int i = 0; i <= pl.nwg; ++i) a.bnd[i] = pl.bnd[i];
    char* ws = static_cast<char*>(workspace);
    a.cnt = reinterpret_cast<uint32_t*>(ws + L.cnt);
    a.ml = reinterpret_cast<float*>(ws + L.ml);
    a.part = reinterpret_cast<float*>(ws + L.part);
    a.len_q = p->n_quant > 0 ? p->seq_lens_quant : nullptr;
    a.len_s0 = p->seg_n[0] > 0 ? p->seq_lens_seg0 : nullptr;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // x: KV head, y: piece; workgroups dispatch x-fastest, so piece 0 of
    // every head goes first
    const dim3 grid(static_cast<unsigned>(p->bh_kv), static_cast<unsigned>(pl.nwg)), block(THREADS);
    const size_t lds = lds_bytes(p->kv_repeat);
    const int bits = p->n_quant > 0 ? 10 * p->k_bits + p->v_bits : 44;   // no prefix: any instance
    switch (bits) {
        case 44: decode_kernel<4, 4><<<grid, block, lds, s>>>(a); break;
        case 42: decode_kernel<4, 2><<<grid, block, lds, s>>>(a); break;
        case 48: decode_kernel<4, 8><<<grid, block, lds, s>>>(a); break;
        case 24: decode_kernel<2, 4><<<grid, block, lds, s>>>(a); break;
        case 22: decode_kernel<2, 2><<<grid, block, lds, s>>>(a); break;
        case 28: decode_kernel<2, 8><<<grid, block, lds, s>>>(a); break;
        case 84: decode_kernel<8, 4><<<grid, block, lds, s>>>(a); break;
        case 82: decode_kernel<8, 2><<<grid, block, lds, s>>>(a); break;
        default: decode_kernel<8, 8><<<grid, block, lds, s>>>(a); break;
    }
    return check_launch("hyq_decode_hybrid");
}

// validation, plan and layout shared by both decode entry points
int prepare(const hyq_decode_params* p, Plan& pl, Layout& L) {
    int rc = validate(p);
    if (rc != HYQ_OK) return rc;
    if (p->bh_kv == 0) return HYQ_OK;
    pl = plan_for(p);
    if (pl.nwg == 0) return fail(HYQ_EINVAL, "decode with zero key tokens");
    if (static_cast<int64_t>(pl.nwg) * p->kv_repeat > MAX_PARTIALS || pl.nwg > MAX_NWG)
        return fail(HYQ_ENOTSUP, "too many pieces per head for the merge tables");
    L = layout(pl, p->bh_kv, p->kv_repeat);
    return HYQ_OK;
}

// ---------------------------------------------------------------------------
// allocation-free variant: the workspace is a file-scope device array
// ---------------------------------------------------------------------------
constexpr size_t SCRATCH_BYTES = 16u << 20;     // counters (2 MiB) + (m, l) table and partials
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

__global__ void clear_words_kernel(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// This device's address of `scratch`, looked up once per device with that
// device current; the first lookup also clears the counter area on `stream`
// (a fill kernel, so that a captured first call records no memset node).
// Every completed decode launch leaves the counters at zero again.
int scratch_for_current_device(hipStream_t stream, void** out) {
    static std::mutex mu;
    static void* ptrs[64] = {nullptr};
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64)
        return fail(HYQ_EDEVICE, "hyq_decode_hybrid_noalloc: no current HIP device");
    std::lock_guard<std::mutex> lock(mu);
    if (ptrs[dev] == nullptr) {
        void* ptr = nullptr;
        const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || ptr == nullptr)
            return fail(HYQ_EDEVICE, std::string("hyq_decode_hybrid_noalloc: hipGetSymbolAddress failed: ") +
                                         hipGetErrorString(e));
        const int64_t words = static_cast<int64_t>(CNT_CAP) * CNT_PAD;
        clear_words_kernel<<<dim3(static_cast<unsigned>((words + 255) / 256)), dim3(256), 0, stream>>>(
            static_cast<uint32_t*>(ptr), words);
        if (int rc = check_launch("hyq_decode_hybrid_noalloc (clear)")) return rc;
        ptrs[dev] = ptr;
    }
    *out = ptrs[dev];
    return HYQ_OK;
}

}  // namespace
}  // namespace hyq

extern "C" int hyq_decode_hybrid(const hyq_decode_params* p, void* workspace, size_t ws_bytes, void* stream) {
    Plan pl{};
    Layout L{};
    int rc = prepare(p, pl, L);
    if (rc != HYQ_OK || p->bh_kv == 0) return rc;
    if (!workspace || ws_bytes < L.total || !aligned(workspace, 256))
        return fail(HYQ_ENOSPC, "decode workspace too small or misaligned: need " + std::to_string(L.total) + " bytes");
    return launch_decode(p, pl, L, workspace, stream);
}

extern "C" int hyq_decode_hybrid_noalloc(const hyq_decode_params* p, void* stream) {
    Plan pl{};
    Layout L{};
    int rc = prepare(p, pl, L);
    if (rc != HYQ_OK || p->bh_kv == 0) return rc;
    if (L.total > SCRATCH_BYTES)
        return fail(HYQ_ENOSPC, "hyq_decode_hybrid_noalloc: the call needs " + std::to_string(L.total) +
                                    " bytes of workspace, above the " + std::to_string(SCRATCH_BYTES) +
                                    "-byte scratch; use hyq_decode_hybrid");
    void* ws = nullptr;
    rc = scratch_for_current_device(static_cast<hipStream_t>(stream), &ws);
    if (rc != HYQ_OK) return rc;
    return launch_decode(p, pl, L, ws, stream);
}

#ifdef HYQ_PHASE_TRACE
// Copies the trace ring (TRACE_SLOTS x 4 TRACE_MAX_WG x TRACE_PH uint64) and
// the number of launches recorded to the host; trace build only.
extern "C" int hyq_phase_trace_read(uint64_t* dst, size_t bytes, uint32_t* launches) {
    const size_t need = sizeof(uint64_t) * TRACE_SLOTS * TRACE_MAX_WG * 4 * TRACE_PH;
    if (bytes < need) return fail(HYQ_ENOSPC, "phase trace buffer too small");
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_trace), need) != hipSuccess ||
        hipMemcpyFromSymbol(launches, HIP_SYMBOL(g_trace_launch), sizeof(uint32_t)) != hipSuccess)
        return fail(HYQ_EDEVICE, "phase trace copy failed");
    return HYQ_OK;
}
extern "C" int hyq_phase_trace_geometry(int32_t* slots, int32_t* max_wg, int32_t* phases) {
    *slots = TRACE_SLOTS; *max_wg = TRACE_MAX_WG * 4; *phases = TRACE_PH;
    return HYQ_OK;
}
#endif

extern "C" size_t hyq_decode_bf16_workspace_size(int32_t bh_kv, int32_t kv_repeat, int64_t n, int32_t d) {
    if (bh_kv < 0 || kv_repeat < 1 || kv_repeat > 16 || d != D || n < 0) return 0;
    const int64_t seg_n[3] = {n, 0, 0};
    const Plan pl = make_plan(0, seg_n, bh_kv, kv_repeat, 0, 4, 4, resident_slots(4, 4, kv_repeat));
    return layout(pl, bh_kv, kv_repeat).total;
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

extern "C" size_t hyq_decode_legacy_workspace_size(const hyq_legacy_params* p) {
    if (validate_legacy(p) != HYQ_OK || p->bh_kv == 0) return 0;
    Plan dp{};
    dp.nwg = legacy_plan(p).nwg;
    return layout(dp, p->bh_kv, p->kv_repeat).total;
}

extern "C" int hyq_decode_legacy(const hyq_legacy_params* p, void* workspace, size_t ws_bytes, void* stream) {
    int rc = validate_legacy(p);
    if (rc != HYQ_OK || p->bh_kv == 0) return rc;
    const LegPlan pl = legacy_plan(p);
    Plan dp{};
    dp.nwg = pl.nwg;
    const Layout L = layout(dp, p->bh_kv, p->kv_repeat);
    if (!workspace || ws_bytes < L.total || !aligned(workspace, 256))
        return fail(HYQ_ENOSPC, "hyq_decode_legacy: workspace too small or misaligned: need " + std::to_string(L.total) + " bytes");
    return launch_legacy(p, pl, L, workspace, stream);
}
