// Vertical-line selector (compute_vertical_indices, src/patch/_common.py:144-190)
// and the prefill->decode cache reorganisation (DStageLayerCache.freeze,
// src/ops/d_stage_kv_cache.py:106-189) for gfx950.
//
// Selector definition (bit-exact contract shared with the CPU oracle):
//   qm[b,ho,:]  = bf16( sum_t bf16( sum_r q[b, ho*R+r, QL-tail+t, :] / R ) / tail )
//                 (R = 1 for the prefill-time, per-query-head call; R = kv_repeat
//                 for the freeze-time call, src/ops/d_stage_kv_cache.py:131-133),
//                 each sum exact in float64 and each mean rounded once (RNE) to bf16;
//   score[p]    = bf16( sum_d qm[d] * k[p, d] )  with the sum taken in d order in
//                 float64 (bf16 x bf16 products are exact in float64);
//   an fp16 model (is_fp16) rounds the means and scores to fp16 instead: the
//                 reference computes them in the model dtype.
//   top-T       = the T largest scores, ties broken by the lower index, returned
//                 in (score desc, index asc) order (the lower-index rule fixes
//                 the unspecified tie order of torch.topk, src/patch/_common.py:189).
// Kernels:
//   qmean16_kernel    one workgroup per (b, ho): 16-byte row chunks x tail slots
//                     (qmean_kernel, channel pairs x tail slices, for query
//                     rows that are not 16-byte aligned); writes the means in
//                     float64 and as model-dtype bits, and zeroes the row's
//                     certified-key histogram.
//   score_mfma_kernel bf16 models: the scores on the matrix cores with a
//                     worst-case bound of their error; a key is stored exact
//                     where the bound certifies it, else as an upper bound
//                     with the position flagged uncertain; certified keys are
//                     counted per output row (HIST_BINS bins of the key).
//   score_kernel      fp16 models: one thread per key row in float64, G output
//                     heads sharing the row (exact keys, the same outputs).
//   topk_kernel       one workgroup per (b, ho) row: a candidate list of the
//                     positions whose stored key reaches the T-th largest
//                     certified key, float64 keys for its uncertain entries,
//                     then a counting rank (or a radix select and sort); the
//                     exact two-pass radix selection over the whole row when
//                     the list does not apply.  Output order "score desc,
//                     index asc" ("composite desc" for the unique composite
//                     (key << IDX_BITS) | (IDX_MASK - idx)).
//   mark_row_kernel (mark_kernel) / compact_quant_kernel / gather_rows_kernel  the freeze: a
//                     bitmap of selected prefix positions, quantisation of the
//                     unselected prefix rows straight into their compact slots
//                     (ascending position, F6), and the bf16 copies of the
//                     top-k rows (score order, F5) and of the window.
#include "hyq_common.h"

#include <algorithm>
#include <string>
#include <type_traits>

namespace hyq {
namespace {

constexpr int TOPK_THREADS = 512;            // threads of a top-k workgroup (at most; 256 when rows are many)
constexpr int64_t TOPK_NARROW_P = 65536;   // rows up to this long use 32-bit composites (16-bit index)
constexpr int64_t TOPK_MAX_P = 0x7fffffff; // 64-bit composites carry a 32-bit index
constexpr int TOPK_MAX_T = 1 << 30;         // the sort's power-of-two size n2 stays an int

// Certified keys per output row are counted in HIST_BINS bins of key >> HIST_SHIFT
// (half a bf16 binade each).  Inside a score workgroup the counts are 16-bit
// halves of LDS words (a workgroup counts at most 1024 rows per head).
constexpr int HIST_BINS = 1024;
constexpr int HIST_SHIFT = 6;
__device__ __forceinline__ void hist_add16(uint32_t* h, uint32_t key) {
    const uint32_t bin = key >> HIST_SHIFT;
    atomicAdd(&h[bin >> 1], 1u << (16 * (bin & 1)));
}
// adds a workgroup's packed counts of heads g < G to the rows' histograms
__device__ __forceinline__ void hist_flush16(const uint32_t* h, int G, uint32_t* __restrict__ hist, int64_t row0) {
    for (int i = threadIdx.x; i < G * (HIST_BINS / 2); i += blockDim.x) {
        const uint32_t c = h[i];
        if (!c) continue;
        uint32_t* r = hist + (row0 + i / (HIST_BINS / 2)) * HIST_BINS + 2 * (i % (HIST_BINS / 2));
        if (c & 0xffffu) atomicAdd(r, c & 0xffffu);
        if (c >> 16) atomicAdd(r + 1, c >> 16);
    }
}


__device__ __forceinline__ double bf16_bits_to_f64(uint16_t b) { return static_cast<double>(bf16_to_f32(b)); }

// an element of the model dtype (bf16, or fp16 when f16) as float64 (exact)
__device__ __forceinline__ double half_bits_to_f64(uint16_t b, bool f16) {
    return f16 ? static_cast<double>(f16_bits_to_f32(b)) : bf16_bits_to_f64(b);
}
// one RNE rounding of a float64 to the model dtype, as bits
__device__ __forceinline__ uint16_t f64_to_half_rne(double x, bool f16) {
    return f16 ? f64_to_f16_rne(x) : f64_to_bf16_rne(x);
}

// monotone key of a bf16 or fp16 value (-0 and +0 share a key); both formats
// keep the sign in bit 15 above a biased exponent, so one mapping orders both
__device__ __forceinline__ uint32_t orderable_key(uint16_t b) {
    uint32_t u = b;
    if (u == 0x8000u) u = 0;
    return (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
}

// qm as float64 (the exact value of the bf16 mean) for the score kernel.
// One workgroup of QM_THREADS per (b, hk, g < GP): lane l of wavefront w sums
// channel pair (2l, 2l+1) over the tail rows t = w, w + QM_SLICES, ...; the
// slices are added in LDS.  Heads g >= G (padding) get zeros.  Every partial
// sum is a sum of bf16 values (or of bf16 group means), exact in float64, so
// the split of the tail does not change the result.
constexpr int QM_THREADS = 1024;
constexpr int QM_SLICES = QM_THREADS / 64;

__global__ __launch_bounds__(QM_THREADS) void qmean_kernel(const uint16_t* __restrict__ q, int64_t qs_b, int64_t qs_h,
                                                           int64_t qs_t, int QL, int tail, int R, int HK, int G,
                                                           int GP, int f16, double* __restrict__ qm,
                                                           uint16_t* __restrict__ qb, uint32_t* __restrict__ hist) {
    const int row = blockIdx.x;                    // (b, hk, g)
    const int g = row % GP;
    const int bhk = row / GP;
    const int lane = threadIdx.x & 63, slice = threadIdx.x >> 6;
    double* out = qm + static_cast<int64_t>(row) * 128;
    uint16_t* outb = qb + static_cast<int64_t>(row) * 128;
    if (g >= G) {
        out[threadIdx.x & 127] = 0.0;
        outb[threadIdx.x & 127] = 0;
        return;
    }
    if (threadIdx.x < HIST_BINS) hist[(static_cast<int64_t>(bhk) * G + g) * HIST_BINS + threadIdx.x] = 0;
    const int b = bhk / HK, ho = (bhk % HK) * G + g;
    const uint32_t* base = reinterpret_cast<const uint32_t*>(
        q + b * qs_b + static_cast<int64_t>(ho * R) * qs_h + static_cast<int64_t>(QL - tail) * qs_t) + lane;
    const int64_t st = qs_t / 2, sh = qs_h / 2;     // in channel pairs
    double lo = 0.0, hi = 0.0;
    if (R == 1) {
        int t = slice;
        for (; t + 3 * QM_SLICES < tail; t += 4 * QM_SLICES) {
            uint32_t v[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) v[u] = base[static_cast<int64_t>(t + u * QM_SLICES) * st];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                lo += half_bits_to_f64(static_cast<uint16_t>(v[u]), f16);
                hi += half_bits_to_f64(static_cast<uint16_t>(v[u] >> 16), f16);
            }
        }
        for (; t < tail; t += QM_SLICES) {
            const uint32_t v = base[static_cast<int64_t>(t) * st];
            lo += half_bits_to_f64(static_cast<uint16_t>(v), f16);
            hi += half_bits_to_f64(static_cast<uint16_t>(v >> 16), f16);
        }
    } else {
        // four tail rows at a time, so that 4 R loads are in flight per step
        for (int t = slice; t < tail; t += 4 * QM_SLICES) {
            double ilo[4] = {0.0, 0.0, 0.0, 0.0}, ihi[4] = {0.0, 0.0, 0.0, 0.0};
            for (int r = 0; r < R; ++r) {
                uint32_t v[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int tu = t + u * QM_SLICES;
                    v[u] = tu < tail ? base[static_cast<int64_t>(r) * sh + static_cast<int64_t>(tu) * st] : 0u;
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    ilo[u] += half_bits_to_f64(static_cast<uint16_t>(v[u]), f16);
                    ihi[u] += half_bits_to_f64(static_cast<uint16_t>(v[u] >> 16), f16);
                }
            }
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                if (t + u * QM_SLICES < tail) {
                    lo += half_bits_to_f64(f64_to_half_rne(ilo[u] / R, f16), f16);
                    hi += half_bits_to_f64(f64_to_half_rne(ihi[u] / R, f16), f16);
                }
            }
        }
    }
    __shared__ double s_sum[QM_SLICES][128];
    s_sum[slice][2 * lane] = lo;
    s_sum[slice][2 * lane + 1] = hi;
    __syncthreads();
    if (threadIdx.x < 128) {
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < QM_SLICES; ++k) sum += s_sum[k][threadIdx.x];
        const uint16_t m = f64_to_half_rne(sum / tail, f16);
        out[threadIdx.x] = half_bits_to_f64(m, f16);
        outb[threadIdx.x] = m;
    }
}

// The same means from 16-byte loads, for query rows that are 16-byte aligned
// (every contiguous query tensor): 16 lanes hold one row (8 channels each),
// THREADS / 16 rows per pass of the workgroup, so each load instruction reads
// four whole rows.  The four row slots of a wavefront are added by lane
// shuffles, the wavefronts' sums in LDS; as above, every partial sum is exact
// in float64, so the result equals qmean_kernel's.  256 threads for the
// per-query-head means (one workgroup per output head), 1024 for the group
// means (a quarter as many workgroups, R heads read per row).

__device__ __forceinline__ void add8_f64(double (&acc)[8], uint4 v, bool f16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc[2 * i] += half_bits_to_f64(static_cast<uint16_t>(w[i]), f16);
        acc[2 * i + 1] += half_bits_to_f64(static_cast<uint16_t>(w[i] >> 16), f16);
    }
}

template <int THREADS, bool F16>
__global__ __launch_bounds__(THREADS) void qmean16_kernel(const uint16_t* __restrict__ q, int64_t qs_b, int64_t qs_h,
                                                            int64_t qs_t, int QL, int tail, int R, int HK, int G,
                                                            int GP, double* __restrict__ qm,
                                                            uint16_t* __restrict__ qb, uint32_t* __restrict__ hist) {
    const int row = blockIdx.x;                    // (b, hk, g)
    const int g = row % GP;
    const int bhk = row / GP;
    const int tid = threadIdx.x;
    double* out = qm + static_cast<int64_t>(row) * 128;
    uint16_t* outb = qb + static_cast<int64_t>(row) * 128;
    if (g >= G) {
        if (tid < 128) {
            out[tid] = 0.0;
            outb[tid] = 0;
        }
        return;
    }
    for (int i = tid; i < HIST_BINS; i += THREADS) hist[(static_cast<int64_t>(bhk) * G + g) * HIST_BINS + i] = 0;
    constexpr int QV_SLOTS = THREADS / 16;
    const int b = bhk / HK, ho = (bhk % HK) * G + g;
    const int sub = tid & 15, slot = tid >> 4;
    const uint16_t* base = q + b * qs_b + static_cast<int64_t>(ho * R) * qs_h + static_cast<int64_t>(QL - tail) * qs_t + 8 * sub;
    auto ld = [&](int r, int t) { return *reinterpret_cast<const uint4*>(base + r * qs_h + static_cast<int64_t>(t) * qs_t); };
    double acc[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
    const bool f16 = F16;
    if (R == 1) {
        // eight rows' loads in flight per thread (the kernel is bound by
        // their latency), added in row order
        int t = slot;
        for (; t + 7 * QV_SLOTS < tail; t += 8 * QV_SLOTS) {
            uint4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = ld(0, t + u * QV_SLOTS);
#pragma unroll
            for (int u = 0; u < 8; ++u) add8_f64(acc, v[u], f16);
        }
        for (; t < tail; t += QV_SLOTS) add8_f64(acc, ld(0, t), f16);
    } else {
        // the R heads of a row are averaged (one rounding to the model
        // dtype), then the row means summed; two rows per pass, two heads'
        // loads of both in flight at a time.  x / R is x * (1 / R), exact,
        // when R is a power of two.
        const bool pow2 = (R & (R - 1)) == 0;
        const double rinv = 1.0 / R;
        for (int t = slot; t < tail; t += 2 * QV_SLOTS) {
            const int t1 = min(t + QV_SLOTS, tail - 1);
            double g0[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0}, g1[8] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0};
            int r = 0;
            for (; r + 1 < R; r += 2) {
                uint4 v0[2], v1[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    v0[u] = ld(r + u, t);
                    v1[u] = ld(r + u, t1);
                }
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    add8_f64(g0, v0[u], f16);
                    add8_f64(g1, v1[u], f16);
                }
            }
            for (; r < R; ++r) {
                const uint4 v0 = ld(r, t), v1 = ld(r, t1);
                add8_f64(g0, v0, f16);
                add8_f64(g1, v1, f16);
            }
            const bool has1 = t + QV_SLOTS < tail;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const double m0 = pow2 ? g0[i] * rinv : g0[i] / R;
                const double m1 = pow2 ? g1[i] * rinv : g1[i] / R;
                acc[i] += half_bits_to_f64(f64_to_half_rne(m0, f16), f16);
                if (has1) acc[i] += half_bits_to_f64(f64_to_half_rne(m1, f16), f16);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        acc[i] += __shfl_xor(acc[i], 16, 64);
        acc[i] += __shfl_xor(acc[i], 32, 64);
    }
    __shared__ double s_sum[THREADS / 64][128];
    if ((tid & 63) < 16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) s_sum[tid >> 6][8 * sub + i] = acc[i];
    }
    __syncthreads();
    if (tid < 128) {
        double sum = 0.0;
#pragma unroll
        for (int k = 0; k < THREADS / 64; ++k) sum += s_sum[k][tid];
        const uint16_t m = f64_to_half_rne(sum / tail, F16);
        out[tid] = half_bits_to_f64(m, F16);
        outb[tid] = m;
    }
}

// keys of one output row start 16-byte aligned
__host__ __device__ inline int64_t key_pitch(int64_t P) { return (P + 7) / 8 * 8; }
// words of the uncertain bitmap per output row
__host__ __device__ inline int64_t unc_words(int64_t P) { return (P + 31) / 32; }

// Buffer descriptor over `bytes` bytes at `base`: loads past the range read
// zeros without touching memory, so the score kernel's loads need no branch
// (a branch around a load makes the compiler drain every load at the join).
typedef __amdgpu_buffer_rsrc_t Rsrc;
__device__ __forceinline__ Rsrc make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
constexpr int POL_NT = 2;                   // non-temporal: the K prefix is read once

// One workgroup per SC_WG_ROWS key rows of one (b, hk); wavefront w takes the
// 64-row blocks w, w + 4, ... of them.  The query means (float64, [GM][128])
// are the same for every lane: they are read by scalar loads and enter each
// FMA as an SGPR pair (read from LDS, every broadcast read moves 1 KB to the
// registers, and the GM = 4 kernel was bound by LDS bandwidth).  A block is
// streamed as two half-rows (64 channels, one 128-byte line per row): 8
// lanes per row, 16 bytes each, one 1 KB non-temporal load per 8 rows, into
// two register stages that are copied to the wavefront's LDS rows (pitch
// 144 B: the per-row reads hit every bank once per 16 lanes) and reloaded at
// once, so two half-blocks are in flight while lane r accumulates the GM dot products
// of row r sequentially in channel order in float64.  GM is G rounded up to
// 1, 2, 4, 8 or 16; the means are stored with zero rows past G, so the FMA
// loop has no branches and only the key store skips heads g >= G.  Rows past
// the prefix read zeros through the descriptor and are not stored.
constexpr int SC_ROWS = 64;                 // rows per block
constexpr int SC_PITCH = 144;               // LDS bytes per half-row (128 + 16)
constexpr int SC_BLOCKS = 4;                // blocks per wavefront
constexpr int SC_WG_ROWS = 4 * SC_BLOCKS * SC_ROWS;

template <int GM, bool F16>
__global__ __launch_bounds__(256) void score_kernel(const uint16_t* __restrict__ k, int64_t ks_b, int64_t ks_h,
                                                    int64_t ks_n, int HK, int G, int64_t P, int64_t KP,
                                                    const double* __restrict__ qm, uint16_t* __restrict__ keys,
                                                    uint32_t* __restrict__ unc, uint32_t* __restrict__ hist) {
    __shared__ __align__(16) uint8_t s_rows[4][SC_ROWS * SC_PITCH];
    __shared__ uint32_t s_hist[GM][HIST_BINS / 2];  // certified (here: all) keys, packed 16-bit counts
    for (int i = threadIdx.x; i < GM * (HIST_BINS / 2); i += 256) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    const int bh = blockIdx.y;                     // b * HK + hk
    const int b = bh / HK, hk = bh % HK;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * SC_WG_ROWS;
    const int nrows = static_cast<int>(min<int64_t>(SC_WG_ROWS, P - r0));
    const uint32_t rowb = static_cast<uint32_t>(ks_n) * 2;          // bytes between rows (host: < 2^20)
    const Rsrc rk = make_rsrc(k + b * ks_b + hk * ks_h + r0 * ks_n, static_cast<uint32_t>(nrows) * rowb);
    // blocks of this wavefront that hold rows: wave, wave + 4, ... below nrows
    const int nblk = (nrows + SC_ROWS - 1) / SC_ROWS;
    const int mine = nblk > wave ? (nblk - wave + 3) / 4 : 0;
    const int nst = 2 * mine;                      // half-block stages
    // lane l loads 16-byte chunk (l & 7) of rows 8i + (l >> 3) of a half-block
    const int sub = lane & 7, rq = lane >> 3;
    uint32_t vo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) vo[i] = static_cast<uint32_t>(8 * i + rq) * rowb + 16 * sub;
    // stage s: block wave + 4 (s >> 1), half s & 1
    auto soff = [&](int s) -> uint32_t {
        return static_cast<uint32_t>((wave + 4 * (s >> 1)) * SC_ROWS) * rowb + 128u * (s & 1);
    };
    auto load = [&](uint4 (&r)[8], int s) {
        const uint32_t so = soff(s);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, vo[i], so, POL_NT));
        // keep the stages in issue order: the wait for a stage counts the
        // loads issued after it, so interleaved stages would wait for each other
        __builtin_amdgcn_sched_barrier(0);
    };
    const double* qg = qm + static_cast<int64_t>(bh) * GM * 128;
    const int64_t UW = unc_words(P);
    uint4 ra[8], rb[8];
    if (nst > 0) {                                 // (nst is even: both first stages hold rows)
    load(ra, 0);
    load(rb, 1);
    uint8_t* lds = s_rows[wave];
    double acc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) acc[g] = 0.0;
    // One wavefront writes and reads its own LDS rows; its LDS accesses
    // execute in program order, so a stage's writes follow every read of the
    // previous stage and precede the reads of its own.
    auto stage = [&](const uint4 (&r)[8]) {
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(lds + (8 * i + rq) * SC_PITCH + 16 * sub) = r[i];
        __builtin_amdgcn_wave_barrier();
    };
    auto compute = [&](int s) {
        const uint8_t* row = lds + lane * SC_PITCH;
        const int half = s & 1;
#pragma unroll 1
        for (int c = 0; c < 8; ++c) {
            const uint4 w = *reinterpret_cast<const uint4*>(row + 16 * c);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
            double kv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                kv[j] = F16 ? static_cast<double>(f16_bits_to_f32(static_cast<uint16_t>(ww[j >> 1] >> (16 * (j & 1)))))
                            : static_cast<double>(__uint_as_float(j & 1 ? ww[j >> 1] & 0xffff0000u : ww[j >> 1] << 16));
            const int d0 = 64 * half + 8 * c;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[g] = fma(qg[g * 128 + d0 + j], kv[j], acc[g]);
            }
        }
        if (half) {
            const int64_t pb = r0 + (wave + 4 * (s >> 1)) * SC_ROWS;
            const int64_t p = pb + lane;
            if (p < P) {
#pragma unroll
                for (int g = 0; g < GM; ++g)
                    if (g < G) {
                        const uint32_t key = orderable_key(f64_to_half_rne(acc[g], F16));
                        keys[(static_cast<int64_t>(bh) * G + g) * KP + p] = static_cast<uint16_t>(key);
                        hist_add16(s_hist[g], key);
                    }
            }
            // every key here is exact: the block's uncertain words are zero
            if (lane < 2 * G && pb + 32 * (lane & 1) < P)
                unc[(static_cast<int64_t>(bh) * G + (lane >> 1)) * UW + pb / 32 + (lane & 1)] = 0u;
#pragma unroll
            for (int g = 0; g < GM; ++g) acc[g] = 0.0;
        }
    };
    // Two register stages and the LDS rows: a stage's registers are reloaded
    // as soon as they are copied to LDS, so the loads of the next two stages
    // are in flight while one is computed (stages past nst lie past the
    // descriptor's range: no memory access).  nst is even: no exit mid-loop,
    // which keeps the compiler's wait counts exact.
    for (int s = 0; s < nst; s += 2) {
        stage(ra);
        load(ra, s + 2);
        compute(s);
        stage(rb);
        load(rb, s + 3);
        compute(s + 1);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the last (empty) loads retire before the wave ends
    }
    __syncthreads();
    hist_flush16(&s_hist[0][0], G, hist, static_cast<int64_t>(bh) * G);
}

// ---------------------------------------------------------------------------
// bf16 scores on the matrix cores, with certified keys
// ---------------------------------------------------------------------------
// The score is bf16(R), R the float64 sequential sum of the exact products
// qm[g, d] * k[p, d] (score_kernel).  Here v_mfma_f32_16x16x32_bf16 takes 16
// key rows (M) by 32 channels (K) against the query means (N): each 32-channel
// chunk c of a row gives an fp32 partial D_c in an accumulator of its own,
// s = (D_0 + D_1) + (D_2 + D_3), and MFMAs over |k| and |qm| give
// A' = sum_c A'_c >= (1 - 2^-17) A, A = sum_d |qm_d k_d|.
//
// Error bound.  Model of the MFMA: the products of bf16 values are exact; the
// result differs from the exact sum of the products and the accumulator input
// by at most 32 * 2^-23 times the sum of their magnitudes, whatever the order
// and rounding of its additions, and equals the accumulator input when every
// product is zero; subnormal inputs, products and results may be flushed to
// zero.  Then
//   |D_c - S_c| <= 2^-18 A_c + 2^-120      (S_c the chunk's exact sum),
//   the three fp32 additions add at most 2^-23 A,
//   R lies within 127 * 2^-53 A of the exact sum,
//   flushed subnormal key elements lose at most 2^-126 sum_d |qm_d| <= 2^-59
//   when every nonzero |qm_d| lies in [2^-60, 2^60],
// so |s - R| <= 1.04 * 2^-18 A' + 2^-58.9.  With E = 2^-17 A' + 2^-56 the fp32
// ends lo = s - E and hi = s + E (rounded: below 2^-24 (|s| + E) each) still
// enclose R.  RNE to bf16 is monotone, so when bf16(lo) and bf16(hi) are one
// value, its key is the key of R: the score is certified.  Otherwise the pass
// stores the key of bf16(hi), an upper bound of the exact key, and sets the
// position's bit in the uncertain bitmap; A' above 2^100 (overflow, an
// infinite or NaN input) stores the largest key.  The top-k recomputes, in
// float64, the uncertain positions that can still be selected.  When a query
// mean has a NaN, an infinity or a nonzero |qm_d| outside [2^-60, 2^60], the
// pass computes that key head's scores in float64 instead (exact keys).
//
// The pass also counts each output row's certified keys in HIST_BINS bins
// (hist, zeroed by the query-mean kernel); the top-k starts from that count.
//
// One workgroup per SM_WG_ROWS rows of one (b, hk); wavefront w takes the
// 32-row stages w, w + 4, ...  A stage is 8 KB: eight 1 KB non-temporal loads
// (lane l: row 4i + l / 16, bytes 16 (l % 16) of it, so each instruction reads
// four whole rows) into one of two register stages, copied to the wavefront's
// LDS rows (pitch 272 B) and read back in the MFMA layout: lane l holds row
// l % 16, channels 32c + 8 (l / 16) .. + 7.
//
// Packing: with GM heads, TPK = 16 / GM row tiles share one accumulator.  The
// B operand of tile j is the query means in columns GM j .. GM j + GM - 1 and
// zero elsewhere, so column n ends up with head n % GM of tile n / GM, and
// every lane's four results (rows 4 (l / 16) + v of its column) are scores:
// the certification work is spread over all 64 lanes.  Tile j of a packed
// group of stages sits in stage j / 2 of the group, rows 16 (j % 2).
constexpr int SM_ROWS = 32;                 // rows per stage
constexpr int SM_PITCH = 272;               // LDS bytes per row (256 + 16)
constexpr int SM_STAGES = 8;                // stages per wavefront
constexpr int SM_WG_ROWS = 4 * SM_STAGES * SM_ROWS;

typedef __bf16 sel_bf16x8 __attribute__((ext_vector_type(8)));
typedef float sel_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));   // (non-temporal stores take clang vectors)
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// the exact (float64, d order) key of one bf16 row held in LDS, as score_kernel
__device__ __forceinline__ uint32_t exact_key_lds(const uint8_t* row, const double* q) {
    double acc = 0.0;
#pragma unroll 4
    for (int c = 0; c < 16; ++c) {
        const uint4 w = *reinterpret_cast<const uint4*>(row + 16 * c);
        const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float kv = __uint_as_float(j & 1 ? ww[j >> 1] & 0xffff0000u : ww[j >> 1] << 16);
            acc = fma(q[8 * c + j], static_cast<double>(kv), acc);
        }
    }
    return orderable_key(f64_to_bf16_rne(acc));
}

template <int GM>
__global__ __launch_bounds__(256) void score_mfma_kernel(const uint16_t* __restrict__ k, int64_t ks_b, int64_t ks_h,
                                                         int64_t ks_n, int HK, int G, int64_t P, int64_t KP,
                                                         const double* __restrict__ qm, const uint16_t* __restrict__ qb,
                                                         uint16_t* __restrict__ keys, uint32_t* __restrict__ unc,
                                                         uint32_t* __restrict__ hist) {
    constexpr int TPK = 16 / GM;                   // tiles per packed accumulator
    constexpr int SPK = TPK >= 2 ? TPK / 2 : 1;    // stages per packed group
    constexpr int SGRP = SPK >= 2 ? SPK : 2;       // stages per loop pass (two register stages)
    // GM <= 8: the workgroup's keys and uncertain words wait in LDS and are
    // written after its stream (GM = 16 would need 32 KB more LDS, one
    // workgroup per CU: its epilogues store directly)
    constexpr bool DEFER = GM <= 8;
    __shared__ __align__(16) uint8_t s_rows[4][SM_ROWS * SM_PITCH];
    __shared__ uint32_t s_hist[GM][HIST_BINS / 2];  // certified keys, packed 16-bit counts
    __shared__ __align__(16) uint16_t s_keys[DEFER ? GM : 1][DEFER ? SM_WG_ROWS : 8];
    __shared__ uint32_t s_unc[DEFER ? GM : 1][DEFER ? SM_WG_ROWS / 32 : 1];
    const int bh = blockIdx.y;                     // b * HK + hk
    const int b = bh / HK, hk = bh % HK;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int64_t r0 = static_cast<int64_t>(blockIdx.x) * SM_WG_ROWS;
    const int nrows = static_cast<int>(min<int64_t>(SM_WG_ROWS, P - r0));
    const uint32_t rowb = static_cast<uint32_t>(ks_n) * 2;          // bytes between rows (host: < 2^21)
    const Rsrc rk = make_rsrc(k + b * ks_b + hk * ks_h + r0 * ks_n, static_cast<uint32_t>(nrows) * rowb);
    const int nblk = (nrows + SM_ROWS - 1) / SM_ROWS;
    const int mine = nblk > wave ? (nblk - wave + 3) / 4 : 0;
    const int n = lane & 15, kg = lane >> 4;
    const int h = n % GM, jt = n / GM;             // head and tile of this lane's column
    // B operand of head h (bf16 bits of the means), and whether the means of
    // the key head's query heads are fit for the bound
    uint4 qw[4];
    bool bad = false;
    const uint16_t* qbrow = qb + (static_cast<int64_t>(bh) * GM + h) * 128;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        qw[c] = *reinterpret_cast<const uint4*>(qbrow + 32 * c + 8 * kg);
        const uint32_t ww[4] = {qw[c].x, qw[c].y, qw[c].z, qw[c].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t e = (ww[j >> 1] >> (16 * (j & 1))) & 0x7fffu;
            // zero, or |x| in [2^-60, 2^60]: biased exponent in [67, 187]
            bad |= !(e == 0 || (e >= (67u << 7) && e < (188u << 7)));
        }
    }
    const bool exact = __ballot(bad && h < G) != 0;   // the same in every workgroup of bh
    for (int i = threadIdx.x; i < GM * (HIST_BINS / 2); i += 256) (&s_hist[0][0])[i] = 0;
    __syncthreads();
    uint8_t* lds = s_rows[wave];
    const int sub = lane & 15, rq = lane >> 4;
    const uint32_t vo0 = static_cast<uint32_t>(rq) * rowb + 16 * sub;
    // the whole offset in the lane offset, which the descriptor's range check
    // covers: stages past the rows read zeros without touching memory
    auto load = [&](uint4 (&r)[8], int st) {
        const uint32_t so = static_cast<uint32_t>((wave + 4 * st) * SM_ROWS) * rowb;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            r[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rk, vo0 + so + 4 * i * rowb, 0, POL_NT));
        // keep the stages in issue order: a stage's wait counts the loads issued after it
        __builtin_amdgcn_sched_barrier(0);
    };
    // One wavefront writes and reads its own LDS rows, and its LDS accesses
    // execute in program order
    auto stage = [&](const uint4 (&r)[8]) {
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(lds + (4 * i + rq) * SM_PITCH + 16 * sub) = r[i];
        __builtin_amdgcn_wave_barrier();
    };
    const int64_t UW = unc_words(P);
    sel_f32x4 d[4], a[4];
    auto zero_acc = [&]() {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            d[c] = sel_f32x4{0.f, 0.f, 0.f, 0.f};
            a[c] = sel_f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // tile tj of the packed accumulator from LDS rows 16 t .. 16 t + 15
    auto mfma_tile = [&](int tj, int t) {
        uint32_t msk = jt == tj ? 0xffffffffu : 0u;
        asm volatile("" : "+v"(msk));              // per tile: hoisted, the masked operands would take 128 VGPRs
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const uint4 w = *reinterpret_cast<const uint4*>(lds + (16 * t + n) * SM_PITCH + 64 * c + 16 * kg);
            const uint4 wa = {w.x & 0x7fff7fffu, w.y & 0x7fff7fffu, w.z & 0x7fff7fffu, w.w & 0x7fff7fffu};
            const uint4 qv = {qw[c].x & msk, qw[c].y & msk, qw[c].z & msk, qw[c].w & msk};
            const uint4 qa = {qv.x & 0x7fff7fffu, qv.y & 0x7fff7fffu, qv.z & 0x7fff7fffu, qv.w & 0x7fff7fffu};
            d[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sel_bf16x8, w),
                                                          __builtin_bit_cast(sel_bf16x8, qv), d[c], 0, 0, 0);
            a[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sel_bf16x8, wa),
                                                          __builtin_bit_cast(sel_bf16x8, qa), a[c], 0, 0, 0);
        }
    };
    // Keys, histogram counts and uncertain bits of the packed accumulator of
    // the group starting at stage sfirst (GM <= 8), or of tile t1 of stage
    // sfirst (GM = 16).  Returns this lane's bits of its stage's word, OR-ed
    // over the lanes that share the word.
    auto epilogue = [&](int sfirst, int t1) -> uint32_t {
        const int st = TPK >= 2 ? sfirst + jt / 2 : sfirst;
        const int tin = TPK >= 2 ? (jt & 1) : t1;
        const int blk = wave + 4 * st;
        const int rt = blk * SM_ROWS + 16 * tin + 4 * kg;   // first of this lane's four rows
        uint32_t kv[4], nib = 0;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float sv = (d[0][v] + d[1][v]) + (d[2][v] + d[3][v]);
            const float av = (a[0][v] + a[1][v]) + (a[2][v] + a[3][v]);
            const float e = fmaf(av, 0x1p-17f, 0x1p-56f);
            const uint32_t lo = __float_as_uint(sv - e), hi = __float_as_uint(sv + e);
            const uint32_t blo = (lo + 0x7fffu + ((lo >> 16) & 1u)) >> 16;   // RNE to bf16 (finite values)
            const uint32_t bhi = (hi + 0x7fffu + ((hi >> 16) & 1u)) >> 16;
            const bool fin = av <= 0x1p100f;                                  // false for NaN
            const bool cert = fin && blo == bhi;
            const uint32_t key = orderable_key(static_cast<uint16_t>(bhi));
            kv[v] = fin ? key : 0xffffu;
            if (cert && rt + v < nrows && h < G) hist_add16(s_hist[h], key);
            nib |= (cert ? 0u : 1u) << v;
        }
        const u32x2_t kpair = {kv[0] | (kv[1] << 16), kv[2] | (kv[3] << 16)};
        if (DEFER) {
            // rt + 3 < SM_WG_ROWS: rt is a multiple of 4 below the workgroup's rows
            if (h < G && rt < SM_WG_ROWS) *reinterpret_cast<u32x2_t*>(&s_keys[DEFER ? h : 0][rt]) = kpair;
        } else if (h < G && rt < nrows) {
            uint16_t* kr = keys + (static_cast<int64_t>(bh) * G + h) * KP + r0 + rt;
            if (rt + 3 < nrows) {
                __builtin_nontemporal_store(kpair, reinterpret_cast<u32x2_t*>(kr));
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    if (rt + v < nrows) kr[v] = static_cast<uint16_t>(kv[v]);
            }
        }
        const int nv = min(4, max(0, nrows - rt));     // rows past the workgroup's end are not uncertain
        uint32_t word = (nib & ((1u << nv) - 1u)) << (16 * tin + 4 * kg);
        word |= __shfl_xor(word, 16, 64);
        word |= __shfl_xor(word, 32, 64);
        if (TPK >= 2) {                                // (DEFER)
            word |= __shfl_xor(word, GM, 64);          // the stage's other tile
            if (kg == 0 && (jt & 1) == 0 && h < G && blk < nblk) s_unc[DEFER ? h : 0][DEFER ? blk : 0] = word;
        }
        return word;
    };
    // float64 keys of one stage (rows of lanes 0 .. 31), every head
    auto exact_stage = [&](int blk) {
        const int rbase = blk * SM_ROWS;
        if (lane < SM_ROWS && rbase + lane < nrows) {
            for (int g = 0; g < G; ++g) {
                const uint32_t key = exact_key_lds(lds + lane * SM_PITCH, qm + (static_cast<int64_t>(bh) * GM + g) * 128);
                keys[(static_cast<int64_t>(bh) * G + g) * KP + r0 + rbase + lane] = static_cast<uint16_t>(key);
                hist_add16(s_hist[g], key);
            }
        }
        if (lane < G) unc[(static_cast<int64_t>(bh) * G + lane) * UW + r0 / 32 + blk] = 0u;
    };
    // stage st, already in LDS (sg: its place in the packed group): MFMAs,
    // or the float64 keys
    auto compute = [&](int st, int sg) {
        const int blk = wave + 4 * st;
        if (exact) {
            if (blk < nblk) exact_stage(blk);
            return;
        }
        if (TPK >= 2) {
            if (sg == 0) zero_acc();
            mfma_tile(2 * sg, 0);
            mfma_tile(2 * sg + 1, 1);
            if (sg == SPK - 1) epilogue(st - SPK + 1, 0);
        } else {
            zero_acc();
            mfma_tile(0, 0);
            uint32_t w = epilogue(st, 0);
            zero_acc();
            mfma_tile(0, 1);
            w |= epilogue(st, 1);
            if (kg == 0 && h < G && blk < nblk) unc[(static_cast<int64_t>(bh) * G + h) * UW + r0 / 32 + blk] = w;
        }
    };
    // Stages past `mine` lie past the descriptor's range (zeros, nothing
    // stored).  The loop runs whole packed groups of stages and whole pairs
    // of register stages; a register stage is reloaded as soon as it is
    // copied to LDS, so two stages' loads are in flight while one is computed.
    const int nst = (mine + SGRP - 1) / SGRP * SGRP;
    if (nst > 0) {
        uint4 ra[8], rb[8];
        load(ra, 0);
        load(rb, 1);
        for (int s0 = 0; s0 < nst; s0 += SGRP) {
#pragma unroll
            for (int u = 0; u < SGRP; u += 2) {
                stage(ra);
                load(ra, s0 + u + 2);
                compute(s0 + u, u % SPK);
                stage(rb);
                load(rb, s0 + u + 3);
                compute(s0 + u + 1, (u + 1) % SPK);
            }
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the last (empty) loads retire before the wave ends
    }
    __syncthreads();
    if (DEFER && !exact) {
        // The keys and uncertain words of the workgroup's rows.  Stores mixed
        // into the K stream cost about as much as 20 us of reading per 32 MB
        // written on MI355X's HBM wherever they fall; written here, in whole
        // 16-byte pieces and non-temporal, they cost the least measured.
        for (int i = threadIdx.x; i < G * (SM_WG_ROWS / 8); i += 256) {
            const int hh = i / (SM_WG_ROWS / 8), row = 8 * (i % (SM_WG_ROWS / 8));
            if (row >= nrows) continue;
            uint16_t* kr = keys + (static_cast<int64_t>(bh) * G + hh) * KP + r0 + row;
            const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&s_keys[DEFER ? hh : 0][DEFER ? row : 0]);
            if (row + 8 <= nrows) {
                __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(kr));   // KP and r0: multiples of 8
            } else {
                for (int j = 0; j < nrows - row; ++j) kr[j] = static_cast<uint16_t>(v[j >> 1] >> (16 * (j & 1)));
            }
        }
        for (int i = threadIdx.x; i < G * (SM_WG_ROWS / 32); i += 256) {
            const int hh = i / (SM_WG_ROWS / 32), blk = i % (SM_WG_ROWS / 32);
            if (blk < nblk) unc[(static_cast<int64_t>(bh) * G + hh) * UW + r0 / 32 + blk] = s_unc[DEFER ? hh : 0][DEFER ? blk : 0];
        }
    }
    hist_flush16(&s_hist[0][0], G, hist, static_cast<int64_t>(bh) * G);
}

constexpr int TOPK_WAVES = TOPK_THREADS / 64;
// histogram copies: one per pair of wavefronts, which keeps a 16K-key row's
// LDS (keys, histograms, winners) under 40 KiB, four workgroups per CU
constexpr int TOPK_HIST = TOPK_WAVES / 2;
// the LDS histogram area: the copies above, or the certified-key histogram
constexpr int TOPK_HIST_AREA = TOPK_HIST * 256 > HIST_BINS ? TOPK_HIST * 256 : HIST_BINS;
static_assert(TOPK_HIST_AREA == HIST_BINS, "both block sizes share one LDS layout");
constexpr int TOPK_RANK_MAX = 2048;        // winners the rank path's per-thread arrays can hold
// rows with up to this many winners are placed by rank (each winner compared
// with every other: T / 4 LDS steps per thread); larger rows are bitonic
// sorted (log2(n2) (log2(n2) + 1) / 2 barrier-separated stages), which costs
// less vector work from about 512 winners up
constexpr int TOPK_RANK_LIMIT = 512;
// key offsets above the candidate bound that the counting rank covers
constexpr int TOPK_SPAN = 1024;
constexpr size_t TOPK_LDS_MAX = 64 * 1024; // keys are cached in LDS while the row fits this budget

// Wavefront 0: the bin holding the need-th largest entry of an NBINS-bin
// histogram, scanning from the top.  Writes the bin and the entries still
// needed inside it.
template <int NBINS>
__device__ __forceinline__ void topk_find_bin_n(const uint32_t* hist, uint32_t need, int lane, uint32_t* s_bin,
                                                uint32_t* s_need) {
    constexpr int PER = NBINS / 64;               // bins per lane, from the top
    uint32_t c[PER];
    uint32_t mine = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        c[j] = hist[NBINS - 1 - (PER * lane + j)];
        mine += c[j];
    }
    uint32_t incl = mine;                          // inclusive prefix over lanes (bins from the top)
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    uint32_t acc = incl - mine;
    int found = -1;
    uint32_t before = 0;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        if (found < 0 && acc + c[j] >= need) {
            found = NBINS - 1 - (PER * lane + j);
            before = acc;
        }
        acc += c[j];
    }
    // the first lane (highest bins) that found it wins; the candidates always
    // number at least `need`, so some lane finds it (were it not so, bin 0
    // would be taken, as a top-down scan would)
    const uint64_t ball = __ballot(found >= 0);
    const int first = ball ? __ffsll(static_cast<long long>(ball)) - 1 : 63;
    if (lane == first) {
        if (found < 0) {
            found = 0;
            before = acc - c[PER - 1];
        }
        *s_bin = static_cast<uint32_t>(found);
        *s_need = need - before;
    }
}
__device__ __forceinline__ void topk_find_bin(const uint32_t* hist, uint32_t need, int lane, uint32_t* s_bin,
                                              uint32_t* s_need) {
    topk_find_bin_n<256>(hist, need, lane, s_bin, s_need);
}

// The composite of one entry: (key << IDX_BITS) | (IDX_MASK - idx), unique,
// and "score desc, index asc" is "composite desc".  32 bits (16-bit index)
// while the row has at most 65536 positions, 64 bits (32-bit index) beyond.
template <typename C>
struct Comp {
    static constexpr int IDX_BITS = sizeof(C) == 4 ? 16 : 32;
    static constexpr C IDX_MASK = (static_cast<C>(1) << IDX_BITS) - 1;
    __device__ static C make(uint32_t key, int64_t idx) {
        return (static_cast<C>(key) << IDX_BITS) | (IDX_MASK - static_cast<C>(idx));
    }
    __device__ static int64_t index(C c) { return static_cast<int64_t>(IDX_MASK - (c & IDX_MASK)); }
};

// four composites starting at s[4j] (16-byte aligned groups)
__device__ __forceinline__ void load4(const uint32_t* s, int j, uint32_t (&w)[4]) {
    const uint4 v = reinterpret_cast<const uint4*>(s)[j];
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
}
__device__ __forceinline__ void load4(const uint64_t* s, int j, uint64_t (&w)[4]) {
    const ulonglong2 a = reinterpret_cast<const ulonglong2*>(s)[2 * j];
    const ulonglong2 b = reinterpret_cast<const ulonglong2*>(s)[2 * j + 1];
    w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y;
}

// Writes the indices of the T composites in sel (unique, zero-padded to n2)
// in descending order: each at its rank among them (rank_ok: T <= TOPK_RANK_LIMIT
// and sel in LDS; a thread ranks its up to four winners in one sweep, every
// lane of a wavefront reading the same four composites per step), or after
// a bitonic sort of the n2 entries.  Ends with the workgroup's threads done.
template <typename C, int NT>
__device__ void topk_sort_out(C* sel, int T, int n2, bool rank_ok, int64_t* __restrict__ orow) {
    const int tid = threadIdx.x;
    if (rank_ok) {
        constexpr int E = TOPK_RANK_MAX / NT;
        C v[E];
        uint32_t rank[E];
#pragma unroll
        for (int u = 0; u < E; ++u) {
            v[u] = tid + u * NT < T ? sel[tid + u * NT] : C(0);
            rank[u] = 0;
        }
        const int ne = (T - tid + NT - 1) / NT;   // winners of this thread
        if (ne > 2) {
            for (int j = 0; j < n2 / 4; ++j) {
                C w[4];
                load4(sel, j, w);
#pragma unroll
                for (int u = 0; u < E; ++u) rank[u] += (w[0] > v[u]) + (w[1] > v[u]) + (w[2] > v[u]) + (w[3] > v[u]);
            }
        } else if (ne > 0) {
            for (int j = 0; j < n2 / 4; ++j) {
                C w[4];
                load4(sel, j, w);
#pragma unroll
                for (int u = 0; u < 2; ++u) rank[u] += (w[0] > v[u]) + (w[1] > v[u]) + (w[2] > v[u]) + (w[3] > v[u]);
            }
        }
#pragma unroll
        for (int u = 0; u < E; ++u)
            if (u < ne) orow[rank[u]] = Comp<C>::index(v[u]);
        return;
    }
    if (n2 == 2 * NT) {
        // 1024 entries in registers, two per thread: entry 128 w + 64 r + l
        // sits in register r of lane l of wavefront w.  Compare-exchanges
        // with partners in the same wavefront use the other register
        // (stride 64) or a lane shuffle; strides of 128 and more go through
        // sel with a barrier on each side.
        const int wv = tid >> 6, ln = tid & 63;
        C v[2] = {sel[128 * wv + ln], sel[128 * wv + 64 + ln]};
        auto keep = [](C mine, C other, bool take_max) { return take_max ? (mine > other ? mine : other)
                                                                        : (mine < other ? mine : other); };
        for (int size = 2; size <= n2; size <<= 1) {
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                if (stride >= 128) {
#pragma unroll
                    for (int r = 0; r < 2; ++r) sel[128 * wv + 64 * r + ln] = v[r];
                    __syncthreads();
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const int i = 128 * wv + 64 * r + ln;
                        v[r] = keep(v[r], sel[i ^ stride], ((i & stride) == 0) == ((i & size) == 0));
                    }
                    __syncthreads();
                } else if (stride == 64) {
                    const int i0 = 128 * wv + ln;              // the lower entry of the pair is register 0
                    const bool desc = (i0 & size) == 0;
                    const C hi = v[0] > v[1] ? v[0] : v[1], lo = v[0] > v[1] ? v[1] : v[0];
                    v[0] = desc ? hi : lo;
                    v[1] = desc ? lo : hi;
                } else {
#pragma unroll
                    for (int r = 0; r < 2; ++r) {
                        const int i = 128 * wv + 64 * r + ln;
                        C o;
                        if constexpr (sizeof(C) == 4) {
                            o = static_cast<C>(__shfl_xor(static_cast<int>(v[r]), stride, 64));
                        } else {
                            const int lo32 = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v[r])), stride, 64);
                            const int hi32 = __shfl_xor(static_cast<int>(static_cast<uint32_t>(v[r] >> 32)), stride, 64);
                            o = (static_cast<C>(static_cast<uint32_t>(hi32)) << 32) | static_cast<uint32_t>(lo32);
                        }
                        v[r] = keep(v[r], o, ((i & stride) == 0) == ((i & size) == 0));
                    }
                }
            }
        }
        for (int r = 0; r < 2; ++r) {
            const int i = 128 * wv + 64 * r + ln;
            if (i < T) orow[i] = Comp<C>::index(v[r]);
        }
        return;
    }
    // bitonic sort, descending
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n2 / 2; i += NT) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const C x = sel[lo], y = sel[hi];
                if ((x < y) == desc) {
                    sel[lo] = y;
                    sel[hi] = x;
                }
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < T; i += NT) orow[i] = Comp<C>::index(sel[i]);
}

// The top T of one row of exact 16-bit keys kr (global; s_keys: a copy in
// LDS, or null).  Two radix passes over the keys (one histogram per pair of
// wavefronts) find the threshold key K and how many of the entries equal to
// K are taken (the r of lowest index: a prefix count over contiguous
// per-thread index ranges); the T winners' composites are collected in sel
// (n2 entries, LDS or this row's slice of a global buffer) and placed by
// topk_sort_out.
template <typename C, int NT>
__device__ void topk_exact_row(const uint16_t* __restrict__ kr, const uint16_t* s_keys, int64_t P, int T, int n2,
                               bool rank_ok, C* sel, uint32_t* hist, int64_t* __restrict__ orow) {
    __shared__ uint32_t s_bin, s_need, s_count;
    __shared__ uint32_t s_wsum[(NT / 64)];
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    auto key_at = [&](int64_t i) -> uint32_t { return s_keys ? s_keys[i] : kr[i]; };
    uint32_t need = static_cast<uint32_t>(T);
    uint32_t khi = 0;
    for (int pass = 0; pass < 2; ++pass) {
        for (int i = tid; i < (NT / 128) * 256; i += NT) hist[i] = 0;
        __syncthreads();
        for (int64_t i = tid; i < P; i += NT) {
            const uint32_t key = key_at(i);
            if (pass == 0) atomicAdd(&hist[(wave >> 1) * 256 + (key >> 8)], 1u);
            else if ((key >> 8) == khi) atomicAdd(&hist[(wave >> 1) * 256 + (key & 0xffu)], 1u);
        }
        __syncthreads();
        if (tid < 256) {
            uint32_t sum = 0;
#pragma unroll
            for (int w = 0; w < (NT / 128); ++w) sum += hist[w * 256 + tid];
            hist[tid] = sum;
        }
        __syncthreads();
        if (wave == 0) topk_find_bin(hist, need, lane, &s_bin, &s_need);
        __syncthreads();
        if (pass == 0) khi = s_bin;
        need = s_need;
    }
    const uint32_t kth = (khi << 8) | s_bin;       // threshold key
    const uint32_t r = need;                       // entries equal to kth that are taken
    // thread t scans indices [t*C, t*C + C) (C a multiple of 8, read 16 bytes
    // at a time): entries above kth are winners; the entries equal to kth are
    // numbered in index order by a prefix count over the threads
    const int64_t CH = (P + 8 * NT - 1) / (8 * NT) * 8;
    const int64_t i0 = static_cast<int64_t>(tid) * CH;
    const uint4* k4 = s_keys ? reinterpret_cast<const uint4*>(s_keys) : reinterpret_cast<const uint4*>(kr);
    if (tid == 0) s_count = 0;
    uint32_t eq = 0;
    for (int64_t ib = i0; ib < i0 + CH && ib < P; ib += 8) {
        const uint4 w = k4[ib >> 3];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) eq += (ib + j < P) && ((ws[j >> 1] >> (16 * (j & 1))) & 0xffffu) == kth;
    }
    uint32_t incl = eq;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    if (lane == 63) s_wsum[wave] = incl;
    __syncthreads();
    uint32_t base = incl - eq;
    for (int w = 0; w < wave; ++w) base += s_wsum[w];
    for (int64_t ib = i0; ib < i0 + CH && ib < P; ib += 8) {
        const uint4 w = k4[ib >> 3];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int64_t i = ib + j;
            const uint32_t key = (ws[j >> 1] >> (16 * (j & 1))) & 0xffffu;
            bool take = i < P && key > kth;
            if (i < P && key == kth) take = base++ < r;
            if (take) sel[atomicAdd(&s_count, 1u)] = Comp<C>::make(key, i);
        }
    }
    for (int i = T + tid; i < n2; i += NT) sel[i] = 0;   // real composites are > 0
    __syncthreads();
    topk_sort_out<C, NT>(sel, T, n2, rank_ok, orow);
}

// The exact key (float64, d order, one rounding to the model dtype: the
// score kernels' arithmetic) of the key row at krow; q: the query mean in LDS
template <bool F16>
__device__ __forceinline__ uint32_t exact_key_row_t(const uint16_t* __restrict__ krow, const double* q) {
    uint4 w[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) w[c] = reinterpret_cast<const uint4*>(krow)[c];
    // an offset the compiler cannot see through: the mean's 128 loads stay
    // in the loop body instead of 256 VGPRs hoisted out of it
    int z = 0;
    asm volatile("" : "+v"(z));
    double acc = 0.0;
#pragma unroll
    for (int c = 0; c < 16; ++c) {
        const uint32_t ww[4] = {w[c].x, w[c].y, w[c].z, w[c].w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
            acc = fma(q[z + 8 * c + j], half_bits_to_f64(static_cast<uint16_t>(ww[j >> 1] >> (16 * (j & 1))), F16), acc);
    }
    return orderable_key(f64_to_half_rne(acc, F16));
}
// (the model dtype chosen once: a run-time dtype inside the unrolled loop
// kept both conversions of all 128 elements live)
__device__ __forceinline__ uint32_t exact_key_row(const uint16_t* __restrict__ krow, const double* q, bool f16) {
    return f16 ? exact_key_row_t<true>(krow, q) : exact_key_row_t<false>(krow, q);
}

struct TopkArgs {
    uint16_t* keys;                  // [rows][KP] keys (exact, or upper bounds where uncertain)
    const uint32_t* unc;             // [rows][UW] uncertain bits
    const uint32_t* hist;            // [rows][HIST_BINS] certified keys by key >> HIST_SHIFT
    int64_t P, KP, UW;
    int T, n2, cap;                  // winners, sort size, candidate list capacity
    int fast;                        // the candidate path fits the LDS (else every row takes the exact path)
    int gsort;                       // the exact path sorts in gsel (n2 composites per row)
    void* gsel;
    const uint16_t* k;               // key rows of the uncertain positions' recomputation
    int64_t ks_b, ks_h, ks_n;
    int HK, G, GP, f16;
    const double* qm;                // [b * HK][GP][128] query means
    int64_t* out;                    // [rows][T]
};

// One workgroup per (b, ho) row.
// Candidate path: the certified histogram (bins of key >> HIST_SHIFT) gives
// the bin b of the T-th largest certified key.  One pass over the row lists
// every position whose stored key (exact, or an upper bound) is >= the bin's
// first key and counts the certified keys of bin b by their low bits, which
// gives L, the T-th largest certified key.
// The certified keys are exact and at least T of them are >= L, so the T-th
// largest exact key K is >= L, and the list holds every position whose exact
// key is >= L: the row's top T (were the list over its capacity, a second
// pass lists the keys >= L only).  The uncertain entries whose stored key is
// >= L get their exact keys in float64 (the others are below L, so below K,
// whatever their exact key), four (six) byte passes of a radix select over
// the unique composites (key << IDX_BITS) | (IDX_MASK - idx) find the T-th
// largest, and the T composites at or above it are placed by topk_sort_out.
// Exact path (fewer than T certified keys, or a list over its capacity): the
// row's uncertain keys are recomputed in place in the keys array, then
// topk_exact_row runs on the exact keys.
// Dynamic LDS: [hist][list (cap C)][sel (n2 C)][uncertain flags (cap bytes)];
// the exact path uses [hist][sel] (gsort: the global buffer).
template <typename C, int NT>
__global__ __launch_bounds__(NT) void topk_kernel(TopkArgs a) {
    extern __shared__ __align__(16) uint32_t tk_lds[];
    uint32_t* hist = tk_lds;                       // [TOPK_HIST_AREA]
    C* list = reinterpret_cast<C*>(tk_lds + TOPK_HIST_AREA);
    C* sel_f = list + a.cap;
    uint8_t* flags = reinterpret_cast<uint8_t*>(sel_f + a.n2);   // uncertain entries of the list
    uint32_t* brk = reinterpret_cast<uint32_t*>(flags + (a.cap + 15) / 16 * 16);   // buckets: counts, starts
    C* brank_tmp = reinterpret_cast<C*>(brk + 2 * TOPK_SPAN);      // entries >= L in bucket order
    __shared__ uint32_t s_bin, s_need, s_count, s_total, s_ovf;
    __shared__ uint32_t s_wtot[(NT / 64)];
    __shared__ uint32_t s_lohist[64];
    __shared__ double s_q[128];
    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    uint16_t* kr = a.keys + static_cast<int64_t>(row) * a.KP;
    const uint32_t* ur = a.unc + static_cast<int64_t>(row) * a.UW;
    int64_t* orow = a.out + static_cast<int64_t>(row) * a.T;
    // key rows and query means of this output row
    const int H_out = a.HK * a.G;
    const int b = row / H_out, ho = row % H_out, hk = ho / a.G, g = ho % a.G;
    const uint16_t* kbase = a.k + b * a.ks_b + hk * a.ks_h;
    if (tid < 128) s_q[tid] = a.qm[(static_cast<int64_t>(b * a.HK + hk) * a.GP + g) * 128 + tid];
    const double* q = s_q;                         // (read after the first barrier below)
    constexpr int NB = sizeof(C) == 4 ? 4 : 6;     // significant bytes of a composite
    bool exact_path = !a.fast;
    if (a.fast) {
        for (int i = tid; i < HIST_BINS; i += NT) hist[i] = a.hist[static_cast<int64_t>(row) * HIST_BINS + i];
        if (tid == 0) s_count = 0;
        __syncthreads();
        if (wave == 0) {
            uint32_t t = 0;
#pragma unroll
            for (int j = 0; j < HIST_BINS / 64; ++j) t += hist[(HIST_BINS / 64) * lane + j];
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off, 64);
            if (lane == 0) s_total = t;
            topk_find_bin_n<HIST_BINS>(hist, static_cast<uint32_t>(a.T), lane, &s_bin, &s_need);
        }
        __syncthreads();
        exact_path = s_total < static_cast<uint32_t>(a.T);
        if (!exact_path) {
            constexpr uint32_t LOW = (1u << HIST_SHIFT) - 1u;
            const uint32_t bsel = s_bin, need_lo = s_need;
            uint32_t* lohist = s_lohist;            // certified keys of bin bsel by their low bits
            if (tid < 64) lohist[tid] = 0;
            __syncthreads();
            // One pass over the row, CU x 8 keys (16-byte loads) and their
            // uncertain bits per thread at a time: every key >= the first key
            // of bin bsel joins the list (one LDS atomic per wavefront and step), and the
            // certified keys of bin bsel are counted by their low bits.  L, the
            // T-th largest certified key, is then the bound; list entries
            // below it are harmless (their exact keys are below L <= K).
            constexpr int CU = NT == 256 ? 8 : 4;   // 16-byte key loads in flight per thread
            auto collect = [&](uint32_t lim, bool count_lo) {
                // (the trip count is the wavefront's: the shuffles below need every lane)
                for (int64_t i0 = 8 * static_cast<int64_t>(tid); i0 - 8 * lane < a.P; i0 += 8 * CU * NT) {
                    uint4 w[CU];
                    uint32_t ub[CU];
#pragma unroll
                    for (int u = 0; u < CU; ++u) {
                        const int64_t ib = i0 + u * 8 * NT;
                        w[u] = ib < a.P ? *reinterpret_cast<const uint4*>(kr + ib) : uint4{0, 0, 0, 0};
                        ub[u] = ib < a.P ? (ur[ib >> 5] >> (ib & 31)) & 0xffu : 0u;
                    }
                    uint32_t take[CU], c = 0;
#pragma unroll
                    for (int u = 0; u < CU; ++u) {
                        const int64_t ib = i0 + u * 8 * NT;
                        const uint32_t ws[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
                        take[u] = 0;
#pragma unroll
                        for (int j = 0; j < 8; ++j) {
                            const uint32_t key = (ws[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                            const bool in = ib + j < a.P;
                            take[u] |= static_cast<uint32_t>(in && key >= lim) << j;
                            if (count_lo && in && !((ub[u] >> j) & 1u) && (key >> HIST_SHIFT) == bsel)
                                atomicAdd(&lohist[key & LOW], 1u);
                        }
                        c += __popc(take[u]);
                    }
                    // one wavefront-aggregated block of slots for the whole step
                    uint32_t incl = c;
#pragma unroll
                    for (int off = 1; off < 64; off <<= 1) {
                        const uint32_t o = __shfl_up(incl, off, 64);
                        if (lane >= off) incl += o;
                    }
                    uint32_t base = 0;
                    if (lane == 63 && incl) base = atomicAdd(&s_count, incl);
                    base = __shfl(base, 63, 64) + incl - c;
#pragma unroll
                    for (int u = 0; u < CU; ++u) {
                        const int64_t ib = i0 + u * 8 * NT;
                        const uint32_t ws[4] = {w[u].x, w[u].y, w[u].z, w[u].w};
                        uint32_t t = take[u];
                        while (t) {
                            const int j = __ffs(static_cast<int>(t)) - 1;
                            t &= t - 1;
                            if (base < static_cast<uint32_t>(a.cap)) {
                                const uint32_t key = (ws[j >> 1] >> (16 * (j & 1))) & 0xffffu;
                                list[base] = Comp<C>::make(key, ib + j);
                                flags[base] = static_cast<uint8_t>((ub[u] >> j) & 1u);
                            }
                            ++base;
                        }
                    }
                }
            };
            collect(bsel << HIST_SHIFT, true);
            __syncthreads();
            if (wave == 0) topk_find_bin_n<(1 << HIST_SHIFT)>(lohist, need_lo, lane, &s_bin, &s_need);
            __syncthreads();
            const uint32_t L = (bsel << HIST_SHIFT) | s_bin;
            if (s_count > static_cast<uint32_t>(a.cap)) {
                // over the capacity: collect again from the bound itself
                __syncthreads();
                if (tid == 0) s_count = 0;
                __syncthreads();
                collect(L, false);
                __syncthreads();
            }
            const uint32_t cnt = s_count;
            exact_path = cnt > static_cast<uint32_t>(a.cap);
            if (!exact_path) {
                // exact keys of the uncertain entries that can reach the bound:
                // their slots are gathered first (in sel_f, free until the
                // winners are collected), so that a thread recomputes one row
                uint32_t* uslot = reinterpret_cast<uint32_t*>(sel_f);
                const uint32_t ucap = static_cast<uint32_t>(a.n2) * sizeof(C) / 4;
                if (tid == 0) s_total = 0;
                __syncthreads();
                for (uint32_t i0 = tid; i0 - lane < cnt; i0 += NT) {
                    const bool u = i0 < cnt && flags[i0] &&
                                   static_cast<uint32_t>(list[i0] >> Comp<C>::IDX_BITS) >= L;
                    const uint64_t m = __ballot(u);
                    uint32_t base = 0;
                    if (lane == 0 && m) base = atomicAdd(&s_total, static_cast<uint32_t>(__popcll(m)));
                    base = __shfl(base, 0, 64) + static_cast<uint32_t>(__popcll(m & ((1ull << lane) - 1ull)));
                    if (u && base < ucap) uslot[base] = i0;
                }
                __syncthreads();
                const uint32_t ucnt = s_total;
                if (ucnt <= ucap) {
                    for (uint32_t u = tid; u < ucnt; u += NT) {
                        const uint32_t i = uslot[u];
                        const int64_t idx = Comp<C>::index(list[i]);
                        list[i] = Comp<C>::make(exact_key_row(kbase + idx * a.ks_n, q, a.f16 != 0), idx);
                    }
                } else {
                    for (uint32_t i = tid; i < cnt; i += NT) {
                        if (!flags[i]) continue;
                        const C c = list[i];
                        if (static_cast<uint32_t>(c >> Comp<C>::IDX_BITS) < L) continue;
                        const int64_t idx = Comp<C>::index(c);
                        list[i] = Comp<C>::make(exact_key_row(kbase + idx * a.ks_n, q, a.f16 != 0), idx);
                    }
                }
                __syncthreads();
                // Ranks by counting, while every entry at or above L has a
                // key within TOPK_SPAN of L: each such entry is counted in
                // its key's bucket, a bucket's first rank is the number of
                // entries with larger keys, and inside a bucket the larger
                // composite (the lower index) comes first.  The entries ranked
                // below T are the winners, each written at its rank.
                {
                    uint32_t* bcnt = brk;                   // bucket counts (then fill counters)
                    uint32_t* bstart = brk + TOPK_SPAN;     // first rank of each bucket
                    for (int i = tid; i < TOPK_SPAN; i += NT) bcnt[i] = 0;
                    if (tid == 0) s_ovf = 0;
                    __syncthreads();
                    for (uint32_t i = tid; i < cnt; i += NT) {
                        const uint32_t key = static_cast<uint32_t>(list[i] >> Comp<C>::IDX_BITS);
                        if (key >= L) {
                            if (key - L < static_cast<uint32_t>(TOPK_SPAN)) atomicAdd(&bcnt[key - L], 1u);
                            else s_ovf = 1;
                        }
                    }
                    __syncthreads();
                    if (!s_ovf) {
                        // exclusive prefix over the buckets in descending key order
                        // (thread t: buckets SPAN - 1 - BPT t - u, u < BPT)
                        constexpr int BPT = TOPK_SPAN / NT;
                        uint32_t cu[BPT], sum = 0;
#pragma unroll
                        for (int u = 0; u < BPT; ++u) {
                            cu[u] = bcnt[TOPK_SPAN - 1 - BPT * tid - u];
                            sum += cu[u];
                        }
                        uint32_t incl = sum;
#pragma unroll
                        for (int off = 1; off < 64; off <<= 1) {
                            const uint32_t o = __shfl_up(incl, off, 64);
                            if (lane >= off) incl += o;
                        }
                        if (lane == 63) s_wtot[wave] = incl;
                        __syncthreads();
                        uint32_t excl = incl - sum;
                        for (int w = 0; w < wave; ++w) excl += s_wtot[w];
#pragma unroll
                        for (int u = 0; u < BPT; ++u) {
                            bstart[TOPK_SPAN - 1 - BPT * tid - u] = excl;
                            bcnt[TOPK_SPAN - 1 - BPT * tid - u] = 0;
                            excl += cu[u];
                        }
                        __syncthreads();
                        for (uint32_t i = tid; i < cnt; i += NT) {
                            const C c = list[i];
                            const uint32_t key = static_cast<uint32_t>(c >> Comp<C>::IDX_BITS);
                            if (key >= L) brank_tmp[bstart[key - L] + atomicAdd(&bcnt[key - L], 1u)] = c;
                        }
                        __syncthreads();
                        // the entries at or above L, bucket by bucket (the fill counters are the counts again)
                        const uint32_t tot = bstart[0] + bcnt[0];
                        for (uint32_t pos = tid; pos < tot; pos += NT) {
                            const C c = brank_tmp[pos];
                            const uint32_t off = static_cast<uint32_t>(c >> Comp<C>::IDX_BITS) - L;
                            const uint32_t s0 = bstart[off], n = bcnt[off];
                            if (s0 >= static_cast<uint32_t>(a.T)) continue;
                            uint32_t rin = 0;
                            for (uint32_t j = 0; j < n; ++j) rin += brank_tmp[s0 + j] > c;
                            if (s0 + rin < static_cast<uint32_t>(a.T)) orow[s0 + rin] = Comp<C>::index(c);
                        }
                        return;
                    }
                }
                // radix select of the T-th largest composite, a byte at a time
                C prefix = 0, pmask = 0;
                uint32_t need = static_cast<uint32_t>(a.T);
                for (int pass = 0; pass < NB; ++pass) {
                    const int shift = 8 * (NB - 1 - pass);
                    for (int i = tid; i < (NT / 128) * 256; i += NT) hist[i] = 0;
                    __syncthreads();
                    for (uint32_t i = tid; i < cnt; i += NT) {
                        const C c = list[i];
                        // (entries below L are not winners)
                        if ((c & pmask) == prefix && static_cast<uint32_t>(c >> Comp<C>::IDX_BITS) >= L)
                            atomicAdd(&hist[(wave >> 1) * 256 + static_cast<uint32_t>((c >> shift) & 0xffu)], 1u);
                    }
                    __syncthreads();
                    if (tid < 256) {
                        uint32_t sum = 0;
#pragma unroll
                        for (int w = 0; w < (NT / 128); ++w) sum += hist[w * 256 + tid];
                        hist[tid] = sum;
                    }
                    __syncthreads();
                    if (wave == 0) topk_find_bin(hist, need, lane, &s_bin, &s_need);
                    __syncthreads();
                    prefix |= static_cast<C>(s_bin) << shift;
                    pmask |= static_cast<C>(0xffu) << shift;
                    need = s_need;
                }
                // the T composites >= the T-th largest
                if (tid == 0) s_count = 0;
                __syncthreads();
                for (uint32_t i = tid; i < cnt; i += NT) {
                    const C c = list[i];
                    if (c >= prefix) {
                        const uint32_t slot = atomicAdd(&s_count, 1u);
                        if (slot < static_cast<uint32_t>(a.n2)) sel_f[slot] = c;
                    }
                }
                for (int i = a.T + tid; i < a.n2; i += NT) sel_f[i] = 0;   // real composites are > 0
                __syncthreads();
                topk_sort_out<C, NT>(sel_f, a.T, a.n2, a.T <= TOPK_RANK_LIMIT, orow);
                return;
            }
        }
    }
    // exact path: recompute the row's uncertain keys in place
    __syncthreads();                               // (s_q written)
    for (int64_t wi = tid; wi < a.UW; wi += NT) {
        uint32_t bits = ur[wi];
        while (bits) {
            const int j = __ffs(static_cast<int>(bits)) - 1;
            bits &= bits - 1;
            const int64_t p = wi * 32 + j;
            if (p < a.P) kr[p] = static_cast<uint16_t>(exact_key_row(kbase + p * a.ks_n, q, a.f16 != 0));
        }
    }
    __syncthreads();                               // the keys written above are visible to the workgroup
    C* sel = a.gsort ? static_cast<C*>(a.gsel) + static_cast<int64_t>(row) * a.n2 : list;
    topk_exact_row<C, NT>(kr, static_cast<const uint16_t*>(nullptr), a.P, a.T, a.n2,
                   !a.gsort && a.T <= TOPK_RANK_LIMIT, sel, hist, orow);
}

// Launch plan of topk_kernel for rows of P keys and T winners
struct TopkPlan {
    int n2, wide, gsort, fast, cap;
    size_t lds;
    size_t gbytes;               // global sort buffer bytes per row (gsort)
};
TopkPlan topk_plan(int64_t P, int T, size_t lds_budget) {
    TopkPlan t{};
    t.wide = P > TOPK_NARROW_P;
    const size_t cs = t.wide ? 8 : 4;
    if (T <= TOPK_RANK_LIMIT) {
        t.n2 = (T + 3) / 4 * 4;
    } else {
        t.n2 = 1;
        while (t.n2 < T) t.n2 <<= 1;
    }
    const size_t budget = std::min<size_t>(lds_budget, TOPK_LDS_MAX);
    const size_t hist = static_cast<size_t>(TOPK_HIST_AREA) * 4;
    const size_t sel = static_cast<size_t>(t.n2) * cs;
    t.gsort = hist + sel > budget;
    // candidate path: list (cap composites) + sel + uncertain flags (cap
    // bytes) + the counting rank's buckets and cap composites
    const size_t buckets = static_cast<size_t>(2 * TOPK_SPAN) * 4;
    if (hist + sel + buckets + 16 < budget) {
        const int64_t room = static_cast<int64_t>((budget - hist - sel - buckets - 16) / (2 * cs + 1)) / 16 * 16;
        // (about 34 KB at T ~ 800: four rows' workgroups share a CU)
        const int64_t want = std::min<int64_t>((std::max<int64_t>(2 * static_cast<int64_t>(T), 2048) + 15) / 16 * 16,
                                               (P + 15) / 16 * 16);
        t.cap = static_cast<int>(std::min<int64_t>({want, room, 65536}));
        t.fast = t.cap >= T;
    }
    t.lds = hist + (t.fast ? static_cast<size_t>(t.cap) * (2 * cs + 1) + 16 + buckets + sel
                           : (t.gsort ? 0 : sel));
    t.lds = (t.lds + 15) / 16 * 16;
    t.gbytes = t.gsort ? (sel + 255) / 256 * 256 : 0;
    return t;
}

// compute units of the current device (cached per device)
int device_cus() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    if (cache[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cache[dev] = v;
    }
    return cache[dev];
}

// LDS a topk workgroup may use on the current device (cached per device)
size_t topk_lds_budget() {
    static int cache[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 64 * 1024;
    if (cache[dev] == 0) {
        int v = 0;
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0)
            v = 64 * 1024;
        cache[dev] = v;
    }
    return static_cast<size_t>(cache[dev]) - 1024;   // room for the static LDS of the kernel
}

// ---------------------------------------------------------------------------
// freeze
// ---------------------------------------------------------------------------
// zero fill by a kernel (not hipMemsetAsync) so that the call can be captured
__global__ void zero_words_kernel(uint32_t* __restrict__ p, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0;
}

__global__ void mark_kernel(const int64_t* __restrict__ idx, int T, int64_t P, int64_t words, uint32_t* __restrict__ bits) {
    const int bh = blockIdx.y;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const int64_t p = idx[static_cast<int64_t>(bh) * T + t];
    if (p < 0 || p >= P) return;
    atomicOr(bits + bh * words + (p >> 5), 1u << (p & 31));
}

// One workgroup per row, rows of up to MARK_ROW_WORDS words: the row's bitmap
// is built in LDS and written whole (one launch in place of zero_words_kernel
// and mark_kernel).  Indices outside [0, P) are ignored, as in mark_kernel.
constexpr int MARK_ROW_WORDS = 8192;       // 32 KiB of LDS: P <= 262144
__global__ __launch_bounds__(1024) void mark_row_kernel(const int64_t* __restrict__ idx, int T, int64_t P, int64_t words,
                                                        uint32_t* __restrict__ bits) {
    __shared__ uint32_t s_w[MARK_ROW_WORDS];
    const int64_t bh = blockIdx.x;
    const int nw = static_cast<int>(words);    // <= MARK_ROW_WORDS (host)
    for (int i = threadIdx.x; i < nw; i += blockDim.x) s_w[i] = 0;
    __syncthreads();
    for (int t = threadIdx.x; t < T; t += blockDim.x) {
        const int64_t p = idx[bh * T + t];
        if (p >= 0 && p < P) atomicOr(&s_w[p >> 5], 1u << (p & 31));
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nw; i += blockDim.x) bits[bh * words + i] = s_w[i];
}

// prefix positions per workgroup: 16 KiB of K and V rows read per workgroup.
// Streams of this read:write mix ran faster the fewer bytes each workgroup
// covers, down to about 8 KiB; at 16 positions the per-workgroup set-up
// (the bitmap prefix count and two barriers) costs more than that gains
constexpr int CQ_CHUNK = 32;
constexpr int CQ_UNROLL = 2;                // tokens per 16-lane group per pass (one pass)

// 16 lanes quantise one bf16 (fp16 when f16) row of 128 channels: lane `sub`
// holds channels 8 sub .. 8 sub + 7 (`raw`).  All 16 lanes take part in the
// amax reduction; only the stores depend on `store`.
template <int NBITS, bool F16>
__device__ __forceinline__ void quant_row_group(uint4 raw, int8_t* dst, uint16_t* scl, int sub, bool store) {
    float v[8];
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = F16 ? f16_bits_to_f32(static_cast<uint16_t>(w[i])) : __uint_as_float(w[i] << 16);
        v[2 * i + 1] = F16 ? f16_bits_to_f32(static_cast<uint16_t>(w[i] >> 16)) : __uint_as_float(w[i] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = max16_dpp(amax);
    amax = fmaxf(amax, 1e-5f);
    _Float16 s16;
    uint32_t c[8];                                  // code i in the low NBITS bits
    quant_row_codes<NBITS>(v, amax, s16, c);
    if (!store) return;
    if (NBITS == 4) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= static_cast<uint32_t>(c[i] & 15) << (4 * i);
        reinterpret_cast<uint32_t*>(dst)[sub] = word;
    } else if (NBITS == 8) {
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            lo |= static_cast<uint32_t>(c[i] & 255) << (8 * i);
            hi |= static_cast<uint32_t>(c[i + 4] & 255) << (8 * i);
        }
        reinterpret_cast<uint2*>(dst)[sub] = make_uint2(lo, hi);
    } else {
        uint32_t half = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) half |= static_cast<uint32_t>(c[i] & 3) << (2 * i);
        reinterpret_cast<uint16_t*>(dst)[sub] = static_cast<uint16_t>(half);
    }
    if (sub == 0) *scl = __builtin_bit_cast(uint16_t, s16);
}

struct CompactArgs {
    const uint16_t* k; const uint16_t* v;
    int64_t ks_b, ks_h, ks_n, vs_b, vs_h, vs_n;
    int HK;
    int64_t P;                   // prefix length (N - W)
    int64_t n_compact;           // rows of the compact outputs (P - T)
    int64_t words;               // bitmap words per row
    const uint32_t* bits;
    int8_t* kp; int8_t* vp;      // [BH, P - T, D*bits/8]
    int64_t kp_bh, kp_n, vp_bh, vp_n;
    uint16_t* ksc; uint16_t* vsc;
    int64_t ksc_bh, vsc_bh;
    int k_bits, v_bits;
    int f16;                     // k / v are fp16 (else bf16)
};

// (the element type is a template parameter: chosen at run time inside the
// unrolled conversions, both conversions of every element were issued)
template <int KB, int VB, bool F16>
__global__ __launch_bounds__(256) void compact_quant_kernel(CompactArgs a) {
    __shared__ uint32_t s_base;
    __shared__ uint32_t s_wpre[CQ_CHUNK / 32 + 1];
    const int bh = blockIdx.y;
    const int b = bh / a.HK, hk = bh % a.HK;
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * CQ_CHUNK;
    const uint32_t* rb = a.bits + bh * a.words;
    const int64_t w0 = p0 >> 5;
    // selected positions before p0
    uint32_t cnt = 0;
    for (int64_t w = threadIdx.x; w < w0; w += blockDim.x) cnt += __popc(rb[w]);
    for (int m = 32; m >= 1; m >>= 1) cnt += __shfl_xor(cnt, m, 64);
    if (threadIdx.x == 0) s_base = 0;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) atomicAdd(&s_base, cnt);
    if (threadIdx.x == 0) {
        uint32_t run = 0;
        for (int i = 0; i < CQ_CHUNK / 32; ++i) {
            s_wpre[i] = run;
            const int64_t w = w0 + i;
            if (w < a.words) run += __popc(rb[w]);
        }
        s_wpre[CQ_CHUNK / 32] = run;
    }
    __syncthreads();
    const uint32_t base = s_base;
    // 16 lanes per token; each 16-lane group takes CQ_UNROLL tokens per pass
    // and issues their K and V row loads together (selected rows are loaded
    // too and simply not stored, which keeps the loads unconditional)
    const int sub = threadIdx.x & 15;
    const uint16_t* kbase = a.k + b * a.ks_b + hk * a.ks_h + sub * 8;
    const uint16_t* vbase = a.v + b * a.vs_b + hk * a.vs_h + sub * 8;
    for (int j0 = threadIdx.x >> 4; j0 < CQ_CHUNK; j0 += 16 * CQ_UNROLL) {
        uint4 kr[CQ_UNROLL], vr[CQ_UNROLL];
        int64_t pp[CQ_UNROLL];
#pragma unroll
        for (int u = 0; u < CQ_UNROLL; ++u) {
            const int64_t p = p0 + j0 + 16 * u;
            pp[u] = p;
            const int64_t pc = p < a.P ? p : a.P - 1;
            // default cache policy: with non-temporal loads here the gather of
            // the top-k and window rows that follows ran 1.7x slower
            kr[u] = *reinterpret_cast<const uint4*>(kbase + pc * a.ks_n);
            vr[u] = *reinterpret_cast<const uint4*>(vbase + pc * a.vs_n);
        }
#pragma unroll
        for (int u = 0; u < CQ_UNROLL; ++u) {
            const int64_t p = pp[u];
            const int j = j0 + 16 * u;
            const uint32_t word = p < a.P ? rb[p >> 5] : 1u << (p & 31);
            const uint32_t below = __popc(word & ((1u << (p & 31)) - 1u));
            const int64_t slot = p - (base + s_wpre[j >> 5] + below);
            // selected rows stay bf16 in k/v_topk; the slot bound holds when the
            // indices are distinct and in range, and keeps every store inside
            // the n_compact rows of the outputs when they are not
            const bool keep = p < a.P && !((word >> (p & 31)) & 1u) && slot < a.n_compact;
            const int64_t dst = keep ? slot : 0;
            quant_row_group<KB, F16>(kr[u], a.kp + bh * a.kp_bh + dst * a.kp_n, a.ksc + bh * a.ksc_bh + dst, sub, keep);
            quant_row_group<VB, F16>(vr[u], a.vp + bh * a.vp_bh + dst * a.vp_n, a.vsc + bh * a.vsc_bh + dst, sub, keep);
        }
    }
}

// copies rows: for r < T the top-k rows (score order), else the window rows
struct GatherArgs {
    const uint16_t* k; const uint16_t* v;
    int64_t ks_b, ks_h, ks_n, vs_b, vs_h, vs_n;
    int HK;
    const int64_t* idx; int T;
    int64_t win0; int W;
    uint16_t* kt; uint16_t* vt; int64_t kt_bh, kt_n, vt_bh, vt_n;
    uint16_t* kw; uint16_t* vw; int64_t kw_bh, kw_n, vw_bh, vw_n;
};

__global__ __launch_bounds__(256) void gather_rows_kernel(GatherArgs a) {
    const int bh = blockIdx.y;
    const int b = bh / a.HK, hk = bh % a.HK;
    const int r = blockIdx.x * 16 + (threadIdx.x >> 4);      // 16 lanes x 16 bytes = one row
    const int sub = threadIdx.x & 15;
    if (r >= a.T + a.W) return;
    int64_t src;
    uint16_t *dk, *dv;
    if (r < a.T) {
        src = a.idx[static_cast<int64_t>(bh) * a.T + r];
        dk = a.kt + bh * a.kt_bh + r * a.kt_n;
        dv = a.vt + bh * a.vt_bh + r * a.vt_n;
    } else {
        src = a.win0 + (r - a.T);
        dk = a.kw + bh * a.kw_bh + (r - a.T) * a.kw_n;
        dv = a.vw + bh * a.vw_bh + (r - a.T) * a.vw_n;
    }
    uint4 kr = make_uint4(0u, 0u, 0u, 0u), vr = kr;
    if (r >= a.T || (src >= 0 && src < a.win0)) {  // a top-k index outside [0, P) gives a zero row
        kr = reinterpret_cast<const uint4*>(a.k + b * a.ks_b + hk * a.ks_h + src * a.ks_n)[sub];
        vr = reinterpret_cast<const uint4*>(a.v + b * a.vs_b + hk * a.vs_h + src * a.vs_n)[sub];
    }
    reinterpret_cast<uint4*>(dk)[sub] = kr;
    reinterpret_cast<uint4*>(dv)[sub] = vr;
}

int padded_heads(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 16; }

// workspace: [query means, float64][query means, bf16 bits][keys per row]
// [uncertain bitmaps][certified-key histograms][global sort buffers (large top-k only)]
struct SelectLayout {
    size_t qm, qb, keys, unc, hist, gsel, total;
};
SelectLayout select_layout(int B, int H_out, int64_t P, int T, const TopkPlan& tp) {
    auto up = [](size_t x) { return (x + 255) / 256 * 256; };
    const size_t rows = static_cast<size_t>(B) * H_out;
    SelectLayout L;
    L.qm = 0;
    L.qb = up(rows * 128 * sizeof(double) * 4);    // room for head padding
    L.keys = L.qb + up(rows * 128 * 2 * 4);
    L.unc = L.keys + up(rows * key_pitch(P) * 2);
    L.hist = L.unc + up(rows * unc_words(P) * 4);
    L.gsel = L.hist + up(rows * HIST_BINS * 4);
    L.total = L.gsel + (tp.gsort ? rows * tp.gbytes : 0);
    (void)T;
    return L;
}

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" size_t hyq_vertical_select_workspace_size(int32_t b, int32_t h_out, int64_t p, int32_t top_k) {
    if (b < 0 || h_out < 0 || p < 0 || top_k < 0 || p > TOPK_MAX_P || top_k > TOPK_MAX_T) return 0;
    const TopkPlan tp = topk_plan(p, top_k, topk_lds_budget());
    return select_layout(b, h_out, p, top_k, tp).total;
}

extern "C" int hyq_vertical_select(const uint16_t* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, int32_t q_len,
                                   int32_t hq_in, int32_t group, const uint16_t* k, int64_t ks_b, int64_t ks_h,
                                   int64_t ks_n, int32_t hk, int64_t p, int32_t b, int32_t d, int32_t tail,
                                   int32_t top_k, int32_t is_fp16, int64_t* out_idx, void* workspace, size_t ws_bytes,
                                   void* stream) {
    if (d != 128) return fail(HYQ_ENOTSUP, "hyq_vertical_select: head_dim must be 128");
    if (is_fp16 != 0 && is_fp16 != 1) return fail(HYQ_EINVAL, "hyq_vertical_select: is_fp16 must be 0 or 1");
    if (b < 0 || hq_in <= 0 || hk <= 0 || group <= 0 || hq_in % group) return fail(HYQ_EINVAL, "hyq_vertical_select: bad head counts");
    const int h_out = hq_in / group;
    if (h_out % hk) return fail(HYQ_EINVAL, "hyq_vertical_select: output heads must be a multiple of key heads");
    const int G = h_out / hk;
    if (G > 16) return fail(HYQ_ENOTSUP, "hyq_vertical_select: more than 16 query heads per key head");
    if (p <= 0 || top_k <= 0 || b == 0) return HYQ_OK;
    if (top_k > p) return fail(HYQ_EINVAL, "hyq_vertical_select: top_k > prefix length");
    if (p > TOPK_MAX_P) return fail(HYQ_ENOTSUP, "hyq_vertical_select: prefix longer than 2^31 - 1");
    if (top_k > TOPK_MAX_T) return fail(HYQ_ENOTSUP, "hyq_vertical_select: top_k above 2^30");
    if (tail <= 0 || tail > q_len) return fail(HYQ_EINVAL, "hyq_vertical_select: bad query tail");
    if (!q || !k || !out_idx) return fail(HYQ_EINVAL, "hyq_vertical_select: null pointer");
    if (!aligned(k, 16) || ks_n % 8 || ks_h % 8 || ks_b % 8) return fail(HYQ_EINVAL, "hyq_vertical_select: keys must be 16-byte aligned rows");
    if (ks_n < 128 || ks_n > (1 << 20)) return fail(HYQ_ENOTSUP, "hyq_vertical_select: key row stride must be in [128, 2^20] elements");
    if (!aligned(q, 4) || qs_t % 2 || qs_h % 2 || qs_b % 2) return fail(HYQ_EINVAL, "hyq_vertical_select: query rows must be 4-byte aligned");
    const TopkPlan tp = topk_plan(p, top_k, topk_lds_budget());
    const SelectLayout L = select_layout(b, h_out, p, top_k, tp);
    if (!workspace || ws_bytes < L.total || !aligned(workspace, 16))
        return fail(HYQ_ENOSPC, "hyq_vertical_select: workspace too small or not 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    char* ws = static_cast<char*>(workspace);
    double* qm = reinterpret_cast<double*>(ws + L.qm);
    uint16_t* qb = reinterpret_cast<uint16_t*>(ws + L.qb);
    uint16_t* keys = reinterpret_cast<uint16_t*>(ws + L.keys);
    uint32_t* unc = reinterpret_cast<uint32_t*>(ws + L.unc);
    uint32_t* hist = reinterpret_cast<uint32_t*>(ws + L.hist);
    void* gsel = ws + L.gsel;
    const int GP = padded_heads(G);
    if (aligned(q, 16) && qs_t % 8 == 0 && qs_h % 8 == 0 && qs_b % 8 == 0) {
        auto mean16 = [&](auto f16) {
            constexpr bool F = decltype(f16)::value;
            if (group == 1)
                qmean16_kernel<256, F><<<dim3(static_cast<unsigned>(b * hk * GP)), dim3(256), 0, s>>>(
                    q, qs_b, qs_h, qs_t, q_len, tail, group, hk, G, GP, qm, qb, hist);
            else
                qmean16_kernel<1024, F><<<dim3(static_cast<unsigned>(b * hk * GP)), dim3(1024), 0, s>>>(
                    q, qs_b, qs_h, qs_t, q_len, tail, group, hk, G, GP, qm, qb, hist);
        };
        if (is_fp16) mean16(std::true_type{});
        else mean16(std::false_type{});
    } else
        qmean_kernel<<<dim3(static_cast<unsigned>(b * hk * GP)), dim3(QM_THREADS), 0, s>>>(
            q, qs_b, qs_h, qs_t, q_len, tail, group, hk, G, GP, is_fp16, qm, qb, hist);
    int rc = check_launch("hyq_vertical_select (mean)");
    if (rc) return rc;
    const int64_t KP = key_pitch(p);
    // bf16 models: scores on the matrix cores with certified keys; fp16
    // models: float64 scores (exact keys)
    auto score_f64 = [&](auto gm) {
        const dim3 grid(static_cast<unsigned>((p + SC_WG_ROWS - 1) / SC_WG_ROWS), static_cast<unsigned>(b * hk));
        score_kernel<decltype(gm)::value, true><<<grid, dim3(256), 0, s>>>(
            k, ks_b, ks_h, ks_n, hk, G, p, KP, qm, keys, unc, hist);
    };
    auto score_mfma = [&](auto gm) {
        const dim3 grid(static_cast<unsigned>((p + SM_WG_ROWS - 1) / SM_WG_ROWS), static_cast<unsigned>(b * hk));
        score_mfma_kernel<decltype(gm)::value><<<grid, dim3(256), 0, s>>>(
            k, ks_b, ks_h, ks_n, hk, G, p, KP, qm, qb, keys, unc, hist);
    };
    auto score_gm = [&](auto fn) {
        switch (GP) {
            case 1: fn(std::integral_constant<int, 1>{}); break;
            case 2: fn(std::integral_constant<int, 2>{}); break;
            case 4: fn(std::integral_constant<int, 4>{}); break;
            case 8: fn(std::integral_constant<int, 8>{}); break;
            default: fn(std::integral_constant<int, 16>{}); break;
        }
    };
    if (is_fp16) score_gm(score_f64);
    else score_gm(score_mfma);
    rc = check_launch("hyq_vertical_select (score)");
    if (rc) return rc;
    TopkArgs ta{keys, unc, hist, p, KP, unc_words(p), top_k, tp.n2, tp.cap, tp.fast, tp.gsort, gsel,
                k, ks_b, ks_h, ks_n, hk, G, GP, is_fp16, qm, out_idx};
    // 256-thread workgroups (four rows per CU) when the rows are many, 512
    // (a row's phases shorter) when a CU has at most a row or two
    const dim3 tgrid(static_cast<unsigned>(b * h_out));
    const bool many = static_cast<int64_t>(b) * h_out >= 2 * static_cast<int64_t>(device_cus());
    if (tp.wide) {
        if (many) topk_kernel<uint64_t, 256><<<tgrid, dim3(256), tp.lds, s>>>(ta);
        else topk_kernel<uint64_t, 512><<<tgrid, dim3(512), tp.lds, s>>>(ta);
    } else {
        if (many) topk_kernel<uint32_t, 256><<<tgrid, dim3(256), tp.lds, s>>>(ta);
        else topk_kernel<uint32_t, 512><<<tgrid, dim3(512), tp.lds, s>>>(ta);
    }
    return check_launch("hyq_vertical_select (topk)");
}

extern "C" size_t hyq_freeze_workspace_size(int32_t bh, int64_t p) {
    if (bh < 0 || p < 0) return 0;
    return static_cast<size_t>(bh) * ((p + 31) / 32) * 4 + 256;
}

extern "C" int hyq_freeze_reorganise(const uint16_t* k, int64_t ks_b, int64_t ks_h, int64_t ks_n,
                                     const uint16_t* v, int64_t vs_b, int64_t vs_h, int64_t vs_n,
                                     int32_t b, int32_t hk, int64_t n, int32_t d, int32_t w,
                                     const int64_t* topk_idx, int32_t top_k, int32_t k_bits, int32_t v_bits,
                                     int32_t is_fp16, int8_t* kp, int64_t kp_bh, int64_t kp_n, int8_t* vp, int64_t vp_bh, int64_t vp_n,
                                     uint16_t* ksc, int64_t ksc_bh, uint16_t* vsc, int64_t vsc_bh,
                                     uint16_t* kt, int64_t kt_bh, int64_t kt_n, uint16_t* vt, int64_t vt_bh, int64_t vt_n,
                                     uint16_t* kw, int64_t kw_bh, int64_t kw_n, uint16_t* vw, int64_t vw_bh, int64_t vw_n,
                                     void* workspace, size_t ws_bytes, void* stream) {
    if (d != 128) return fail(HYQ_ENOTSUP, "hyq_freeze_reorganise: head_dim must be 128");
    auto okbits = [](int x) { return x == 2 || x == 4 || x == 8; };
    if (!okbits(k_bits) || !okbits(v_bits)) return fail(HYQ_EINVAL, "hyq_freeze_reorganise: bits must be 2, 4 or 8");
    if (is_fp16 != 0 && is_fp16 != 1) return fail(HYQ_EINVAL, "hyq_freeze_reorganise: is_fp16 must be 0 or 1");
    if (b < 0 || hk <= 0 || n < 0 || w < 0 || w > n || top_k < 0) return fail(HYQ_EINVAL, "hyq_freeze_reorganise: bad shape");
    const int64_t P = n - w;
    if (top_k > P) return fail(HYQ_EINVAL, "hyq_freeze_reorganise: top_k > prefix length");
    const int bh = b * hk;
    if (bh == 0) return HYQ_OK;
    if (!aligned(k, 16) || !aligned(v, 16) || ks_n % 8 || vs_n % 8 || ks_h % 8 || vs_h % 8 || ks_b % 8 || vs_b % 8)
        return fail(HYQ_EINVAL, "hyq_freeze_reorganise: keys/values must be 16-byte aligned rows");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const int64_t words = (P + 31) / 32;
    if (P - top_k > 0) {
        if (!workspace || ws_bytes < static_cast<size_t>(bh) * words * 4)
            return fail(HYQ_ENOSPC, "hyq_freeze_reorganise: workspace too small");
        uint32_t* bits = static_cast<uint32_t*>(workspace);
        const int64_t nw = static_cast<int64_t>(bh) * words;
        if (words <= MARK_ROW_WORDS) {
            mark_row_kernel<<<dim3(static_cast<unsigned>(bh)), dim3(1024), 0, s>>>(topk_idx, top_k, P, words, bits);
            if (int rc0 = check_launch("hyq_freeze_reorganise (mark)")) return rc0;
        } else {
            zero_words_kernel<<<dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, s>>>(bits, nw);
            if (int rc0 = check_launch("hyq_freeze_reorganise (zero)")) return rc0;
            if (top_k > 0) {
                mark_kernel<<<dim3(static_cast<unsigned>((top_k + 255) / 256), static_cast<unsigned>(bh)), dim3(256), 0, s>>>(
                    topk_idx, top_k, P, words, bits);
                int rc = check_launch("hyq_freeze_reorganise (mark)");
                if (rc) return rc;
            }
        }
        CompactArgs a{k, v, ks_b, ks_h, ks_n, vs_b, vs_h, vs_n, hk, P, P - top_k, words, bits,
                      kp, vp, kp_bh, kp_n, vp_bh, vp_n, ksc, vsc, ksc_bh, vsc_bh, k_bits, v_bits, is_fp16};
        dim3 grid(static_cast<unsigned>((P + CQ_CHUNK - 1) / CQ_CHUNK), static_cast<unsigned>(bh));
        auto launch = [&](auto f16) {
            constexpr bool F = decltype(f16)::value;
            switch (10 * k_bits + v_bits) {
                case 44: compact_quant_kernel<4, 4, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 42: compact_quant_kernel<4, 2, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 48: compact_quant_kernel<4, 8, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 24: compact_quant_kernel<2, 4, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 22: compact_quant_kernel<2, 2, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 28: compact_quant_kernel<2, 8, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 84: compact_quant_kernel<8, 4, F><<<grid, dim3(256), 0, s>>>(a); break;
                case 82: compact_quant_kernel<8, 2, F><<<grid, dim3(256), 0, s>>>(a); break;
                default: compact_quant_kernel<8, 8, F><<<grid, dim3(256), 0, s>>>(a); break;
            }
        };
        if (is_fp16) launch(std::true_type{});
        else launch(std::false_type{});
        int rc = check_launch("hyq_freeze_reorganise (compact)");
        if (rc) return rc;
    }
    if (top_k + w > 0) {
        GatherArgs g{k, v, ks_b, ks_h, ks_n, vs_b, vs_h, vs_n, hk, topk_idx, top_k, P, w,
                     kt, vt, kt_bh, kt_n, vt_bh, vt_n, kw, vw, kw_bh, kw_n, vw_bh, vw_n};
        gather_rows_kernel<<<dim3(static_cast<unsigned>((top_k + w + 15) / 16), static_cast<unsigned>(bh)), dim3(256), 0, s>>>(g);
        return check_launch("hyq_freeze_reorganise (gather)");
    }
    return HYQ_OK;
}
