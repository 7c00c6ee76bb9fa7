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
//   top-T       = the T largest scores, ties broken by the lower index, returned
//                 in (score desc, index asc) order (BASELINE's tie rule for the
//                 unspecified order of torch.topk, src/patch/_common.py:189).
// Kernels:
//   qmean_kernel      one thread per (b, ho, d).
//   score_kernel      one thread per key row, G output heads sharing the row
//                     (GQA-native, the K prefix is read once); writes the
//                     monotone 16-bit key of each bf16 score.
//   topk_kernel       one workgroup per (b, ho) row: 4-pass radix select on the
//                     unique composite (key << 16) | (0xffff - idx) (so "score
//                     desc, index asc" is just "composite desc"), gather of the
//                     T survivors into LDS, bitonic sort.
//   mark_kernel / compact_quant_kernel / gather_rows_kernel  the freeze: a
//                     bitmap of selected prefix positions, quantisation of the
//                     unselected prefix rows straight into their compact slots
//                     (ascending position, F6), and the bf16 copies of the
//                     top-k rows (score order, F5) and of the window.
#include "hyq_common.h"

#include <algorithm>
#include <string>

namespace hyq {
namespace {

constexpr int TOPK_THREADS = 1024;
constexpr int TOPK_MAX_T = 8192;           // bitonic sort buffer in LDS
constexpr int64_t TOPK_MAX_P = 65536;      // 16-bit index in the composite


__device__ __forceinline__ double bf16_bits_to_f64(uint16_t b) { return static_cast<double>(bf16_to_f32(b)); }

// monotone key of a bf16 value (-0 and +0 share a key)
__device__ __forceinline__ uint32_t orderable_key(uint16_t b) {
    uint32_t u = b;
    if (u == 0x8000u) u = 0;
    return (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
}

// qm as float64 (the exact value of the bf16 mean) for the score kernel
// one thread per (b, hk, g < GP, d); heads g >= G (padding) get zeros
__global__ __launch_bounds__(128) void qmean_kernel(const uint16_t* __restrict__ q, int64_t qs_b, int64_t qs_h,
                                                    int64_t qs_t, int QL, int tail, int R, int HK, int G, int GP,
                                                    int D, int B, double* __restrict__ qm) {
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t total = static_cast<int64_t>(B) * HK * GP * D;
    if (idx >= total) return;
    const int d = static_cast<int>(idx % D);
    const int g = static_cast<int>((idx / D) % GP);
    const int bhk = static_cast<int>(idx / (static_cast<int64_t>(D) * GP));
    if (g >= G) {
        qm[idx] = 0.0;
        return;
    }
    const int b = bhk / HK, ho = (bhk % HK) * G + g;
    const uint16_t* base = q + b * qs_b + static_cast<int64_t>(ho * R) * qs_h + static_cast<int64_t>(QL - tail) * qs_t + d;
    // every partial sum below is a sum of bf16 values (or of bf16 means),
    // exact in float64, so the association order does not change the result
    double outer[4] = {0.0, 0.0, 0.0, 0.0};
    int t = 0;
    if (R == 1) {
        for (; t + 8 <= tail; t += 8) {
            uint16_t v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) v[u] = base[static_cast<int64_t>(t + u) * qs_t];
#pragma unroll
            for (int u = 0; u < 8; ++u) outer[u & 3] += bf16_bits_to_f64(v[u]);
        }
        for (; t < tail; ++t) outer[0] += bf16_bits_to_f64(base[static_cast<int64_t>(t) * qs_t]);
    } else {
        for (; t < tail; ++t) {
            double inner = 0.0;
            for (int r = 0; r < R; ++r) inner += bf16_bits_to_f64(base[static_cast<int64_t>(r) * qs_h + static_cast<int64_t>(t) * qs_t]);
            outer[t & 3] += bf16_bits_to_f64(f64_to_bf16_rne(inner / R));
        }
    }
    const double s = (outer[0] + outer[1]) + (outer[2] + outer[3]);
    qm[idx] = bf16_bits_to_f64(f64_to_bf16_rne(s / tail));
}

// One workgroup per 256 key rows of one (b, hk).  The query means (float64,
// [GM][128]) sit in LDS and are read with same-address (broadcast) loads.
// Each wavefront stages half-rows (64 channels) of its 64 rows through LDS
// with coalesced 1 KB loads (pitch 144 B: the per-row reads hit every bank
// once per 16 lanes), then lane r accumulates the GM dot products of row r
// sequentially in channel order in float64.  GM is G rounded up to 1, 2, 4,
// 8 or 16; the means are stored with zero rows past G, so the FMA loop has no
// branches and only the key store skips heads g >= G.
constexpr int SC_ROWS = 64;                 // rows per wavefront
constexpr int SC_PITCH = 144;               // LDS bytes per half-row (128 + 16)

template <int GM>
__global__ __launch_bounds__(256) void score_kernel(const uint16_t* __restrict__ k, int64_t ks_b, int64_t ks_h,
                                                    int64_t ks_n, int HK, int G, int64_t P,
                                                    const double* __restrict__ qm, uint16_t* __restrict__ keys) {
    __shared__ __align__(16) double s_q[GM * 128];
    __shared__ __align__(16) uint8_t s_rows[4][SC_ROWS * SC_PITCH];
    const int bh = blockIdx.y;                     // b * HK + hk
    const int b = bh / HK, hk = bh % HK;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const double* qg = qm + static_cast<int64_t>(bh) * GM * 128;
    for (int i = threadIdx.x; i < GM * 128; i += 256) s_q[i] = qg[i];
    const int64_t p0 = static_cast<int64_t>(blockIdx.x) * 256 + wave * SC_ROWS;
    const uint16_t* kb = k + b * ks_b + hk * ks_h;
    uint8_t* lds = s_rows[wave];
    // lane l loads 16-byte chunk (l & 7) of half-row `half` of rows p0 + 8i + (l >> 3)
    const int sub = lane & 7, rq = lane >> 3;
    double acc[GM];
#pragma unroll
    for (int g = 0; g < GM; ++g) acc[g] = 0.0;
    __syncthreads();
#pragma unroll 1
    for (int half = 0; half < 2; ++half) {
        uint4 raw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int64_t p = min(p0 + 8 * i + rq, P - 1);
            raw[i] = *reinterpret_cast<const uint4*>(kb + p * ks_n + 64 * half + 8 * sub);
        }
        // One wavefront writes and reads its own LDS rows; its LDS accesses
        // execute in program order, so the writes of this half follow every
        // read of the previous one and precede the reads below.
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < 8; ++i) *reinterpret_cast<uint4*>(lds + (8 * i + rq) * SC_PITCH + 16 * sub) = raw[i];
        __builtin_amdgcn_wave_barrier();
        const uint8_t* row = lds + lane * SC_PITCH;
#pragma unroll 1
        for (int c = 0; c < 8; ++c) {
            const uint4 w = *reinterpret_cast<const uint4*>(row + 16 * c);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
            double kv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j)
                kv[j] = static_cast<double>(__uint_as_float(j & 1 ? ww[j >> 1] & 0xffff0000u : ww[j >> 1] << 16));
            const int d0 = 64 * half + 8 * c;
#pragma unroll
            for (int g = 0; g < GM; ++g) {
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[g] = fma(s_q[g * 128 + d0 + j], kv[j], acc[g]);
            }
        }
    }
    const int64_t p = p0 + lane;
    if (p < P) {
#pragma unroll
        for (int g = 0; g < GM; ++g)
            if (g < G) keys[(static_cast<int64_t>(bh) * G + g) * P + p] = static_cast<uint16_t>(orderable_key(f64_to_bf16_rne(acc[g])));
    }
}

constexpr int TOPK_WAVES = TOPK_THREADS / 64;
constexpr int64_t TOPK_LDS_KEYS = 24576;   // rows up to this many keys are cached in LDS

// One workgroup per (b, ho) row.  The composite (key << 16) | (0xffff - idx)
// is unique per position and orders "score desc, index asc" as "composite
// desc": a 4-pass radix select (8 bits per pass, one private histogram per
// wavefront) finds the T-th largest composite, the T survivors are gathered
// into LDS and bitonic-sorted.  Rows of up to TOPK_LDS_KEYS keys are read
// from memory once into LDS.
__global__ __launch_bounds__(TOPK_THREADS) void topk_kernel(const uint16_t* __restrict__ keys, int64_t P, int T,
                                                            int64_t* __restrict__ out) {
    __shared__ uint32_t hist[TOPK_WAVES][256];
    __shared__ uint32_t s_prefix, s_need;
    __shared__ uint32_t s_count;
    __shared__ uint32_t sel[TOPK_MAX_T];
    __shared__ uint16_t s_keys[TOPK_LDS_KEYS];
    const int row = blockIdx.x;
    const uint16_t* kr = keys + static_cast<int64_t>(row) * P;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const bool cached = P <= TOPK_LDS_KEYS;
    if (cached) {
        for (int64_t i = tid; i < P; i += TOPK_THREADS) s_keys[i] = kr[i];
    }
    if (tid == 0) {
        s_prefix = 0;
        s_need = static_cast<uint32_t>(T);
        s_count = 0;
    }
    auto key_at = [&](int64_t i) -> uint32_t { return cached ? s_keys[i] : kr[i]; };
    // radix select, most significant byte first: find the T-th largest composite
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < TOPK_WAVES * 256; i += TOPK_THREADS) (&hist[0][0])[i] = 0;
        __syncthreads();
        const uint32_t prefix = s_prefix;
        const uint32_t pmask = pass == 0 ? 0u : (0xffffffffu << (32 - 8 * pass));
        for (int64_t i = tid; i < P; i += TOPK_THREADS) {
            const uint32_t comp = (key_at(i) << 16) | (0xffffu - static_cast<uint32_t>(i));
            if ((comp & pmask) == prefix) atomicAdd(&hist[wave][(comp >> shift) & 0xffu], 1u);
        }
        __syncthreads();
        // fold the per-wavefront histograms into hist[0]
        if (tid < 256) {
            uint32_t s = 0;
#pragma unroll
            for (int w = 0; w < TOPK_WAVES; ++w) s += hist[w][tid];
            hist[0][tid] = s;
        }
        __syncthreads();
        if (tid < 64) {
            // wavefront 0: find the bin holding the need-th largest, from the top
            const uint32_t need = s_need;
            uint32_t c[4];
            uint32_t mine = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[j] = hist[0][255 - (4 * tid + j)];
                mine += c[j];
            }
            // exclusive prefix over lanes (bins from the top)
            uint32_t incl = mine;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = __shfl_up(incl, off, 64);
                if (tid >= off) incl += o;
            }
            uint32_t acc = incl - mine;
            int found = -1;
            uint32_t before = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (found < 0 && acc + c[j] >= need) {
                    found = 255 - (4 * tid + j);
                    before = acc;
                }
                acc += c[j];
            }
            // the first lane (highest bins) that found it wins; the candidates
            // always number at least `need`, so some lane finds it (were it
            // not so, bin 0 would be taken, as a top-down scan would)
            const uint64_t ball = __ballot(found >= 0);
            const int first = ball ? __ffsll(static_cast<long long>(ball)) - 1 : 63;
            if (tid == first) {
                if (found < 0) {
                    found = 0;
                    before = acc - c[3];
                }
                s_need = need - before;
                s_prefix = prefix | (static_cast<uint32_t>(found) << shift);
            }
        }
        __syncthreads();
    }
    const uint32_t thr = s_prefix;                 // exactly T composites are >= thr
    for (int64_t i = tid; i < P; i += TOPK_THREADS) {
        const uint32_t comp = (key_at(i) << 16) | (0xffffu - static_cast<uint32_t>(i));
        if (comp >= thr) {
            const uint32_t pos = atomicAdd(&s_count, 1u);
            if (pos < static_cast<uint32_t>(T)) sel[pos] = comp;
        }
    }
    __syncthreads();
    int n2 = 1;
    while (n2 < T) n2 <<= 1;
    for (int i = T + tid; i < n2; i += TOPK_THREADS) sel[i] = 0;   // real composites are > 0
    __syncthreads();
    // bitonic sort, descending
    for (int size = 2; size <= n2; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < n2 / 2; i += TOPK_THREADS) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const uint32_t a = sel[lo], bb = sel[hi];
                if ((a < bb) == desc) {
                    sel[lo] = bb;
                    sel[hi] = a;
                }
            }
            __syncthreads();
        }
    }
    for (int i = tid; i < T; i += TOPK_THREADS)
        out[static_cast<int64_t>(row) * T + i] = static_cast<int64_t>(0xffffu - (sel[i] & 0xffffu));
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

constexpr int CQ_CHUNK = 256;               // prefix positions per workgroup

template <int NBITS>
__device__ __forceinline__ void quant_row_group(const uint16_t* src, int8_t* dst, uint16_t* scl, int sub) {
    constexpr int QMAX = (1 << (NBITS - 1)) - 1;
    constexpr int QMIN = -(1 << (NBITS - 1));
    const uint4 raw = *reinterpret_cast<const uint4*>(src + sub * 8);
    float v[8];
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 64));
    amax = fmaxf(amax, 1e-5f);
    const float s32 = amax / static_cast<float>(QMAX);
    const _Float16 s16 = static_cast<_Float16>(s32);
    const float sf = static_cast<float>(s16);
    int c[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float r = rintf(v[i] / sf);
        r = fminf(fmaxf(r, static_cast<float>(QMIN)), static_cast<float>(QMAX));
        c[i] = static_cast<int>(r);
    }
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
    int64_t words;               // bitmap words per row
    const uint32_t* bits;
    int8_t* kp; int8_t* vp;      // [BH, P - T, D*bits/8]
    int64_t kp_bh, kp_n, vp_bh, vp_n;
    uint16_t* ksc; uint16_t* vsc;
    int64_t ksc_bh, vsc_bh;
    int k_bits, v_bits;
};

template <int KB, int VB>
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
    // 16 lanes per token, 16 tokens per pass
    const int sub = threadIdx.x & 15;
    for (int j = threadIdx.x >> 4; j < CQ_CHUNK; j += 16) {
        const int64_t p = p0 + j;
        if (p >= a.P) break;
        const uint32_t word = rb[p >> 5];
        if ((word >> (p & 31)) & 1u) continue;   // selected: stays bf16 in k/v_topk
        const uint32_t below = __popc(word & ((1u << (p & 31)) - 1u));
        const int64_t dst = p - (base + s_wpre[j >> 5] + below);
        quant_row_group<KB>(a.k + b * a.ks_b + hk * a.ks_h + p * a.ks_n,
                            a.kp + bh * a.kp_bh + dst * a.kp_n, a.ksc + bh * a.ksc_bh + dst, sub);
        quant_row_group<VB>(a.v + b * a.vs_b + hk * a.vs_h + p * a.vs_n,
                            a.vp + bh * a.vp_bh + dst * a.vp_n, a.vsc + bh * a.vsc_bh + dst, sub);
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
    reinterpret_cast<uint4*>(dk)[sub] = reinterpret_cast<const uint4*>(a.k + b * a.ks_b + hk * a.ks_h + src * a.ks_n)[sub];
    reinterpret_cast<uint4*>(dv)[sub] = reinterpret_cast<const uint4*>(a.v + b * a.vs_b + hk * a.vs_h + src * a.vs_n)[sub];
}

int padded_heads(int G) { return G <= 1 ? 1 : G <= 2 ? 2 : G <= 4 ? 4 : G <= 8 ? 8 : 16; }

size_t select_ws(int B, int H_out, int64_t P) {
    const size_t qm = static_cast<size_t>(B) * H_out * 128 * sizeof(double) * 4;   // room for head padding
    return ((qm + 255) / 256) * 256 + static_cast<size_t>(B) * H_out * P * 2;
}

}  // namespace
}  // namespace hyq

using namespace hyq;

extern "C" size_t hyq_vertical_select_workspace_size(int32_t b, int32_t h_out, int64_t p) {
    if (b < 0 || h_out < 0 || p < 0) return 0;
    return select_ws(b, h_out, p);
}

extern "C" int hyq_vertical_select(const uint16_t* q, int64_t qs_b, int64_t qs_h, int64_t qs_t, int32_t q_len,
                                   int32_t hq_in, int32_t group, const uint16_t* k, int64_t ks_b, int64_t ks_h,
                                   int64_t ks_n, int32_t hk, int64_t p, int32_t b, int32_t d, int32_t tail,
                                   int32_t top_k, int64_t* out_idx, void* workspace, size_t ws_bytes, void* stream) {
    if (d != 128) return fail(HYQ_ENOTSUP, "hyq_vertical_select: head_dim must be 128");
    if (b < 0 || hq_in <= 0 || hk <= 0 || group <= 0 || hq_in % group) return fail(HYQ_EINVAL, "hyq_vertical_select: bad head counts");
    const int h_out = hq_in / group;
    if (h_out % hk) return fail(HYQ_EINVAL, "hyq_vertical_select: output heads must be a multiple of key heads");
    const int G = h_out / hk;
    if (G > 16) return fail(HYQ_ENOTSUP, "hyq_vertical_select: more than 16 query heads per key head");
    if (p <= 0 || top_k <= 0 || b == 0) return HYQ_OK;
    if (top_k > p) return fail(HYQ_EINVAL, "hyq_vertical_select: top_k > prefix length");
    if (p > TOPK_MAX_P) return fail(HYQ_ENOTSUP, "hyq_vertical_select: prefix longer than 65536");
    if (top_k > TOPK_MAX_T) return fail(HYQ_ENOTSUP, "hyq_vertical_select: top_k above 8192");
    if (tail <= 0 || tail > q_len) return fail(HYQ_EINVAL, "hyq_vertical_select: bad query tail");
    if (!q || !k || !out_idx) return fail(HYQ_EINVAL, "hyq_vertical_select: null pointer");
    if (!aligned(k, 16) || ks_n % 8 || ks_h % 8 || ks_b % 8) return fail(HYQ_EINVAL, "hyq_vertical_select: keys must be 16-byte aligned rows");
    const size_t need = select_ws(b, h_out, p);
    if (!workspace || ws_bytes < need) return fail(HYQ_ENOSPC, "hyq_vertical_select: workspace too small");
    hipStream_t s = static_cast<hipStream_t>(stream);
    double* qm = static_cast<double*>(workspace);
    const size_t qm_bytes = ((static_cast<size_t>(b) * h_out * 128 * sizeof(double) * 4 + 255) / 256) * 256;
    uint16_t* keys = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) + qm_bytes);
    const int GP = padded_heads(G);
    const int64_t nq = static_cast<int64_t>(b) * hk * GP * 128;
    qmean_kernel<<<dim3(static_cast<unsigned>((nq + 127) / 128)), dim3(128), 0, s>>>(q, qs_b, qs_h, qs_t, q_len, tail, group,
                                                                                   hk, G, GP, 128, b, qm);
    int rc = check_launch("hyq_vertical_select (mean)");
    if (rc) return rc;
    const dim3 sgrid(static_cast<unsigned>((p + 255) / 256), static_cast<unsigned>(b * hk));
    switch (GP) {
        case 1: score_kernel<1><<<sgrid, dim3(256), 0, s>>>(k, ks_b, ks_h, ks_n, hk, G, p, qm, keys); break;
        case 2: score_kernel<2><<<sgrid, dim3(256), 0, s>>>(k, ks_b, ks_h, ks_n, hk, G, p, qm, keys); break;
        case 4: score_kernel<4><<<sgrid, dim3(256), 0, s>>>(k, ks_b, ks_h, ks_n, hk, G, p, qm, keys); break;
        case 8: score_kernel<8><<<sgrid, dim3(256), 0, s>>>(k, ks_b, ks_h, ks_n, hk, G, p, qm, keys); break;
        default: score_kernel<16><<<sgrid, dim3(256), 0, s>>>(k, ks_b, ks_h, ks_n, hk, G, p, qm, keys); break;
    }
    rc = check_launch("hyq_vertical_select (score)");
    if (rc) return rc;
    topk_kernel<<<dim3(static_cast<unsigned>(b * h_out)), dim3(TOPK_THREADS), 0, s>>>(keys, p, top_k, out_idx);
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
                                     int8_t* kp, int64_t kp_bh, int64_t kp_n, int8_t* vp, int64_t vp_bh, int64_t vp_n,
                                     uint16_t* ksc, int64_t ksc_bh, uint16_t* vsc, int64_t vsc_bh,
                                     uint16_t* kt, int64_t kt_bh, int64_t kt_n, uint16_t* vt, int64_t vt_bh, int64_t vt_n,
                                     uint16_t* kw, int64_t kw_bh, int64_t kw_n, uint16_t* vw, int64_t vw_bh, int64_t vw_n,
                                     void* workspace, size_t ws_bytes, void* stream) {
    if (d != 128) return fail(HYQ_ENOTSUP, "hyq_freeze_reorganise: head_dim must be 128");
    auto okbits = [](int x) { return x == 2 || x == 4 || x == 8; };
    if (!okbits(k_bits) || !okbits(v_bits)) return fail(HYQ_EINVAL, "hyq_freeze_reorganise: bits must be 2, 4 or 8");
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
        zero_words_kernel<<<dim3(static_cast<unsigned>((nw + 255) / 256)), dim3(256), 0, s>>>(bits, nw);
        if (int rc0 = check_launch("hyq_freeze_reorganise (zero)")) return rc0;
        if (top_k > 0) {
            mark_kernel<<<dim3(static_cast<unsigned>((top_k + 255) / 256), static_cast<unsigned>(bh)), dim3(256), 0, s>>>(
                topk_idx, top_k, P, words, bits);
            int rc = check_launch("hyq_freeze_reorganise (mark)");
            if (rc) return rc;
        }
        CompactArgs a{k, v, ks_b, ks_h, ks_n, vs_b, vs_h, vs_n, hk, P, words, bits,
                      kp, vp, kp_bh, kp_n, vp_bh, vp_n, ksc, vsc, ksc_bh, vsc_bh, k_bits, v_bits};
        dim3 grid(static_cast<unsigned>((P + CQ_CHUNK - 1) / CQ_CHUNK), static_cast<unsigned>(bh));
        if (k_bits == 4 && v_bits == 4) compact_quant_kernel<4, 4><<<grid, dim3(256), 0, s>>>(a);
        else if (k_bits == 4 && v_bits == 2) compact_quant_kernel<4, 2><<<grid, dim3(256), 0, s>>>(a);
        else if (k_bits == 2 && v_bits == 4) compact_quant_kernel<2, 4><<<grid, dim3(256), 0, s>>>(a);
        else if (k_bits == 8 && v_bits == 8) compact_quant_kernel<8, 8><<<grid, dim3(256), 0, s>>>(a);
        else if (k_bits == 2 && v_bits == 2) compact_quant_kernel<2, 2><<<grid, dim3(256), 0, s>>>(a);
        else return fail(HYQ_ENOTSUP, "hyq_freeze_reorganise: unsupported bit pair");
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
