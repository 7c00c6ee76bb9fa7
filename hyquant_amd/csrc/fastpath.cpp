// Eager fast path of fused_d_stage_decode (src/ops/decode_d_stage.py:
// 470-1005 is the reference's call): a Python extension that reads the
// tensors' metadata natively, fills one hyq_decode_params, allocates the
// output and calls hyq_decode_hybrid through the pointer the Python side
// hands over at set-up (the library ctypes loaded, whichever file that is).
//
// It takes exactly the calls the Python fast path takes (bf16 / fp16 q with
// unit channel stride, kv_repeat dividing the query heads, CUDA tensors, the
// three bf16 segments with unit channel strides, equal K / V lengths and one
// dtype, the quantised prefix with unit innermost strides); anything else
// returns status -1 and the caller takes its other paths.  The library
// validates every field (alignment, 32-bit strides, sizes) before it
// launches, as for every other caller.  Host code only: no kernel here.

#include <torch/extension.h>

#include <cmath>
#include <cstddef>
#include <cstdint>

#include "../../include/hyq.h"

namespace {

using HybridFn = int (*)(const hyq_decode_params*, void*, size_t, void*);
HybridFn g_hybrid = nullptr;

// one bf16 / fp16 segment: 0 empty, 1 bf16, 2 fp16, -1 not taken
int segment(const at::Tensor& k, const at::Tensor& v, hyq_decode_params& p, int s) {
    if (k.dim() != 3 || v.dim() != 3) return -1;
    const int64_t n = k.size(1);
    if (n == 0) return 0;
    const auto dt = k.scalar_type();
    if (k.stride(2) != 1 || v.stride(2) != 1 || v.size(1) != n || v.scalar_type() != dt) return -1;
    if (dt != at::kBFloat16 && dt != at::kHalf) return -1;
    p.seg_k[s] = static_cast<const uint16_t*>(k.data_ptr());
    p.seg_k_stride_bh[s] = k.stride(0);
    p.seg_k_stride_n[s] = k.stride(1);
    p.seg_v[s] = static_cast<const uint16_t*>(v.data_ptr());
    p.seg_v_stride_bh[s] = v.stride(0);
    p.seg_v_stride_n[s] = v.stride(1);
    p.seg_n[s] = n;
    return dt == at::kBFloat16 ? 1 : 2;
}

}  // namespace

// the library entry point (an address from ctypes)
void set_entry(int64_t hybrid) { g_hybrid = reinterpret_cast<HybridFn>(hybrid); }

// (status, out): status 0 launched; -1 not taken (nothing launched); any
// other value is the library's status for this call (nothing launched)
std::tuple<int64_t, at::Tensor> decode(const at::Tensor& q, const at::Tensor& kp, const at::Tensor& vp,
                                       const at::Tensor& ks, const at::Tensor& vs, const at::Tensor& kt,
                                       const at::Tensor& vt, const at::Tensor& kst, const at::Tensor& vst,
                                       const at::Tensor& kw, const at::Tensor& vw, int64_t k_bits, int64_t v_bits,
                                       int64_t kv_repeat, double sm_scale, int64_t split_tokens, int64_t stream,
                                       int64_t ws, int64_t ws_bytes) {
    const std::tuple<int64_t, at::Tensor> skip{-1, at::Tensor()};
    if (!g_hybrid || q.dim() != 2 || !q.is_cuda()) return skip;
    hyq_decode_params p{};
    const auto qdt = q.scalar_type();
    if (qdt == at::kBFloat16) p.dtype_flags = 0;
    else if (qdt == at::kHalf) p.dtype_flags = HYQ_DT_Q_FP16 | HYQ_DT_OUT_FP16;
    else return skip;
    const int64_t bh_q = q.size(0), d = q.size(1);
    if (q.stride(1) != 1 || kv_repeat < 1 || bh_q % kv_repeat) return skip;
    int dts = 0;
    const at::Tensor* segs[3][2] = {{&kt, &vt}, {&kst, &vst}, {&kw, &vw}};
    for (int s = 0; s < 3; ++s) {
        const int dt = segment(*segs[s][0], *segs[s][1], p, s);
        if (dt < 0) return skip;
        if (dt > 0) {
            if (dts && dts != dt) return skip;
            dts = dt;
        }
    }
    if (dts == 2) p.dtype_flags |= HYQ_DT_SEG_FP16;
    if (kp.dim() != 3 || vp.dim() != 3 || ks.dim() != 2 || vs.dim() != 2) return skip;
    const int64_t nq = kp.size(1);
    if (nq > 0) {
        if (kp.stride(2) != 1 || vp.stride(2) != 1 || ks.stride(1) != 1 || vs.stride(1) != 1) return skip;
        p.k_packed = static_cast<const int8_t*>(kp.data_ptr());
        p.kp_stride_bh = kp.stride(0);
        p.kp_stride_n = kp.stride(1);
        p.v_packed = static_cast<const int8_t*>(vp.data_ptr());
        p.vp_stride_bh = vp.stride(0);
        p.vp_stride_n = vp.stride(1);
        p.k_scale = static_cast<const uint16_t*>(ks.data_ptr());
        p.ks_stride_bh = ks.stride(0);
        p.v_scale = static_cast<const uint16_t*>(vs.data_ptr());
        p.vs_stride_bh = vs.stride(0);
    }
    p.n_quant = nq;
    at::Tensor out = at::empty({bh_q, d}, q.options());
    p.q = static_cast<const uint16_t*>(q.data_ptr());
    p.q_stride = q.stride(0);
    p.out = static_cast<uint16_t*>(out.data_ptr());
    p.out_stride = d;
    p.bh_kv = static_cast<int32_t>(bh_q / kv_repeat);
    p.kv_repeat = static_cast<int32_t>(kv_repeat);
    p.head_dim = static_cast<int32_t>(d);
    p.k_bits = static_cast<int32_t>(k_bits);
    p.v_bits = static_cast<int32_t>(v_bits);
    // (head_dim ** -0.5 as Python computes it, then rounded to float)
    p.sm_scale = std::isnan(sm_scale) ? static_cast<float>(std::pow(static_cast<double>(d), -0.5))
                                      : static_cast<float>(sm_scale);
    p.split_tokens = static_cast<int32_t>(split_tokens);
    const int st = g_hybrid(&p, reinterpret_cast<void*>(ws), static_cast<size_t>(ws_bytes),
                            reinterpret_cast<void*>(stream));
    return {st, out};
}

// the parameter block's size and the offsets of its first and last fields,
// which the caller compares with its own view of include/hyq.h before it
// uses this module
std::tuple<int64_t, int64_t, int64_t> layout() {
    return {static_cast<int64_t>(sizeof(hyq_decode_params)),
            static_cast<int64_t>(offsetof(hyq_decode_params, seg_n)),
            static_cast<int64_t>(offsetof(hyq_decode_params, dtype_flags))};
}

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.def("layout", &layout, "sizeof(hyq_decode_params), offsetof(seg_n), offsetof(dtype_flags)");
    m.def("set_entry", &set_entry, "hyq_decode_hybrid's address");
    m.def("decode", &decode, "fused_d_stage_decode eager fast path");
}
