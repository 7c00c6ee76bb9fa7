"""GPU parity of the hybrid prefill (hyq_prefill_hybrid via
sage_vertical_attention_v2), its per-block int8 quantiser (hyq_per_block_int8)
and rest / vertical lists (hyq_prefill_lists) against the CPU oracle.

Quantiser codes and scales and the index lists are compared bit-exactly.
Attention outputs: elementwise |out - ref| <= 2e-3 + 2^-10 ref_abs + 2^-8 |ref|
with ref the float64 restatement and ref_abs = sum p|v| / l: the fp16
rounding of p before P.V (both here and in the reference kernel, <= 2^-11
relative per weight) and the bf16 rounding of the output; max-abs and relative
error are printed."""

import math

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import exact_attention_gpu as _exact_attention_gpu, first_tile_max_inputs, to_dev_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _rand_bf16(rng, shape, scale=1.0):
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def _check(name, out, ref, ref_abs):
    diff = np.abs(out - ref)
    err = float(diff.max())
    rel = err / float(np.abs(ref).max())
    msg = f"{name}: max-abs {err:.3e} rel {rel:.3e} (max|ref| {float(np.abs(ref).max()):.3f})"
    print(msg, flush=True)
    assert np.all(np.isfinite(out))
    bound = ATOL + 2.0 ** -10 * ref_abs + 2.0 ** -8 * np.abs(ref)
    bad = np.argwhere(diff > bound)
    for idx in bad[:6]:
        i = tuple(idx)
        print(f"  violation at {i}: out {out[i]:.6f} ref {ref[i]:.6f} bound {bound[i]:.3e}", flush=True)
    assert bad.size == 0, msg


def _run(q, k, v, vidx, W, **kw):
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    dev = torch.device("cuda")
    vi = torch.from_numpy(np.ascontiguousarray(vidx, dtype=np.int64)).to(dev)
    out = sage_vertical_attention_v2(to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev), vi,
                                     window_size=W, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("layout", ["HND", "NHD"])
def test_per_block_int8_bit_exact(layout):
    from hyquant_amd.sage_unified import per_block_int8
    rng = np.random.default_rng(1)
    q = _rand_bf16(rng, (2, 3, 300, 128), 2.0)
    k = _rand_bf16(rng, (2, 1, 300, 128), 3.0)
    q[1, 2, 128:256] = 0.0                                   # a zero block: scale 0, codes 0
    q[0, 0, 5, 7] = 127.0 / (128 ** -0.5 * O.LOG2E)          # dominant value
    q = O.bf16_round(q)
    km = O.mean_bf16(k, axis=2)[:, :, None, :]
    dev = torch.device("cuda")
    qd, kd, kmd = to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(km, dev)
    if layout == "NHD":
        qd, kd, kmd = qd.transpose(1, 2), kd.transpose(1, 2), kmd.transpose(1, 2)
    q8, qs, k8, ks = per_block_int8(qd, kd, km=kmd, tensor_layout=layout)
    torch.cuda.synchronize()
    if layout == "NHD":
        q8, k8 = q8.transpose(1, 2), k8.transpose(1, 2)
    eq8, eqs = O.per_block_int8(q, np.float32(128 ** -0.5 * O.LOG2E), 128)
    ek8, eks = O.per_block_int8(O.bf16_round(k - km), 1.0, 64)
    assert np.array_equal(q8.cpu().numpy(), eq8)
    assert np.array_equal(qs.cpu().numpy().view(np.uint32), eqs.view(np.uint32))
    assert np.array_equal(k8.cpu().numpy(), ek8)
    assert np.array_equal(ks.cpu().numpy().view(np.uint32), eks.view(np.uint32))


@pytest.mark.parametrize("N,W,T", [(700, 100, 40), (5000, 128, 300), (1000, 1, 999), (300, 64, 0), (100, 256, 5),
                                   (150000, 128, 9000),     # past 131072 positions and 8192 indices, lists in LDS
                                   (700000, 128, 5000)])    # lists larger than LDS: workspace
def test_lists_bit_exact(N, W, T):
    from hyquant_amd.sage_unified import vertical_lists
    rng = np.random.default_rng(N + T)
    B, H = 2, 3
    P = max(0, N - W)
    vidx = rng.integers(-5, max(P, 1) + 5, size=(B, H, T)).astype(np.int64)   # repeats and out-of-range
    got = vertical_lists(torch.from_numpy(vidx).cuda(), N, W)
    torch.cuda.synchronize()
    for b in range(B):
        for h in range(H):
            vert, rest, nv, nr = O.prefill_lists(vidx[b, h], N, W)
            i = b * H + h
            assert np.array_equal(got["nr"][i].cpu().numpy(), nr)
            assert np.array_equal(got["nv"][i].cpu().numpy(), nv)
            if P:
                assert np.array_equal(got["vert"][i].cpu().numpy(), vert)
                rc = int(got["rcount"][i])
                assert rc == len(rest)
                assert np.array_equal(got["rest"][i, :rc].cpu().numpy(), rest)


CASES = [
    dict(B=1, HQ=4, HKV=1, N=640, W=128, T=30, seed=1),            # GQA 4, block-aligned
    dict(B=2, HQ=8, HKV=2, N=1000, W=100, T=45, seed=2),           # ragged last block, W not a multiple of 64
    dict(B=1, HQ=2, HKV=2, N=777, W=256, T=26, seed=3),            # no GQA, wide window
    dict(B=1, HQ=4, HKV=2, N=300, W=512, T=0, seed=4),             # N <= W: window only
    dict(B=1, HQ=2, HKV=1, N=520, W=64, T=0, seed=5),              # no vertical lines
    dict(B=1, HQ=2, HKV=1, N=129, W=1, T=3, seed=6),               # window of one token
]


@pytest.mark.parametrize("cfg", CASES, ids=[f"N{c['N']}W{c['W']}T{c['T']}" for c in CASES])
def test_prefill_small_vs_oracle(cfg):
    print(f"prefill {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"])
    B, HQ, HKV, N, W, T = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W", "T"))
    q = _rand_bf16(rng, (B, HQ, N, 128))
    k = _rand_bf16(rng, (B, HKV, N, 128), 1.5) + O.bf16_round(rng.standard_normal((1, HKV, 1, 128)).astype(np.float32))
    k = O.bf16_round(k)
    v = _rand_bf16(rng, (B, HKV, N, 128))
    P = max(0, N - W)
    vidx = np.stack([np.stack([rng.permutation(P)[:T] if P else np.zeros(0, np.int64) for _ in range(HQ)])
                     for _ in range(B)]).astype(np.int64).reshape(B, HQ, T)
    out = _run(q, k, v, vidx, W)
    ref = O.hybrid_prefill_fp64(q, k, v, vidx, W)
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, W, abs_v=True)
    _check(f"prefill {cfg}", out, ref, ref_abs)


def test_prefill_options_and_strided_inputs():
    rng = np.random.default_rng(9)
    B, HQ, HKV, N, W = 1, 4, 2, 400, 128
    q = _rand_bf16(rng, (B, HQ, N, 128))
    k = _rand_bf16(rng, (B, HKV, N, 128), 2.0)
    v = _rand_bf16(rng, (B, HKV, N, 128))
    vidx = rng.integers(-3, N - W + 3, size=(B, HQ, 20))            # repeats and clamping
    for smooth in (True, False):
        out = _run(q, k, v, vidx, W, smooth_k=smooth, sm_scale=0.05)
        ref = O.hybrid_prefill_fp64(q, k, v, vidx, W, sm_scale=0.05, smooth=smooth)
        ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, W, sm_scale=0.05, smooth=smooth, abs_v=True)
        _check(f"smooth={smooth}", out, ref, ref_abs)
    # NHD-strided views give the same bytes as contiguous inputs
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    dev = torch.device("cuda")
    qd = to_dev_bf16(q, dev).transpose(1, 2).contiguous().transpose(1, 2)
    kd = to_dev_bf16(k, dev).transpose(1, 2).contiguous().transpose(1, 2)
    vd = to_dev_bf16(v, dev).transpose(1, 2).contiguous().transpose(1, 2)
    vi = torch.from_numpy(vidx).cuda()
    a = sage_vertical_attention_v2(qd, kd, vd, vi, window_size=W)
    b = sage_vertical_attention_v2(qd.contiguous(), kd.contiguous(), vd.contiguous(), vi, window_size=W)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("N", [8192, 16384])
def test_prefill_config4(N):
    """Config 4 shape (B=1, 32/8 heads, d128, W=128, rho=5%, seeded Gaussian
    with planted vertical lines).  Two query heads against the float64
    oracle; every head against fp32 exact attention (MSE)."""
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    print(f"prefill config4 N={N}", flush=True)
    q, k, v = O.make_prefill_inputs(B=1, HQ=32, HKV=8, N=N, W=128, seed=0)
    vidx = O.compute_vertical_indices(q, k, 128, 0.05, kv_repeat=4)
    dev = torch.device("cuda")
    qd, kd, vd = to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev)
    out = sage_vertical_attention_v2(qd, kd, vd, torch.from_numpy(vidx).to(dev), window_size=128)
    exact = _exact_attention_gpu(qd, kd, vd)
    mse = float(((out.float() - exact) ** 2).mean())
    print(f"config4 N={N}: MSE vs exact fp32 attention {mse:.3e}", flush=True)
    assert mse < 1e-4
    heads = [5] if N > 8192 else [0, 13]
    o = out.float().cpu().numpy()
    for h in heads:
        hk = h // 4
        sl = lambda a, lo, hi: a[:, lo:hi]
        ref = O.hybrid_prefill_fp64(sl(q, h, h + 1), sl(k, hk, hk + 1), sl(v, hk, hk + 1), sl(vidx, h, h + 1), 128)
        ref_abs = O.hybrid_prefill_fp64(sl(q, h, h + 1), sl(k, hk, hk + 1), sl(v, hk, hk + 1), sl(vidx, h, h + 1),
                                        128, abs_v=True)
        _check(f"config4 N={N} head {h}", o[:, h:h + 1], ref, ref_abs)


def test_prefill_deterministic():
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    q, k, v = O.make_prefill_inputs(B=1, HQ=8, HKV=2, N=2048, W=128, seed=4)
    vidx = O.compute_vertical_indices(q, k, 128, 0.05, kv_repeat=4)
    dev = torch.device("cuda")
    args = (to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev), torch.from_numpy(vidx).to(dev))
    a = sage_vertical_attention_v2(*args, window_size=128)
    b = sage_vertical_attention_v2(*args, window_size=128)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


FP8_CASES = [CASES[0], CASES[1], CASES[2], CASES[3]]


@pytest.mark.parametrize("cfg", FP8_CASES, ids=[f"fp8-N{c['N']}W{c['W']}T{c['T']}" for c in FP8_CASES])
def test_prefill_fp8_pv_vs_oracle(cfg):
    """pv_mode='fp8' against the fp8 restatement.  The kernel rounds P' to e4m3
    relative to its running maximum and the oracle relative to the row
    maximum, so each weight may sit on a different e4m3 neighbour (3 mantissa
    bits: 2^-4 relative each): |out - ref| <= 2e-3 + 2^-3 ref_abs + 2^-8 |ref|."""
    print(f"prefill fp8 {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"] + 100)
    B, HQ, HKV, N, W, T = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W", "T"))
    q = _rand_bf16(rng, (B, HQ, N, 128))
    k = O.bf16_round(_rand_bf16(rng, (B, HKV, N, 128), 1.5) +
                     O.bf16_round(rng.standard_normal((1, HKV, 1, 128)).astype(np.float32)))
    v = _rand_bf16(rng, (B, HKV, N, 128))
    P = max(0, N - W)
    vidx = np.stack([np.stack([rng.permutation(P)[:T] if P else np.zeros(0, np.int64) for _ in range(HQ)])
                     for _ in range(B)]).astype(np.int64).reshape(B, HQ, T)
    out = _run(q, k, v, vidx, W, pv_mode="fp8")
    ref = O.hybrid_prefill_fp64(q, k, v, vidx, W, pv_mode="fp8")
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, W, abs_v=True)
    diff = np.abs(out - ref)
    bound = ATOL + 2.0 ** -3 * ref_abs + 2.0 ** -8 * np.abs(ref)
    print(f"fp8 {cfg}: max-abs {float(diff.max()):.3e}, max diff/bound {float((diff / bound).max()):.3f}", flush=True)
    assert np.all(np.isfinite(out))
    assert np.all(diff <= bound)
    # and the fp8 output stays close to exact attention
    exact = O.exact_causal_attention(q, k, v)
    mse = float(np.mean((out - exact) ** 2))
    print(f"fp8 {cfg}: MSE vs exact {mse:.3e}", flush=True)
    assert mse < 1e-4


def test_prefill_fp8_config4_mse():
    """Config 4 shape at 8K with the fp8 PV variant: MSE vs exact attention."""
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    q, k, v = O.make_prefill_inputs(B=1, HQ=32, HKV=8, N=8192, W=128, seed=0)
    vidx = O.compute_vertical_indices(q, k, 128, 0.05, kv_repeat=4)
    dev = torch.device("cuda")
    qd, kd, vd = to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev)
    out8 = sage_vertical_attention_v2(qd, kd, vd, torch.from_numpy(vidx).to(dev), window_size=128, pv_mode="fp8")
    out16 = sage_vertical_attention_v2(qd, kd, vd, torch.from_numpy(vidx).to(dev), window_size=128)
    exact = _exact_attention_gpu(qd, kd, vd)
    mse8 = float(((out8.float() - exact) ** 2).mean())
    mse16 = float(((out16.float() - exact) ** 2).mean())
    print(f"config4 N=8192: MSE vs exact, fp16 PV {mse16:.3e}, fp8 PV {mse8:.3e}", flush=True)
    assert mse8 < 1e-4


UNIFIED_CASES = [
    dict(B=1, HQ=4, HKV=1, N=640, W=0, seed=21),                  # sage_w0: int8 through the diagonal
    dict(B=2, HQ=4, HKV=2, N=777, W=0, seed=22),                  # ragged last block
    dict(B=1, HQ=4, HKV=1, N=700, W=128, seed=23),                # sage_w
    dict(B=1, HQ=2, HKV=1, N=520, W=100, seed=24),                # window not a multiple of 64
    dict(B=1, HQ=2, HKV=2, N=129, W=0, seed=25),                  # one full block and one row
    dict(B=1, HQ=4, HKV=2, N=300, W=512, seed=26),                # window >= N: fp16 everywhere
]


@pytest.mark.parametrize("cfg", UNIFIED_CASES, ids=[f"unified-N{c['N']}W{c['W']}" for c in UNIFIED_CASES])
def test_unified_prefill_vs_oracle(cfg):
    """sage_unified_attention (hyq_prefill_unified): window-only INT8-QK
    prefill against the float64 restatement of sage_unified.py:112-313."""
    from hyquant_amd.sage_unified import sage_unified_attention
    print(f"unified {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"])
    B, HQ, HKV, N, W = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W"))
    q = _rand_bf16(rng, (B, HQ, N, 128))
    k = O.bf16_round(_rand_bf16(rng, (B, HKV, N, 128), 1.5)
                     + O.bf16_round(rng.standard_normal((1, HKV, 1, 128)).astype(np.float32)))
    v = _rand_bf16(rng, (B, HKV, N, 128))
    dev = torch.device("cuda")
    out = sage_unified_attention(to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev), window_size=W)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    ref = O.unified_prefill_fp64(q, k, v, W)
    ref_abs = O.unified_prefill_fp64(q, k, v, W, abs_v=True)
    _check(f"unified {cfg}", out, ref, ref_abs)



FP8QK_CASES = [
    dict(B=1, HQ=4, HKV=1, N=640, W=128, T=30, seed=41),
    dict(B=2, HQ=8, HKV=2, N=1000, W=100, T=45, seed=42),          # ragged last block, GQA 4
    dict(B=1, HQ=2, HKV=1, N=520, W=64, T=0, seed=43),             # no vertical lines
]


@pytest.mark.parametrize("cfg", FP8QK_CASES, ids=[f"fp8qk-N{c['N']}W{c['W']}T{c['T']}" for c in FP8QK_CASES])
def test_prefill_fp8qk_vs_oracle(cfg):
    """sage_vertical_attention_v2_fp8 (hyq_prefill_hybrid_fp8qk): e4m3 Q and
    rest K against the float64 restatement of sage_unified_fp8.py."""
    from hyquant_amd.sage_unified import sage_vertical_attention_v2_fp8
    print(f"fp8qk {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"])
    B, HQ, HKV, N, W, T = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W", "T"))
    q = _rand_bf16(rng, (B, HQ, N, 128))
    k = O.bf16_round(_rand_bf16(rng, (B, HKV, N, 128), 1.5)
                     + O.bf16_round(rng.standard_normal((1, HKV, 1, 128)).astype(np.float32)))
    v = _rand_bf16(rng, (B, HKV, N, 128))
    P = max(0, N - W)
    vidx = np.stack([np.stack([rng.permutation(P)[:T] for _ in range(HQ)]) for _ in range(B)]).astype(np.int64)
    vidx = vidx.reshape(B, HQ, T)
    dev = torch.device("cuda")
    out = sage_vertical_attention_v2_fp8(to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev),
                                         torch.from_numpy(vidx).to(dev), window_size=W)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    ref = O.hybrid_prefill_fp64(q, k, v, vidx, W, qk_mode="fp8")
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, W, qk_mode="fp8", abs_v=True)
    _check(f"fp8qk {cfg}", out, ref, ref_abs)


@pytest.mark.parametrize("cfg", [dict(B=1, HQ=4, HKV=1, N=1000, W=100, T=45, seed=51),
                                 dict(B=1, HQ=8, HKV=2, N=2304, W=128, T=110, seed=52)],
                         ids=["N1000", "N2304"])
def test_prefill_fp8_pv_tight_where_running_max_is_exact(cfg):
    """FP8 P.V (csrc/qattn/qk_int_sv_f8_cuda_sm90.cu:490-512,
    attn_utils.cuh:354-458): P' = e4m3(exp2(s - m + 8.807)).  Where the
    kernel's running max equals the row max from its first tile on, it must
    round each P' to the same e4m3 value as the oracle, except for weights
    that lie within a relative 2^-14 of an e4m3 (or fp16) rounding boundary,
    where fp32 evaluation may take either neighbour (`slack`).  So the bf16
    output must be the rounding of a value within
        slack + 2^-13 sum P'|V|/l + 2^-15 |ref| + 1e-6
    of the float64 fp8 restatement (fp32 accumulation and score rounding);
    a systematic e4m3 error of ~3% of P' breaks this by an order of magnitude."""
    print(f"prefill fp8 tight {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"])
    B, HQ, HKV, N, W, T = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W", "T"))
    q, k, v, vidx = first_tile_max_inputs(rng, B, HQ, HKV, N, W, T)
    out = _run(q, k, v, vidx, W, pv_mode="fp8")
    ref, slack, exact = O.hybrid_prefill_fp64(q, k, v, vidx, W, pv_mode="fp8", fp8_detail=True)
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, W, pv_mode="fp8", abs_v=True)
    frac = float(exact.mean())
    print(f"  rows with an exact running max: {frac:.4f}; mean slack {float(slack.mean()):.2e}", flush=True)
    assert frac > 0.99
    eps = slack + 2.0 ** -13 * ref_abs + 2.0 ** -15 * np.abs(ref) + 1e-6
    from tests.gpu_util import bf16_bracket
    bad = bf16_bracket(out, ref, eps) & exact[..., None]
    diff = np.abs(out - ref)
    print(f"  max-abs {float(diff.max()):.3e}, max |out-ref|/eps on exact rows "
          f"{float((diff / eps)[np.broadcast_to(exact[..., None], diff.shape)].max()):.3f}", flush=True)
    assert not bad.any(), f"{int(bad.sum())} elements outside the tight fp8 bound"
    loose = ATOL + 2.0 ** -3 * ref_abs + 2.0 ** -8 * np.abs(ref)
    assert not ((diff > loose) & ~exact[..., None]).any()
    # the relative L2 error against the fp8 restatement, and what an e4m3
    # rounding with truncation instead of round-to-nearest-even would give
    l2 = float(np.linalg.norm(out - ref) / np.linalg.norm(ref))
    print(f"  relative L2 vs the fp8 oracle {l2:.3e}", flush=True)
    assert l2 < 2.0 ** -9


def test_prefill_past_131072_positions():
    """sage_vertical_attention_v2 at N = 140000 (the reference's
    reorder_kv_for_vertical has no length limit, src/ops/sage_unified.py:499-547):
    one query head against the float64 oracle on its first, a middle and its
    last query blocks, every head against fp32 exact attention (MSE)."""
    from hyquant_amd.sage_unified import sage_vertical_attention_v2
    N, W = 140000, 128
    print(f"prefill long N={N}", flush=True)
    rng = np.random.default_rng(77)
    q = _rand_bf16(rng, (1, 2, N, 128))
    k = O.bf16_round(_rand_bf16(rng, (1, 1, N, 128), 1.5) + O.bf16_round(rng.standard_normal((1, 1, 1, 128)).astype(np.float32)))
    v = _rand_bf16(rng, (1, 1, N, 128))
    vidx = O.compute_vertical_indices(q, k, W, 0.05, kv_repeat=2)
    assert vidx.shape[-1] > 6000
    dev = torch.device("cuda")
    qd, kd, vd = to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev)
    out = sage_vertical_attention_v2(qd, kd, vd, torch.from_numpy(vidx).to(dev), window_size=W)
    exact = _exact_attention_gpu(qd, kd, vd, chunk=2048)
    mse = float(((out.float() - exact) ** 2).mean())
    print(f"  N={N}: MSE vs exact fp32 attention {mse:.3e}", flush=True)
    assert mse < 1e-6
    nblk = (N + 127) // 128
    blocks = [0, nblk // 2, nblk - 1]
    ref = O.hybrid_prefill_fp64(q[:, :1], k, v, vidx[:, :1], W, blocks=blocks)
    ref_abs = O.hybrid_prefill_fp64(q[:, :1], k, v, vidx[:, :1], W, blocks=blocks, abs_v=True)
    rows = np.concatenate([np.arange(b * 128, min(N, (b + 1) * 128)) for b in blocks])
    o = out[:, :1].float().cpu().numpy()
    _check(f"N={N} head 0 blocks {blocks}", o[:, :, rows], ref[:, :, rows], ref_abs[:, :, rows])


FP16_CASES = [
    dict(entry="hybrid", B=2, HQ=8, HKV=2, N=1000, W=100, T=45, seed=61),
    dict(entry="hybrid_fp8pv", B=1, HQ=4, HKV=1, N=640, W=128, T=30, seed=62),
    dict(entry="unified", B=1, HQ=4, HKV=2, N=700, W=128, T=0, seed=63),
    dict(entry="unified_w0", B=1, HQ=2, HKV=1, N=520, W=0, T=0, seed=64),
    dict(entry="fp8qk", B=1, HQ=4, HKV=1, N=640, W=128, T=30, seed=65),
]


@pytest.mark.parametrize("cfg", FP16_CASES, ids=[c["entry"] for c in FP16_CASES])
def test_prefill_fp16_model(cfg):
    """An fp16 model's prefill (src/ops/sage_unified.py:565-580 and
    sage_unified_fp8.py:344-351, the dtype == float16 branch): fp16 q, k, v in,
    fp16 out, against the float64 restatement of that branch.  The kernel
    must also be much closer to it than to the bf16 branch on the same
    values (which rounds q * c and k - km to bf16 first), so a kernel that
    took the wrong branch fails."""
    from hyquant_amd import sage_unified as su
    print(f"prefill fp16 {cfg}", flush=True)
    rng = np.random.default_rng(cfg["seed"])
    B, HQ, HKV, N, W, T = (cfg[x] for x in ("B", "HQ", "HKV", "N", "W", "T"))
    f16 = lambda a: a.astype(np.float16).astype(np.float32)
    q = f16(rng.standard_normal((B, HQ, N, 128)) * 1.3)
    k = f16(rng.standard_normal((B, HKV, N, 128)) * 1.5 + rng.standard_normal((1, HKV, 1, 128)))
    v = f16(rng.standard_normal((B, HKV, N, 128)))
    P = max(0, N - W)
    vidx = np.stack([np.stack([rng.permutation(P)[:T] if P else np.zeros(0, np.int64) for _ in range(HQ)])
                     for _ in range(B)]).astype(np.int64).reshape(B, HQ, T)
    dev = torch.device("cuda")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.float16).to(dev)
    vi = torch.from_numpy(vidx).to(dev)
    e = cfg["entry"]
    if e.startswith("hybrid"):
        pv = "fp8" if e == "hybrid_fp8pv" else "fp16"
        out = su.sage_vertical_attention_v2(d(q), d(k), d(v), vi, window_size=W, pv_mode=pv)
        oracle = lambda fp16, **kw: O.hybrid_prefill_fp64(q, k, v, vidx, W, pv_mode=pv, fp16=fp16, **kw)
    elif e == "fp8qk":
        out = su.sage_vertical_attention_v2_fp8(d(q), d(k), d(v), vi, window_size=W)
        oracle = lambda fp16, **kw: O.hybrid_prefill_fp64(q, k, v, vidx, W, qk_mode="fp8", fp16=fp16, **kw)
    else:
        out = su.sage_unified_attention(d(q), d(k), d(v), window_size=W)
        oracle = lambda fp16, **kw: O.unified_prefill_fp64(q, k, v, W, fp16=fp16, **kw)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    out = out.float().cpu().numpy()
    ref = oracle(True)
    ref_abs = oracle(True, abs_v=True)
    if e == "hybrid_fp8pv":
        # e4m3 P' and V: the loose fp8 bound of test_prefill_fp8_pv_vs_oracle
        diff = np.abs(out - ref)
        assert np.all(diff <= ATOL + 2.0 ** -3 * ref_abs + 2.0 ** -8 * np.abs(ref)), float(diff.max())
    else:
        _check(f"fp16 {e}", out, ref, ref_abs)
    mse16 = float(np.mean((out - ref) ** 2))
    mse_b = float(np.mean((out - oracle(False)) ** 2))
    print(f"  mse vs fp16 branch {mse16:.3e}, vs bf16 branch {mse_b:.3e}", flush=True)
    if e != "hybrid_fp8pv":        # there the e4m3 rounding of P' hides the branch difference
        assert mse16 * 4 < mse_b
