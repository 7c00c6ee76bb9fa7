"""GPU parity at the BASELINE workloads' own sizes.

Each benchmark configuration that the bench times is also checked here, at
the same size, against the CPU oracle:
  config 2: the decode sweep at B=1 (2K, 4K, 16K prefixes; 1K, 8K and 32K are
            in test_gpu_decode) and at B=16 (every prefix 1K..32K);
  config 3: B=32, 16K prefix: Qwen3-32B (64q/8kv) and GLM-4-9B (32q/2kv)
            freeze + decode, and the Llama-shape (32q/8kv) prefill-time
            selector, freeze at W=256 and a 128-token flush over 256 heads;
  config 4: hybrid prefill at N=32768 (all four kernel variants).
States are built on the GPU by the library's own path (selector, freeze,
staging ring), from inputs drawn on the GPU with the benchmark's
distribution (tests/gpu_util.gpu_prefill_inputs).  The oracle runs on sampled
KV heads / batch entries / query blocks (the first, the last and random
ones), which keeps every test to seconds of CPU work:
  int4 codes, scales, bf16 segments and vertical-line indices bit-exact;
  decode outputs within 2e-3 max-abs of the float64 oracle (relative error
  printed), finite everywhere and bit-identical across two calls;
  prefill outputs within the bound of tests/test_gpu_prefill.py against the
  float64 oracle on sampled heads and query blocks, plus MSE and relative L2
  against float32 exact attention over every head."""

import math

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import (bf16_bracket, cache_from_inputs, check_layer_state, exact_attention_gpu,
                            gpu_prefill_inputs, layer_head_state, np_f32, sample_heads, to_dev_bf16)

pytestmark = pytest.mark.gpu

D = 128
RHO = 0.05
ATOL = 2e-3


def _frozen_layer(q_tail, k, v, W, G, k_bits=4, v_bits=4):
    from hyquant_amd.d_stage_kv_cache import DStageLayerCache
    layer = DStageLayerCache(0, k_bits=k_bits, v_bits=v_bits, window_size=W, top_ratio=RHO)
    layer.update_prefill(k, v)
    layer.save_query_tail(q_tail)
    layer.freeze(kv_repeat=G)
    return layer


def _staging_tokens(B, HKV, S, seed, dev):
    g = torch.Generator(device=dev).manual_seed(seed)
    kn = (torch.randn(B, HKV, S, D, generator=g, device=dev) * 1.4).to(torch.bfloat16)
    vn = torch.randn(B, HKV, S, D, generator=g, device=dev).to(torch.bfloat16)
    return kn, vn


def _check_freeze_entry(layer, k, v, q_tail, b, W, G):
    """Batch entry b of a frozen layer against the oracle's freeze of that
    entry alone (entries are independent), bit-exact."""
    HKV = k.shape[1]
    st = O.freeze(np_f32(k[b:b + 1]), np_f32(v[b:b + 1]), np_f32(q_tail[b:b + 1]), W, RHO, G,
                  k_bits=layer.k_bits, v_bits=layer.v_bits)
    rows = slice(b * HKV, (b + 1) * HKV)
    n = st.k_packed.shape[1]
    got_idx = layer.topk_indices[b:b + 1].cpu().numpy()
    assert np.array_equal(got_idx, st.topk_idx), f"vertical-line indices of entry {b}"
    assert layer._kstore.n >= n
    assert np.array_equal(layer._kstore.packed[rows, :n].cpu().numpy(), st.k_packed)
    assert np.array_equal(layer._vstore.packed[rows, :n].cpu().numpy(), st.v_packed)
    assert np.array_equal(layer._kstore.scale[rows, :n].cpu().numpy().view(np.uint16), st.k_scale.view(np.uint16))
    assert np.array_equal(layer._vstore.scale[rows, :n].cpu().numpy().view(np.uint16), st.v_scale.view(np.uint16))
    assert np.array_equal(np_f32(layer.k_topk[rows]), st.k_topk)
    assert np.array_equal(np_f32(layer.v_topk[rows]), st.v_topk)
    assert np.array_equal(np_f32(layer.k_window[rows]), st.k_window)
    assert np.array_equal(np_f32(layer.v_window[rows]), st.v_window)
    print(f"  freeze entry {b}: T={st.topk_idx.shape[-1]} N_q={n} bit-exact", flush=True)


def _decode_sampled(layer, G, name, seed, n_heads=8):
    """Decode one query token per head; sampled KV heads against the fp64
    oracle over the layer's own segments; the whole output finite and
    bit-identical across two calls."""
    B, HKV = layer._B, layer._H_KV
    dev = layer.k_topk.device
    g = torch.Generator(device=dev).manual_seed(seed)
    q = torch.randn(B, HKV * G, 1, D, generator=g, device=dev).to(torch.bfloat16)
    out1 = layer.decode_attention(q, G)
    out2 = layer.decode_attention(q, G)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out1.float()).all()), name
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16)), f"{name}: two calls differ"
    heads = sample_heads(B * HKV, n_heads, seed)
    st = layer_head_state(layer, heads)
    rows = [h * G + g_ for h in heads for g_ in range(G)]
    qf = np_f32(q.reshape(-1, D)[rows])
    ref = O.decode_fp64_state(qf, st, G)
    got = np_f32(out1.reshape(-1, D)[rows])
    err = float(np.max(np.abs(got - ref)))
    rel = err / float(np.max(np.abs(ref)))
    l2 = float(np.linalg.norm(got - ref) / np.linalg.norm(ref))
    print(f"  {name}: decode heads {heads}: max-abs {err:.3e} rel {rel:.3e} rel-L2 {l2:.3e}", flush=True)
    assert err <= ATOL, f"{name}: max-abs {err}"


# ---------------------------------------------------------------------------
# config 3: wide-GQA decode at B=32, 16K prefix
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("name,HQ,HKV", [("Qwen3-32B", 64, 8), ("GLM-4-9B", 32, 2)])
def test_config3_wide_gqa_freeze_and_decode(name, HQ, HKV):
    B, N, W, S = 32, 16384, 128, 64
    G = HQ // HKV
    dev = torch.device("cuda")
    print(f"config3 {name}: B={B} {HQ}q/{HKV}kv N={N} W={W} S={S}", flush=True)
    q, k, v = gpu_prefill_inputs(B, HQ, HKV, N, W, seed=31 + HQ, dev=dev, q_len=W)
    layer = _frozen_layer(q, k, v, W, G)
    layer.append_staging(*_staging_tokens(B, HKV, S, 5, dev))
    torch.cuda.synchronize()
    for b in (0, B - 1):
        _check_freeze_entry(layer, k, v, q, b, W, G)
    del k, v
    _decode_sampled(layer, G, f"config3 {name}", seed=HQ)


def test_config3_select_freeze_flush_llama_shape():
    """The prefill->decode boundary of config 3 (B=32, 32q/8kv, N=16384,
    W=256): the prefill-time selector on the full-length query tensor, the
    freeze, a staging flush of 128 tokens over all 256 KV heads, then decode."""
    from hyquant_amd.vertical import compute_vertical_indices
    B, HQ, HKV, N, W = 32, 32, 8, 16384, 256
    G = HQ // HKV
    dev = torch.device("cuda")
    print(f"config3 boundary: B={B} {HQ}q/{HKV}kv N={N} W={W}", flush=True)
    q, k, v = gpu_prefill_inputs(B, HQ, HKV, N, W, seed=33, dev=dev)
    vidx = compute_vertical_indices(q, k, W, RHO, kv_repeat=G)
    torch.cuda.synchronize()
    T = math.ceil((N - W) * RHO)
    assert tuple(vidx.shape) == (B, HQ, T)
    for b in (0, 13, B - 1):
        exp = O.compute_vertical_indices(np_f32(q[b:b + 1, :, -W:]), np_f32(k[b:b + 1]), W, RHO, kv_repeat=G)
        assert np.array_equal(vidx[b:b + 1].cpu().numpy(), exp), f"selector entry {b}"
        print(f"  selector entry {b}: {T} indices per head bit-exact", flush=True)
    q_tail = q[:, :, -W:].contiguous()
    del q, vidx
    layer = _frozen_layer(q_tail, k, v, W, G)
    torch.cuda.synchronize()
    for b in (0, B - 1):
        _check_freeze_entry(layer, k, v, q_tail, b, W, G)
    del k, v
    # the flush: 128 staging tokens fill the ring, which is quantised and
    # appended to the prefix of every one of the 256 KV heads
    n0 = layer._kstore.n
    kn, vn = _staging_tokens(B, HKV, 128, 7, dev)
    layer.append_staging(kn, vn)
    torch.cuda.synchronize()
    assert layer._staging_ptr == 0 and layer._kstore.n == n0 + 128
    for store, x in ((layer._kstore, kn), (layer._vstore, vn)):
        rp, rs = O.quantize_per_token(np_f32(x).reshape(B * HKV, 128, D), 4)
        assert np.array_equal(store.packed[:, n0:n0 + 128].cpu().numpy(), rp)
        assert np.array_equal(store.scale[:, n0:n0 + 128].cpu().numpy().view(np.uint16), rs.view(np.uint16))
    print("  flush of 128 tokens x 256 heads bit-exact", flush=True)
    layer.append_staging(*_staging_tokens(B, HKV, 64, 8, dev))
    _decode_sampled(layer, G, "config3 Llama after flush", seed=3)


# ---------------------------------------------------------------------------
# config 2: the decode sweep at B=16 (every prefix) and B=1 (2K, 4K, 16K)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("N", [1024, 2048, 4096, 8192, 16384, 32768])
def test_config2_batch16(N):
    B, HQ, HKV, W, S = 16, 32, 8, 128, 64
    G = HQ // HKV
    dev = torch.device("cuda")
    print(f"config2 B={B} N={N}", flush=True)
    q, k, v = gpu_prefill_inputs(B, HQ, HKV, N, W, seed=N, dev=dev, q_len=W)
    layer = _frozen_layer(q, k, v, W, G)
    layer.append_staging(*_staging_tokens(B, HKV, S, N + 1, dev))
    torch.cuda.synchronize()
    _check_freeze_entry(layer, k, v, q, B - 1, W, G)
    del k, v
    _decode_sampled(layer, G, f"config2 B=16 N={N}", seed=N)


@pytest.mark.parametrize("N", [2048, 4096, 16384])
def test_config2_batch1(N):
    """B=1 at the prefixes the other decode tests leave out: inputs drawn on
    the CPU (make_decode_inputs), frozen on the GPU, every head checked."""
    print(f"config2 B=1 N={N}", flush=True)
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=N, W=128, S=64, seed=N + 7)
    layer = cache_from_inputs(inp)
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, 4)
    torch.cuda.synchronize()
    check_layer_state(layer, st)
    layer.append_staging(to_dev_bf16(inp.k_new, "cuda"), to_dev_bf16(inp.v_new, "cuda"))
    O.append_staging(st, inp.k_new, inp.v_new)
    qd = to_dev_bf16(inp.q_dec, "cuda").reshape(1, 32, 1, D)
    out = layer.decode_attention(qd, 4).reshape(-1, D)
    again = layer.decode_attention(qd, 4).reshape(-1, D)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    got = np_f32(out)
    ref = O.decode_fp64_state(inp.q_dec, st, 4)
    err = float(np.max(np.abs(got - ref)))
    print(f"  config2 B=1 N={N}: max-abs {err:.3e} rel {err / float(np.max(np.abs(ref))):.3e}", flush=True)
    assert err <= ATOL


# ---------------------------------------------------------------------------
# config 4: hybrid prefill at N = 32768
# ---------------------------------------------------------------------------

PREFILL_VARIANTS = [
    # (name, entry point, kwargs, oracle kwargs, MSE bound, relative-L2 bound vs fp32 exact)
    ("int8qk-fp16pv", "v2", {}, {}, 1e-6, 0.02),
    ("int8qk-fp8pv", "v2", {"pv_mode": "fp8"}, {"pv_mode": "fp8"}, 5e-6, 0.04),
    ("fp8qk-fp16pv", "v2fp8", {}, {"qk_mode": "fp8"}, 5e-6, 0.04),
    ("window-only", "unified", {}, None, 1e-6, 0.02),
]


@pytest.fixture(scope="module")
def config4_inputs():
    from hyquant_amd.vertical import compute_vertical_indices
    N, W = 32768, 128
    q, k, v = O.make_prefill_inputs(B=1, HQ=32, HKV=8, N=N, W=W, seed=0)
    dev = torch.device("cuda")
    qd, kd, vd = to_dev_bf16(q, dev), to_dev_bf16(k, dev), to_dev_bf16(v, dev)
    vidx = compute_vertical_indices(qd, kd, W, RHO, kv_repeat=4)
    exact = exact_attention_gpu(qd, kd, vd)
    torch.cuda.synchronize()
    return dict(q=q, k=k, v=v, qd=qd, kd=kd, vd=vd, vidx=vidx, vidx_np=vidx.cpu().numpy(), exact=exact, N=N, W=W)


@pytest.mark.parametrize("variant", PREFILL_VARIANTS, ids=[v[0] for v in PREFILL_VARIANTS])
def test_config4_prefill_32k(config4_inputs, variant):
    from hyquant_amd.sage_unified import (sage_unified_attention, sage_vertical_attention_v2,
                                          sage_vertical_attention_v2_fp8)
    name, entry, kw, okw, mse_bound, l2_bound = variant
    c = config4_inputs
    N, W = c["N"], c["W"]
    print(f"config4 N={N} {name}", flush=True)
    if entry == "v2":
        out = sage_vertical_attention_v2(c["qd"], c["kd"], c["vd"], c["vidx"], window_size=W, **kw)
    elif entry == "v2fp8":
        out = sage_vertical_attention_v2_fp8(c["qd"], c["kd"], c["vd"], c["vidx"], window_size=W, **kw)
    else:
        out = sage_unified_attention(c["qd"], c["kd"], c["vd"], window_size=W)
    torch.cuda.synchronize()
    d = out.float() - c["exact"]
    mse = float((d * d).mean())
    l2 = float(d.norm() / c["exact"].norm())
    print(f"  {name}: vs fp32 exact attention MSE {mse:.3e} rel-L2 {l2:.3e} max-abs {float(d.abs().max()):.3e}",
          flush=True)
    assert bool(torch.isfinite(out.float()).all())
    assert mse < mse_bound and l2 < l2_bound
    o = np_f32(out)
    nblk = N // 128
    blocks = [0, nblk // 2, nblk - 2, nblk - 1]
    for h in (0, 31):
        hk = h // 4
        sl = lambda a, lo, hi: a[:, lo:hi]
        qh, kh, vh = sl(c["q"], h, h + 1), sl(c["k"], hk, hk + 1), sl(c["v"], hk, hk + 1)
        if okw is None:
            # W > 0: the hybrid partition without vertical lines
            ref = O.unified_prefill_fp64(qh, kh, vh, W, blocks=blocks)
            ref_abs = O.unified_prefill_fp64(qh, kh, vh, W, abs_v=True, blocks=blocks)
            rows = np.concatenate([np.arange(b * 128, (b + 1) * 128) for b in blocks])
        else:
            vi = sl(c["vidx_np"], h, h + 1)
            exp_vi = O.compute_vertical_indices(qh, kh, W, RHO)
            assert np.array_equal(vi, exp_vi), f"vertical indices of head {h}"
            res = O.hybrid_prefill_fp64(qh, kh, vh, vi, W, blocks=blocks, fp8_detail=True, **okw)
            rows = np.concatenate([np.arange(b * 128, (b + 1) * 128) for b in blocks])
            if okw.get("pv_mode") == "fp8":
                ref, slack, exact_rows = res
                ref_abs = O.hybrid_prefill_fp64(qh, kh, vh, vi, W, blocks=blocks, abs_v=True, **okw)
            else:
                ref = res
                ref_abs = O.hybrid_prefill_fp64(qh, kh, vh, vi, W, blocks=blocks, abs_v=True, **okw)
        got = o[0, h, rows]
        r = ref[0, 0, rows]
        ra = ref_abs[0, 0, rows]
        diff = np.abs(got - r)
        if okw is not None and okw.get("pv_mode") == "fp8":
            # rows whose running maximum is exact round P' like the oracle
            # (tight); the others may take the other e4m3 neighbour per weight
            ex = exact_rows[0, 0, rows]
            eps = slack[0, 0, rows] + 2.0 ** -13 * ra + 2.0 ** -15 * np.abs(r) + 1e-6
            bad_tight = bf16_bracket(got, r, eps) & ex[:, None]
            loose = ATOL + 2.0 ** -3 * ra + 2.0 ** -8 * np.abs(r)
            bad = bad_tight | ((diff > loose) & ~ex[:, None])
            print(f"  head {h}: {int(ex.sum())}/{len(ex)} rows with an exact running max", flush=True)
        else:
            bad = diff > ATOL + 2.0 ** -10 * ra + 2.0 ** -8 * np.abs(r)
        print(f"  head {h} blocks {blocks}: max-abs {float(diff.max()):.3e} "
              f"rel {float(diff.max() / np.abs(r).max()):.3e}", flush=True)
        assert not bad.any(), f"{name} head {h}: {int(bad.sum())} elements outside the bound"
