"""GPU parity of the vertical-line selector (hyq_vertical_select), the freeze
reorganisation (hyq_freeze_reorganise) and the D-stage cache built on them,
against the CPU oracle: indices, int4 codes, scales and bf16 segments
bit-exact; decode through the cache within 2e-3."""

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import cache_from_inputs as _cache_from_inputs, check_layer_state as _check_state, to_dev_bf16

pytestmark = pytest.mark.gpu


def _rand_bf16(rng, shape, scale=1.0):
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("B,HQ,HK,QL,KL,W,rho", [
    (2, 8, 2, 40, 300, 32, 0.1),      # GQA-native (kv_repeat 4)
    (1, 4, 4, 7, 200, 16, 0.2),       # non-GQA, tail shorter than W
    (1, 16, 1, 5, 1000, 64, 0.05),    # GQA 16
    (3, 2, 2, 64, 129, 128, 1.0),     # prefix of one token, rho = 1
    (1, 2, 2, 8, 16064, 64, 0.1),     # 1600 winners: several ranked per thread, keys cached in LDS
    (1, 2, 1, 16, 30064, 64, 0.1),    # 3000 winners: bitonic order, keys read from memory
    (2, 4, 2, 32, 5000, 64, 0.05),    # GQA 2 (two heads per packed column group)
    (1, 6, 2, 32, 5000, 64, 0.05),    # GQA 3 (padded to four: a padding column per group)
    (1, 16, 2, 32, 3000, 64, 0.05),   # GQA 8
])
def test_selector_prefill_variant_bit_exact(B, HQ, HK, QL, KL, W, rho):
    from hyquant_amd.vertical import compute_vertical_indices
    print(f"select B={B} HQ={HQ} HK={HK} QL={QL} KL={KL} W={W} rho={rho}", flush=True)
    rng = np.random.default_rng(B * 1000 + KL)
    q = _rand_bf16(rng, (B, HQ, QL, 128))
    k = _rand_bf16(rng, (B, HK, KL, 128), 2.0)
    got = compute_vertical_indices(to_dev_bf16(q, "cuda"), to_dev_bf16(k, "cuda"), W, rho, kv_repeat=HQ // HK)
    exp = O.compute_vertical_indices(q, k, W, rho, kv_repeat=HQ // HK)
    assert got.shape == exp.shape
    assert np.array_equal(got.cpu().numpy(), exp)


@pytest.mark.parametrize("R", [1, 4])
def test_selector_query_rows_not_16_byte_aligned(R):
    """Query views whose rows are 4- but not 16-byte aligned take the
    channel-pair mean kernel (qmean_kernel), contiguous ones the 16-byte one
    (qmean16_kernel): both against the oracle, for the per-query-head (R = 1)
    and the group-mean (R = kv_repeat) selector."""
    from hyquant_amd.vertical import compute_vertical_indices, freeze_vertical_indices
    rng = np.random.default_rng(11 + R)
    B, HK, QL, P, W = 2, 2, 48, 700, 32
    HQ = HK * (R if R > 1 else 4)
    q = _rand_bf16(rng, (B, HQ, QL, 128))
    k = _rand_bf16(rng, (B, HK, P, 128), 2.0)
    wide = np.zeros((B, HQ, QL, 130), np.float32)
    wide[..., 2:] = q
    qv = to_dev_bf16(wide, "cuda")[..., 2:]           # row stride 130, base 4 bytes past 16-byte alignment
    assert qv.data_ptr() % 16 != 0 and qv.stride(2) % 8 != 0
    kd = to_dev_bf16(k, "cuda")
    if R == 1:
        exp = O.compute_vertical_indices(q, k, W, 0.1, kv_repeat=HQ // HK)
        got_v = compute_vertical_indices(qv, kd, W, 0.1, kv_repeat=HQ // HK)
        got_c = compute_vertical_indices(to_dev_bf16(q, "cuda"), kd, W, 0.1, kv_repeat=HQ // HK)
    else:
        tail = q[:, :, -W:]
        exp = O.compute_vertical_indices(O.group_mean_query(tail, HK), k, W, 0.1)
        got_v = freeze_vertical_indices(qv[:, :, -W:], kd, W, 0.1, R)
        got_c = freeze_vertical_indices(to_dev_bf16(tail, "cuda"), kd, W, 0.1, R)
    assert np.array_equal(got_v.cpu().numpy(), exp)
    assert np.array_equal(got_c.cpu().numpy(), exp)


def test_selector_ties_and_negative_zero():
    from hyquant_amd.vertical import compute_vertical_indices
    rng = np.random.default_rng(5)
    q = np.ones((1, 1, 2, 128), np.float32)
    k = np.zeros((1, 1, 600, 128), np.float32)
    k[0, 0, ::7] = 1.0 / 128                           # many exact ties (score 1)
    k[0, 0, 5::11, :64] = -1.0 / 128                   # score -0.5
    k[0, 0, 3, :64], k[0, 0, 3, 64:] = 1.0, -1.0       # exact zero
    k[0, 0, 4] = -0.0                                  # negative zero
    got = compute_vertical_indices(to_dev_bf16(q, "cuda"), to_dev_bf16(k, "cuda"), 100, 0.3)
    exp = O.compute_vertical_indices(q, k, 100, 0.3)
    assert np.array_equal(got.cpu().numpy(), exp)
    # the tied block comes out in ascending index order
    first = got.cpu().numpy()[0, 0, :10]
    assert list(first) == sorted(first)


@pytest.mark.parametrize("case", ["large_query_mean", "small_query_mean", "overflowing_rows",
                                  "wide_key_spread", "top_k_above_certified", "wide_spread_many_winners"])
def test_selector_certification_paths(case):
    """bf16 models score on the matrix cores with a certified error bound and
    recompute uncertain keys that can be selected.  Inputs that take the
    other paths, each bit-exact against the oracle (prefill-time call with
    GQA 4, and the freeze-time group-mean call):
      large / small query mean: a key head whose mean has entries above 2^60
        or nonzero ones below 2^-60 is scored in float64;
      overflowing rows: key rows of magnitude 2^100 leave the bound's range
        (largest key stored, recomputed when a candidate);
      wide key spread: rows scaled by 2^-30 .. 2^30, so the winners' keys span
        more than the counting rank covers (radix select and sort);
      top_k above certified: rho = 0.97, more winners than certified keys
        (every uncertain key recomputed, then the exact selection);
      wide spread, many winners: both of the last two."""
    from hyquant_amd.vertical import compute_vertical_indices, freeze_vertical_indices
    print(f"certification path {case}", flush=True)
    rng = np.random.default_rng(sum(map(ord, case)))
    B, HQ, HK, QL, W = 1, 8, 2, 64, 64
    KL = 4096 + W
    rho = 0.97 if case in ("top_k_above_certified", "wide_spread_many_winners") else 0.05
    q = rng.standard_normal((B, HQ, QL, 128)).astype(np.float32)
    k = (rng.standard_normal((B, HK, KL, 128)) + 1.5 * rng.standard_normal((1, HK, 1, 128))).astype(np.float32)
    if case == "large_query_mean":
        q[0, 1] *= 2.0 ** 70
    elif case == "small_query_mean":
        q[0, 5] *= 2.0 ** -70
    elif case == "overflowing_rows":
        k[0, 0, rng.choice(KL - W, 40, replace=False)] *= 2.0 ** 100
    elif case in ("wide_key_spread", "wide_spread_many_winners"):
        k *= 2.0 ** rng.integers(-30, 31, size=(B, HK, KL, 1))
    q, k = O.bf16_round(q), O.bf16_round(k)
    qd, kd = to_dev_bf16(q, "cuda"), to_dev_bf16(k, "cuda")
    got = compute_vertical_indices(qd, kd, W, rho, kv_repeat=HQ // HK)
    exp = O.compute_vertical_indices(q, k, W, rho, kv_repeat=HQ // HK)
    assert np.array_equal(got.cpu().numpy(), exp)
    P = KL - W
    got_f = freeze_vertical_indices(qd[:, :, -W:], kd[:, :, :P], W, rho, HQ // HK)
    exp_f = O.compute_vertical_indices(O.group_mean_query(q[:, :, -W:], HK), k[:, :, :P], W, rho)
    assert np.array_equal(got_f.cpu().numpy(), exp_f)


@pytest.mark.parametrize("cfg", [dict(B=1, HQ=32, HKV=8, N=1024), dict(B=2, HQ=32, HKV=8, N=8192),
                                 dict(B=2, HQ=64, HKV=8, N=4096), dict(B=1, HQ=32, HKV=2, N=16384)])
def test_selector_freeze_variant_and_prefill_on_config_inputs(cfg):
    from hyquant_amd.vertical import compute_vertical_indices, freeze_vertical_indices
    print(f"select config {cfg}", flush=True)
    W = 128 if cfg["N"] <= 8192 else 256
    inp = O.make_decode_inputs(W=W, S=4, seed=7, **cfg)
    G = cfg["HQ"] // cfg["HKV"]
    qt = to_dev_bf16(inp.query_tail, "cuda")
    kd = to_dev_bf16(inp.keys, "cuda")
    P = cfg["N"] - W
    got = freeze_vertical_indices(qt, kd[:, :, :P], W, 0.05, G)
    exp = O.compute_vertical_indices(O.group_mean_query(inp.query_tail, cfg["HKV"]), inp.keys[:, :, :P], W, 0.05)
    assert np.array_equal(got.cpu().numpy(), exp)
    got_q = compute_vertical_indices(qt, kd, W, 0.05, kv_repeat=G)
    exp_q = O.compute_vertical_indices(inp.query_tail, inp.keys, W, 0.05, kv_repeat=G)
    assert np.array_equal(got_q.cpu().numpy(), exp_q)


@pytest.mark.parametrize("cfg", [dict(B=1, HQ=32, HKV=8, N=1024, S=37), dict(B=2, HQ=32, HKV=8, N=8192, S=64)])
def test_cache_freeze_flush_decode(cfg):
    print(f"cache {cfg}", flush=True)
    inp = O.make_decode_inputs(W=128, seed=11, **cfg)
    layer = _cache_from_inputs(inp)
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, inp.HQ // inp.HKV)
    torch.cuda.synchronize()
    _check_state(layer, st)
    # staging: S tokens, then enough to cross one flush
    kn, vn = to_dev_bf16(inp.k_new, "cuda"), to_dev_bf16(inp.v_new, "cuda")
    layer.append_staging(kn, vn)
    O.append_staging(st, inp.k_new, inp.v_new)
    rng = np.random.default_rng(3)
    extra_k = _rand_bf16(rng, (cfg["B"], cfg["HKV"], 130, 128), 1.4)
    extra_v = _rand_bf16(rng, (cfg["B"], cfg["HKV"], 130, 128))
    for i in range(0, 130, 1):                   # one token per step, as in decode
        layer.append_staging(to_dev_bf16(extra_k[:, :, i:i + 1], "cuda"), to_dev_bf16(extra_v[:, :, i:i + 1], "cuda"))
    O.append_staging(st, extra_k, extra_v)
    torch.cuda.synchronize()
    _check_state(layer, st)
    assert layer.get_seq_length() == cfg["N"] + cfg["S"] + 130
    q = to_dev_bf16(inp.q_dec, "cuda").reshape(cfg["B"], cfg["HQ"], 1, 128)
    out = layer.decode_attention(q, inp.HQ // inp.HKV).reshape(-1, 128).float().cpu().numpy()
    ref = O.decode_fp64_state(inp.q_dec, st, inp.HQ // inp.HKV)
    err = float(np.max(np.abs(out - ref)))
    print(f"cache decode max-abs {err:.3e}", flush=True)
    assert err <= 2e-3


BIT_PAIRS = [(4, 4), (4, 2), (2, 4), (8, 8), (2, 2), (4, 8), (8, 4), (2, 8), (8, 2)]


@pytest.mark.parametrize("kb,vb", BIT_PAIRS)
def test_cache_freeze_every_bit_pair_bit_exact_and_decode(kb, vb):
    """Every (k_bits, v_bits) pair the mode table and the decode accept
    (src/ops/d_stage_kv_cache.py:167-168 quantises K and V with their own
    widths): freeze bit-exact, then decode through the cache."""
    print(f"cache freeze K{kb}V{vb}", flush=True)
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, W=128, S=9, seed=12)
    layer = _cache_from_inputs(inp, k_bits=kb, v_bits=vb)
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, 4, k_bits=kb, v_bits=vb)
    layer.append_staging(to_dev_bf16(inp.k_new, "cuda"), to_dev_bf16(inp.v_new, "cuda"))
    O.append_staging(st, inp.k_new, inp.v_new)
    torch.cuda.synchronize()
    _check_state(layer, st)
    q = to_dev_bf16(inp.q_dec, "cuda").reshape(1, 32, 1, 128)
    out = layer.decode_attention(q, 4).reshape(-1, 128).float().cpu().numpy()
    ref = O.decode_fp64_state(inp.q_dec, st, 4)
    err = float(np.max(np.abs(out - ref)))
    print(f"  K{kb}V{vb} cache decode max-abs {err:.3e}", flush=True)
    # P' = bf16(p * s_v) is rounded by the reference kernel too (F8): at most
    # 2^-9 sum p|v| / l, plus half a bf16 ulp of the output
    ref_abs = O.decode_fp64_state(inp.q_dec, st, 4, abs_v=True)
    assert np.all(np.abs(out - ref) <= 2e-3 + 2.0 ** -9 * ref_abs + 2.0 ** -8 * np.abs(ref))


def test_cache_short_prompt_no_prefix():
    inp = O.make_decode_inputs(B=1, HQ=8, HKV=2, N=100, W=128, S=3, seed=13)
    layer = _cache_from_inputs(inp)
    assert layer.k_quant_packed.shape[1] == 0 and layer.k_window.shape[1] == 100
    layer.append_staging(to_dev_bf16(inp.k_new, "cuda"), to_dev_bf16(inp.v_new, "cuda"))
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, 4)
    O.append_staging(st, inp.k_new, inp.v_new)
    q = to_dev_bf16(inp.q_dec, "cuda").reshape(1, 8, 1, 128)
    out = layer.decode_attention(q, 4).reshape(-1, 128).float().cpu().numpy()
    assert float(np.max(np.abs(out - O.decode_fp64_state(inp.q_dec, st, 4)))) <= 2e-3


@pytest.mark.parametrize("kv", BIT_PAIRS)
def test_cache_save_load_resumes_bit_identically(tmp_path, kv):
    """A frozen cache written to disk and read back decodes exactly like the
    original, before and after the staging ring flushes into the prefix."""
    from hyquant_amd.d_stage_kv_cache import DStageKVCache
    print(f"cache save/load K{kv[0]}V{kv[1]}", flush=True)
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, W=128, S=37, seed=14)
    G = inp.HQ // inp.HKV
    cache = DStageKVCache(num_layers=2, k_bits=kv[0], v_bits_fn=lambda i: kv[1], window_size=inp.W,
                          top_ratio=inp.rho)
    kd, vd = to_dev_bf16(inp.keys, "cuda"), to_dev_bf16(inp.values, "cuda")
    layer = cache.get_layer(0)
    cache.update(kd, vd, 0)
    layer.save_query_tail(to_dev_bf16(inp.query_tail, "cuda"))
    layer.freeze(kv_repeat=G)
    cache.update(to_dev_bf16(inp.k_new, "cuda"), to_dev_bf16(inp.v_new, "cuda"), 0)
    cache.update(kd[:, :, :50], vd[:, :, :50], 1)              # layer 1 still in prefill
    path = str(tmp_path / "cache.safetensors")
    cache.save(path)
    back = DStageKVCache.load(path)
    assert back.get_layer(1).phase == "prefill" and torch.equal(back.get_layer(1)._keys, kd[:, :, :50])
    q = to_dev_bf16(inp.q_dec, "cuda").reshape(1, inp.HQ, 1, 128)
    a = cache.get_layer(0).decode_attention(q, G)
    b = back.get_layer(0).decode_attention(q, G)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    rng = np.random.default_rng(4)
    ek = to_dev_bf16(_rand_bf16(rng, (1, inp.HKV, 100, 128), 1.4), "cuda")
    ev = to_dev_bf16(_rand_bf16(rng, (1, inp.HKV, 100, 128)), "cuda")
    for c in (cache, back):                                  # 37 + 100 tokens: one flush
        for i in range(100):
            c.update(ek[:, :, i:i + 1], ev[:, :, i:i + 1], 0)
    la, lb = cache.get_layer(0), back.get_layer(0)
    assert la._kstore.n == lb._kstore.n and la._staging_ptr == lb._staging_ptr == 9
    assert torch.equal(la.k_quant_packed, lb.k_quant_packed) and torch.equal(la.v_scale, lb.v_scale)
    a = la.decode_attention(q, G)
    b = lb.decode_attention(q, G)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert back.get_seq_length(0) == cache.get_seq_length(0) == inp.N + 37 + 100


@pytest.mark.parametrize("N", [600, 263208])
def test_freeze_bad_indices_stay_inside_the_outputs(N):
    """hyq_freeze_reorganise with repeated and out-of-range top-k indices (an
    ABI precondition violation): an index outside [0, n - w) yields a zero
    row, nothing is written past the n - w - top_k compact rows, and the
    rows that are written are the right ones (ascending unselected positions).
    N = 263208: a prefix of 263144 positions, past the rows whose bitmap is
    built in one workgroup's LDS (262144)."""
    from hyquant_amd import _lib
    print(f"freeze bad indices N={N}", flush=True)
    rng = np.random.default_rng(17)
    HK, W, T = 2, 64, 20
    P = N - W
    k = _rand_bf16(rng, (1, HK, N, 128))
    v = _rand_bf16(rng, (1, HK, N, 128))
    idx = np.stack([rng.permutation(P)[:T] for _ in range(HK)]).astype(np.int64)
    idx[0, 3] = idx[0, 2]             # a repeat: one position marked, T - 1 distinct
    idx[1, 5] = P + 7                 # a window position: out of [0, P)
    idx[1, 6] = -4                    # negative
    dev = torch.device("cuda")
    kd, vd = to_dev_bf16(k, dev), to_dev_bf16(v, dev)
    nc = P - T
    GUARD = 64
    kp = torch.full((HK, nc + GUARD, 64), 0x5A, dtype=torch.int8, device=dev)
    vp = torch.full((HK, nc + GUARD, 64), 0x5A, dtype=torch.int8, device=dev)
    ks = torch.full((HK, nc + GUARD), 7.0, dtype=torch.float16, device=dev)
    vs = torch.full((HK, nc + GUARD), 7.0, dtype=torch.float16, device=dev)
    kt = torch.empty(HK, T, 128, dtype=torch.bfloat16, device=dev)
    vt = torch.empty_like(kt)
    kw = torch.empty(HK, W, 128, dtype=torch.bfloat16, device=dev)
    vw = torch.empty_like(kw)
    ti = torch.from_numpy(idx).to(dev)
    L = _lib.lib()
    ws = torch.empty(max(L.hyq_freeze_workspace_size(HK, P), 256), dtype=torch.uint8, device=dev)
    st = L.hyq_freeze_reorganise(
        kd.data_ptr(), kd.stride(0), kd.stride(1), kd.stride(2), vd.data_ptr(), vd.stride(0), vd.stride(1),
        vd.stride(2), 1, HK, N, 128, W, ti.data_ptr(), T, 4, 4, 0,
        kp.data_ptr(), kp.stride(0), kp.stride(1), vp.data_ptr(), vp.stride(0), vp.stride(1),
        ks.data_ptr(), ks.stride(0), vs.data_ptr(), vs.stride(0),
        kt.data_ptr(), kt.stride(0), kt.stride(1), vt.data_ptr(), vt.stride(0), vt.stride(1),
        kw.data_ptr(), kw.stride(0), kw.stride(1), vw.data_ptr(), vw.stride(0), vw.stride(1),
        ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "freeze")
    torch.cuda.synchronize()
    assert bool((kp[:, nc:] == 0x5A).all()) and bool((vp[:, nc:] == 0x5A).all())
    assert bool((ks[:, nc:] == 7.0).all()) and bool((vs[:, nc:] == 7.0).all())
    ktn = kt.float().cpu().numpy()
    assert not ktn[1, 5].any() and not ktn[1, 6].any()
    assert np.array_equal(ktn[0, 3], k[0, 0, idx[0, 3]])
    for h in range(HK):
        sel = np.zeros(P, bool)
        good = idx[h][(idx[h] >= 0) & (idx[h] < P)]
        sel[good] = True
        rest = np.nonzero(~sel)[0][:nc]
        rp, rs = O.quantize_per_token(k[0, h][rest][None], 4)
        assert np.array_equal(kp[h, :nc].cpu().numpy(), rp[0])
        assert np.array_equal(ks[h, :nc].cpu().numpy().view(np.uint16), rs[0].view(np.uint16))


@pytest.mark.parametrize("P,rho,HQ,HK", [
    (65600, 0.05, 2, 1),     # past the 16-bit index: 64-bit composites, T = 3280 sorted in LDS
    (100000, 0.1, 1, 1),     # T = 10000 > 8192: 64-bit composites, 16384-entry bitonic sort in LDS
    (100000, 0.2, 1, 1),     # T = 20000: the sort buffer exceeds LDS and lives in the workspace
    (60000, 0.7, 1, 1),      # 32-bit composites, T = 42000: workspace sort
])
def test_selector_long_prefix_many_winners_bit_exact(P, rho, HQ, HK):
    """compute_vertical_indices past the 65536-position / 8192-winner range
    (the reference's torch.topk has no such limit, src/patch/_common.py:187-189):
    bf16 scores of random data tie often, so the lower-index rule is
    exercised throughout."""
    from hyquant_amd.vertical import compute_vertical_indices
    W = 64
    print(f"select long P={P} rho={rho} HQ={HQ} HK={HK}", flush=True)
    rng = np.random.default_rng(P + int(100 * rho))
    q = _rand_bf16(rng, (1, HQ, 16, 128))
    k = _rand_bf16(rng, (1, HK, P + W, 128), 2.0)
    got = compute_vertical_indices(to_dev_bf16(q, "cuda"), to_dev_bf16(k, "cuda"), W, rho, kv_repeat=HQ // HK)
    exp = O.compute_vertical_indices(q, k, W, rho, kv_repeat=HQ // HK)
    assert got.shape == exp.shape and exp.shape[-1] == O.top_k_count(P, rho)
    assert np.array_equal(got.cpu().numpy(), exp)


def test_freeze_long_prefix_bit_exact():
    """The freeze over a 70000-position prefix (the freeze-time selector past
    the 16-bit index range), bit-exact."""
    print("freeze long prefix", flush=True)
    inp = O.make_decode_inputs(B=1, HQ=8, HKV=2, N=70400, W=128, S=5, seed=21)
    layer = _cache_from_inputs(inp)
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, 4)
    torch.cuda.synchronize()
    _check_state(layer, st)


def test_fp16_model_selector_freeze_flush_decode():
    """An fp16 model through the cache (src/ops/d_stage_kv_cache.py:82-217 with
    fp16 K/V): the prefill-time and freeze-time selections bit-exact with the
    oracle's fp16 branch (means and scores rounded to fp16), the frozen
    segments and codes bit-exact, a flush of fp16 staging tokens bit-exact,
    and the decode (fp16 q, fp16 segments, fp16 out) within 2e-3 of the
    float64 oracle on the bf16-rounded segments the reference's kernel sees."""
    from hyquant_amd.d_stage_kv_cache import DStageLayerCache
    from hyquant_amd.vertical import compute_vertical_indices
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=2048, W=128, S=37, seed=17)
    G = inp.HQ // inp.HKV
    rng = np.random.default_rng(17)
    f16 = lambda a: (a * (1 + rng.uniform(-2 ** -8, 2 ** -8, a.shape))).astype(np.float16).astype(np.float32)
    keys, values, qt = f16(inp.keys), f16(inp.values), f16(inp.query_tail)
    kn, vn, qd = f16(inp.k_new), f16(inp.v_new), f16(inp.q_dec)
    dev = torch.device("cuda")
    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.float16).to(dev)
    print("fp16 model cache", flush=True)
    got_q = compute_vertical_indices(d(qt), d(keys), inp.W, inp.rho, kv_repeat=G)
    exp_q = O.compute_vertical_indices(qt, keys, inp.W, inp.rho, kv_repeat=G, fp16=True)
    assert np.array_equal(got_q.cpu().numpy(), exp_q)
    layer = DStageLayerCache(0, k_bits=4, v_bits=4, window_size=inp.W, top_ratio=inp.rho)
    layer.update_prefill(d(keys), d(values))
    layer.save_query_tail(d(qt))
    layer.freeze(kv_repeat=G)
    st = O.freeze(keys, values, qt, inp.W, inp.rho, G, fp16=True)
    torch.cuda.synchronize()
    assert layer.k_topk.dtype == torch.float16
    # the fp16 selection differs from the bf16 one on these inputs
    st_b = O.freeze(keys, values, qt, inp.W, inp.rho, G)
    print(f"  fp16 / bf16 top-k sets differ: {not np.array_equal(st.topk_idx, st_b.topk_idx)}", flush=True)
    _check_state(layer, st)
    layer.append_staging(d(kn), d(vn))
    O.append_staging(st, kn, vn)
    extra_k = f16(_rand_bf16(rng, (1, inp.HKV, 100, 128), 1.4))
    extra_v = f16(_rand_bf16(rng, (1, inp.HKV, 100, 128)))
    for i in range(100):
        layer.append_staging(d(extra_k[:, :, i:i + 1]), d(extra_v[:, :, i:i + 1]))
    O.append_staging(st, extra_k, extra_v)
    torch.cuda.synchronize()
    _check_state(layer, st)
    out = layer.decode_attention(d(qd).reshape(1, inp.HQ, 1, 128), G)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    out = out.reshape(-1, 128).float().cpu().numpy()
    rb = O.bf16_round
    st.k_topk, st.v_topk, st.k_window, st.v_window = rb(st.k_topk), rb(st.v_topk), rb(st.k_window), rb(st.v_window)
    st.k_ring, st.v_ring = rb(st.k_ring), rb(st.v_ring)
    ref = O.decode_fp64_state(rb(qd), st, G)
    err = float(np.max(np.abs(out - ref)))
    print(f"  fp16 cache decode max-abs {err:.3e}", flush=True)
    assert err <= 2e-3
