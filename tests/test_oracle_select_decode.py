"""Pins for the oracle's vertical-line selector (src/patch/_common.py:144-190),
freeze reorganisation (src/ops/d_stage_kv_cache.py:106-189), staging ring
(:195-217) and four-segment decode (src/ops/decode_d_stage.py:916-1005,
src/ops/d_stage_kv_cache.py:309-354)."""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import hyq_oracle as O
from tests._exact import to_bf16, to_fp16


def _rand_bf16(rng, shape, scale=1.0):
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def _brute_select(q, k, W, rho, kv_repeat=1, rnd=to_bf16):
    """Selector by exact rational arithmetic and a full Python sort (rnd: the
    model dtype's rounding)."""
    B, HQ, QL, D = q.shape
    P = max(0, k.shape[2] - W)
    tail = min(W, QL)
    T = min(max(1, math.ceil(P * rho)), P)
    out = np.zeros((B, HQ, T), np.int64)
    for b in range(B):
        for h in range(HQ):
            hk = h // kv_repeat if k.shape[1] != HQ else h
            qm = [rnd(sum(Fraction(float(q[b, h, QL - tail + i, d])) for i in range(tail)) / tail) for d in range(D)]
            sc = []
            for p in range(P):
                s = rnd(sum(qm[d] * Fraction(float(k[b, hk, p, d])) for d in range(D)))
                sc.append((-s, p))
            sc.sort()
            out[b, h] = [p for _, p in sc[:T]]
    return out


@pytest.mark.parametrize("kv_repeat", [1, 2])
def test_selector_brute_force(kv_repeat):
    rng = np.random.default_rng(10)
    HQ = 2
    q = _rand_bf16(rng, (1, HQ, 5, 8))
    k = _rand_bf16(rng, (1, HQ // kv_repeat, 30, 8), 2.0)
    got = O.compute_vertical_indices(q, k, 4, 0.2, kv_repeat=kv_repeat)
    exp = _brute_select(q, k, 4, 0.2, kv_repeat)
    assert got.shape == (1, HQ, 6)
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("kv_repeat", [1, 2])
def test_selector_fp16_model_brute_force(kv_repeat):
    """An fp16 model's selector: fp16 means and scores (torch computes
    query_tail.mean and the matmul in the model dtype), brute-forced with
    exact rationals; scores are spread so that fp16 and bf16 rankings differ."""
    rng = np.random.default_rng(20)
    HQ = 2
    q = (rng.standard_normal((1, HQ, 5, 8))).astype(np.float16).astype(np.float32)
    k = (rng.standard_normal((1, HQ // kv_repeat, 40, 8)) * 2).astype(np.float16).astype(np.float32)
    got = O.compute_vertical_indices(q, k, 4, 0.3, kv_repeat=kv_repeat, fp16=True)
    exp = _brute_select(q, k, 4, 0.3, kv_repeat, rnd=to_fp16)
    assert np.array_equal(got, exp)
    # the group mean of the freeze-time call, in fp16
    qt = (rng.standard_normal((1, 4, 3, 8)) * 3).astype(np.float16).astype(np.float32)
    gm = O.group_mean_query(qt, 2, fp16=True)
    for h in range(2):
        for t in range(3):
            for d in range(8):
                exp_m = to_fp16((Fraction(float(qt[0, 2 * h, t, d])) + Fraction(float(qt[0, 2 * h + 1, t, d]))) / 2)
                assert Fraction(float(gm[0, h, t, d])) == exp_m


def test_selector_fp16_ties_and_signed_zero():
    """Ties and -0 in fp16 keys: same rules as bf16."""
    q = np.ones((1, 1, 1, 2), np.float32)
    k = np.zeros((1, 1, 6, 2), np.float32)
    k[0, 0, 0] = [1.0, -1.0]
    k[0, 0, 2] = [-0.0, -0.0]
    k[0, 0, 1] = [-1.0, 0.0]
    k[0, 0, 3] = [1000.0, 1e-3]     # 1000.001 rounds to 1000 in fp16 (a tie with row 4)
    k[0, 0, 4] = [1000.0, 0.0]
    got = O.compute_vertical_indices(q, k, window_size=1, top_ratio=0.8, fp16=True)
    assert got.tolist() == [[[3, 4, 0, 2]]]


def test_selector_ties_lower_index_first():
    # identical key rows -> identical scores; ties must come out by index
    q = np.ones((1, 1, 2, 4), np.float32)
    k = np.zeros((1, 1, 12, 4), np.float32)
    k[0, 0, [1, 3, 6, 7]] = 1.0      # score 4 (four-way tie)
    k[0, 0, [0, 2]] = 2.0            # score 8 (two-way tie)
    k[0, 0, 5] = -1.0                # score -4
    got = O.compute_vertical_indices(q, k, window_size=2, top_ratio=0.6)
    # P = 10, T = 6: 0,2 (score 8) then 1,3,6,7 (score 4)
    assert got.tolist() == [[[0, 2, 1, 3, 6, 7]]]


def test_selector_negative_zero_ties_positive_zero():
    q = np.ones((1, 1, 1, 2), np.float32)
    k = np.zeros((1, 1, 5, 2), np.float32)
    k[0, 0, 0] = [1.0, -1.0]        # +0 - ... = 0 exactly
    k[0, 0, 2] = [-0.0, -0.0]       # -0
    k[0, 0, 1] = [-1.0, 0.0]
    got = O.compute_vertical_indices(q, k, window_size=1, top_ratio=0.75)
    assert got.tolist() == [[[0, 2, 3]]]


def test_selector_rho_one_selects_all_and_empty_prefix():
    rng = np.random.default_rng(11)
    q = _rand_bf16(rng, (2, 3, 4, 8))
    k = _rand_bf16(rng, (2, 3, 9, 8))
    got = O.compute_vertical_indices(q, k, 4, 1.0)
    assert got.shape == (2, 3, 5)
    assert np.array_equal(np.sort(got, axis=-1), np.broadcast_to(np.arange(5), (2, 3, 5)))
    assert O.compute_vertical_indices(q, k, 9, 0.05).shape == (2, 3, 0)
    assert O.top_k_count(7936, 0.05) == 397 and O.top_k_count(768, 0.05) == 39


def test_selector_planted_lines_known_answer():
    inp = O.make_decode_inputs(B=1, HQ=8, HKV=2, N=512, W=64, S=5, seed=0)
    G = inp.HQ // inp.HKV
    kp = inp.keys[:, :, :512 - 64]
    q_kv = O.group_mean_query(inp.query_tail, inp.HKV)
    idx = O.compute_vertical_indices(q_kv, kp, 64, 0.05)
    T = O.top_k_count(512 - 128, 0.05)
    assert idx.shape == (1, 2, T)
    for h in range(2):
        eligible = set(inp.planted[0, h][inp.planted[0, h] < 512 - 128].tolist())
        n = min(T, len(eligible))
        assert n >= T - 2
        # the planted lines outrank every other key: they fill the first slots
        if len(eligible) >= T:
            assert set(idx[0, h].tolist()) <= eligible
        else:
            assert set(idx[0, h, :n].tolist()) == eligible
    # prefill-time (per Q head, GQA-native) selection also finds planted lines
    idx_q = O.compute_vertical_indices(inp.query_tail, inp.keys, 64, 0.05, kv_repeat=G)
    for h in range(inp.HQ):
        assert set(idx_q[0, h].tolist()) <= set(inp.planted[0, h // G].tolist())


def test_exact_dot_matches_rational():
    rng = np.random.default_rng(12)
    qm = _rand_bf16(rng, (3, 16), 0.1)
    k = _rand_bf16(rng, (3, 7, 16), 3.0)
    got = O.dot_bf16_exact(qm, k)
    for i in range(3):
        for p in range(7):
            s = to_bf16(sum(Fraction(float(qm[i, d])) * Fraction(float(k[i, p, d])) for d in range(16)))
            assert Fraction(float(got[i, p])) == s


def test_freeze_partition_invariants_and_bruteforce():
    rng = np.random.default_rng(13)
    B, HQ, HKV, N, D, W = 2, 4, 2, 40, 8, 6
    keys = _rand_bf16(rng, (B, HKV, N, D), 2.0)
    vals = _rand_bf16(rng, (B, HKV, N, D))
    qt = _rand_bf16(rng, (B, HQ, W, D))
    st = O.freeze(keys, vals, qt, W, 0.1, HQ // HKV)
    P = N - W
    T = O.top_k_count(P - W, 0.1)
    assert st.topk_idx.shape == (B, HKV, T)
    assert st.k_packed.shape == (B * HKV, P - T, D // 2)
    # the selector sees the prefix and drops another W: indices < N - 2W (F3)
    assert st.topk_idx.max() < N - 2 * W
    q_kv = O.group_mean_query(qt, HKV)
    assert np.array_equal(st.topk_idx, _brute_select(q_kv, keys[:, :, :P], W, 0.1))
    for b in range(B):
        for h in range(HKV):
            tk = st.topk_idx[b, h].tolist()
            cp = st.compact_idx[b, h].tolist()
            assert not (set(tk) & set(cp))
            assert sorted(tk + cp) == list(range(P))
            assert cp == sorted(cp)
            bh = b * HKV + h
            assert np.array_equal(st.k_topk[bh], keys[b, h, tk])
            assert np.array_equal(st.v_topk[bh], vals[b, h, tk])
            assert np.array_equal(st.k_window[bh], keys[b, h, N - W:])
            # the compact rows are the quantised prefix rows in position order
            kp, ks = O.quantize_per_token(keys[b, h, cp][None], 4)
            assert np.array_equal(st.k_packed[bh], kp[0])
            assert np.array_equal(st.k_scale[bh], ks[0])


def test_freeze_short_prefix_and_no_vert():
    rng = np.random.default_rng(14)
    keys = _rand_bf16(rng, (1, 2, 10, 8))
    vals = _rand_bf16(rng, (1, 2, 10, 8))
    st = O.freeze(keys, vals, _rand_bf16(rng, (1, 2, 3, 8)), 16, 0.05, 1)
    assert st.k_packed.shape == (2, 0, 4) and st.k_window.shape == (2, 10, 8)
    st = O.freeze(keys, vals, _rand_bf16(rng, (1, 2, 3, 8)), 4, 0.05, 1)
    # prefix 6 <= window 4? P' = 6 - 4 = 2 -> one vertical line
    assert st.k_topk.shape == (2, 1, 8) and st.k_packed.shape == (2, 5, 4)
    st = O.freeze(keys, vals, None, 4, 0.05, 1)
    assert st.k_topk.shape == (2, 0, 8) and st.k_packed.shape == (2, 6, 4)


def test_staging_flush():
    rng = np.random.default_rng(15)
    keys = _rand_bf16(rng, (1, 2, 300, 8))
    st = O.freeze(keys, keys, _rand_bf16(rng, (1, 2, 4, 8)), 4, 0.05, 1)
    n0 = st.k_packed.shape[1]
    new = _rand_bf16(rng, (1, 2, 133, 8))
    O.append_staging(st, new, new)
    assert st.ring_ptr == 5 and st.k_packed.shape[1] == n0 + 128
    kp, ks = O.quantize_per_token(new.reshape(2, 133, 8)[:, :128], 4)
    assert np.array_equal(st.k_packed[:, n0:], kp)
    assert np.array_equal(st.k_scale[:, n0:], ks)
    assert np.array_equal(st.k_staging, new.reshape(2, 133, 8)[:, 128:])


# --- decode -----------------------------------------------------------------


def _empty(BH, D):
    return (np.zeros((BH, 0, D // 2), np.int8), np.zeros((BH, 0), np.float16))


def test_decode_no_prefix_equals_torch_sdpa():
    import torch
    rng = np.random.default_rng(20)
    BHQ, R, D = 8, 4, 16
    BHK = BHQ // R
    q = _rand_bf16(rng, (BHQ, D))
    segs = [_rand_bf16(rng, (BHK, n, D)) for n in (3, 5, 7)]
    vsegs = [_rand_bf16(rng, (BHK, n, D)) for n in (3, 5, 7)]
    kp, ks = _empty(BHK, D)
    out = O.decode_fp64(q, kp, kp, ks, ks, segs[0], vsegs[0], segs[1], vsegs[1], segs[2], vsegs[2], kv_repeat=R)
    K = torch.from_numpy(np.concatenate(segs, 1).astype(np.float64)).repeat_interleave(R, 0)
    V = torch.from_numpy(np.concatenate(vsegs, 1).astype(np.float64)).repeat_interleave(R, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q.astype(np.float64))[:, None, None], K[:, None], V[:, None])[:, 0, 0]
    assert np.allclose(out, ref.numpy(), atol=1e-12, rtol=0)


def test_decode_single_token_returns_value_and_dequant():
    rng = np.random.default_rng(21)
    D = 8
    v = O.bf16_round(np.array([[[7, -7, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5]]], np.float32))
    kp, ks = O.quantize_per_token(_rand_bf16(rng, (1, 1, D)), 4)
    vp, vs = O.quantize_per_token(v, 4)
    e = np.zeros((1, 0, D), np.float32)
    out = O.decode_fp64(_rand_bf16(rng, (1, D)), kp, vp, ks, vs, e, e, e, e, e, e)
    assert out.tolist() == [[7, -7, 4, -4, 0, 2, 2, 0]]


def test_decode_segment_permutation_invariance():
    rng = np.random.default_rng(22)
    BHQ, D = 4, 16
    q = _rand_bf16(rng, (BHQ, D))
    a, b, c = (_rand_bf16(rng, (BHQ, n, D)) for n in (4, 6, 3))
    va, vb, vc = (_rand_bf16(rng, (BHQ, n, D)) for n in (4, 6, 3))
    kp, ks = O.quantize_per_token(_rand_bf16(rng, (BHQ, 9, D)), 4)
    vp, vs = O.quantize_per_token(_rand_bf16(rng, (BHQ, 9, D)), 4)
    o1 = O.decode_fp64(q, kp, vp, ks, vs, a, va, b, vb, c, vc)
    o2 = O.decode_fp64(q, kp, vp, ks, vs, c, vc, a, va, b, vb)
    assert np.allclose(o1, o2, atol=1e-13)


def test_decode_gqa_equals_explicit_expansion():
    rng = np.random.default_rng(23)
    R, BHK, D = 4, 2, 16
    q = _rand_bf16(rng, (R * BHK, D))
    kp, ks = O.quantize_per_token(_rand_bf16(rng, (BHK, 9, D)), 4)
    vp, vs = O.quantize_per_token(_rand_bf16(rng, (BHK, 9, D)), 4)
    t = [_rand_bf16(rng, (BHK, n, D)) for n in (2, 2, 3, 3, 4, 4)]
    o1 = O.decode_fp64(q, kp, vp, ks, vs, *t, kv_repeat=R)
    rep = lambda a: np.repeat(a, R, axis=0)
    o2 = O.decode_fp64(q, rep(kp), rep(vp), rep(ks), rep(vs), *[rep(x) for x in t], kv_repeat=1)
    assert np.allclose(o1, o2, atol=1e-13)


def test_decode_state_and_bf16_eager_close():
    inp = O.make_decode_inputs(B=1, HQ=8, HKV=2, N=384, W=64, S=9, seed=1)
    st = O.build_decode_state(inp)
    assert st.k_staging.shape[1] == 9
    ref = O.decode_fp64_state(inp.q_dec, st, 4)
    eager = O.decode_bf16_eager(inp.q_dec, st, 4, inp.B)
    # the eager path rounds scores/probabilities to bf16: ~1e-2 relative
    assert np.max(np.abs(eager - ref)) < 0.02 * max(1.0, np.max(np.abs(ref)))
