"""GPU parity of the legacy decode format (src/ops/d_stage_cache.py) against
the CPU oracle: the prefix dequantisation bit-exact (hyq_legacy_dequant), the
four legacy decode entry points within the decode tolerance of the float64
restatement."""

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import to_dev_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _legacy_inputs(rng, BHK, N, D, bits, group=128, neg=True):
    packed = rng.integers(0, 256, (BHK, N, D * bits // 8), dtype=np.uint8)
    G = (N + group - 1) // group
    lo = -0.12 if neg else 0.02
    scale = rng.uniform(lo, 0.12, (BHK, G, D)).astype(np.float16)
    return packed, scale


@pytest.mark.parametrize("bits,N", [(4, 300), (4, 128), (2, 257), (2, 1)])
def test_legacy_dequant_bit_exact(bits, N):
    from hyquant_amd.d_stage_cache import legacy_dequantize
    print(f"legacy dequant bits={bits} N={N}", flush=True)
    rng = np.random.default_rng(bits * 100 + N)
    BHK, D = 3, 128
    packed, scale = _legacy_inputs(rng, BHK, N, D, bits)
    scale[0, 0, :4] = 0.0                                     # zero scales: signed zeros
    exp = O.legacy_dequant_bf16(packed, scale, bits)
    got = legacy_dequantize(torch.from_numpy(packed).cuda(), torch.from_numpy(scale).cuda(), D, bits)
    got_bits = got.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got_bits, exp)
    # a scale view with a padded group stride and an output view inside a larger buffer
    wide = torch.zeros(BHK, scale.shape[1], 2 * D, dtype=torch.float16, device="cuda")
    wide[:, :, :D] = torch.from_numpy(scale).cuda()
    buf = torch.full((BHK, N + 7, D), 7.0, dtype=torch.bfloat16, device="cuda")
    legacy_dequantize(torch.from_numpy(packed).cuda(), wide[:, :, :D], D, bits, out=buf[:, 3:3 + N])
    assert np.array_equal(buf[:, 3:3 + N].contiguous().view(torch.int16).cpu().numpy().view(np.uint16), exp)
    assert bool((buf[:, :3] == 7.0).all()) and bool((buf[:, 3 + N:] == 7.0).all())


def _check(name, out, ref, ref_abs):
    out = out.float().cpu().numpy().reshape(ref.shape)
    diff = np.abs(out - ref)
    bound = ATOL + 2.0 ** -9 * ref_abs + 2.0 ** -8 * np.abs(ref)
    print(f"{name}: max-abs {diff.max():.3e}, max diff/bound {(diff / bound).max():.3f}", flush=True)
    assert (diff <= bound).all(), name


@pytest.mark.parametrize("entry,kb,vb,R", [
    ("fused", 4, 4, 4), ("splitk", 4, 4, 4), ("mma", 4, 4, 4), ("mma", 4, 2, 8), ("mma", 2, 4, 1), ("mma", 2, 2, 4),
    ("fused", 4, 4, 1), ("mma", 4, 4, 8), ("mma", 4, 4, 16),
])
def test_legacy_decode_vs_oracle(entry, kb, vb, R):
    import hyquant_amd.d_stage_cache as L
    print(f"legacy decode {entry} K{kb}V{vb} R={R}", flush=True)
    rng = np.random.default_rng(kb * 10 + vb + R)
    B, HKV, N, D, T, S, W = 2, 2, 700, 128, 37, 5, 64
    BHK = B * HKV
    kp, ks = _legacy_inputs(rng, BHK, N, D, kb)
    vp, vs = _legacy_inputs(rng, BHK, N, D, vb)
    f = lambda n, s=1.0: O.bf16_round((rng.standard_normal((BHK, n, D)) * s).astype(np.float32))
    kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
    q = O.bf16_round(rng.standard_normal((B * HKV * R, D)).astype(np.float32))
    d = lambda a: to_dev_bf16(a, "cuda")
    u = lambda a: torch.from_numpy(a).cuda()
    qd = d(q).view(B, HKV * R, 1, D)
    args = (qd, u(kp), u(vp), u(ks), u(vs), d(kt), d(vt), d(kst), d(vst), d(kw), d(vw))
    if entry == "fused":
        out = L.fused_decode_attention_k4v4(*args, kv_repeat=R)
    elif entry == "splitk":
        out = L.splitk_decode_attention_k4v4(*args, kv_repeat=R, split_size=512)
    else:
        out = L.splitk_decode_attention_k4v4_mma(*args, kv_repeat=R, k_bits=kb, v_bits=vb)
    assert out.shape == (B, HKV * R, 1, D) and out.dtype == torch.bfloat16
    oargs = (q, kp, vp, ks, vs, kt, vt, kst, vst, kw, vw)
    ref = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, bf16_operands=True)
    ref_abs = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, bf16_operands=True, abs_v=True)
    _check(f"{entry} K{kb}V{vb}", out, ref, ref_abs)
    # and close to the unrounded legacy math (the FFMA variants' fp32 operands)
    exact = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R)
    assert np.abs(out.float().cpu().numpy().reshape(exact.shape) - exact).max() <= 4 * ATOL


@pytest.mark.parametrize("kb,vb", [(4, 4), (2, 2)])
def test_legacy_direct_long_prefix(kb, vb):
    """A 140000-token legacy prefix through the direct path (the codes read
    in the decode, no bf16 copy): the pieces are doubled until they fit the
    merge tables, and the result stays within the bound of the fp64
    restatement."""
    import hyquant_amd.d_stage_cache as L
    print(f"legacy direct long prefix K{kb}V{vb}", flush=True)
    rng = np.random.default_rng(140 + kb + vb)
    BHK, R, N, D, T, S, W = 1, 4, 140000, 128, 300, 17, 64
    kp, ks = _legacy_inputs(rng, BHK, N, D, kb)
    vp, vs = _legacy_inputs(rng, BHK, N, D, vb)
    f = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
    q = O.bf16_round(rng.standard_normal((BHK * R, D)).astype(np.float32))
    d = lambda a: to_dev_bf16(a, "cuda")
    u = lambda a: torch.from_numpy(a).cuda()
    out = L.splitk_decode_attention_k4v4_mma(d(q).view(1, BHK * R, 1, D), u(kp), u(vp), u(ks), u(vs), d(kt),
                                             d(vt), d(kst), d(vst), d(kw), d(vw), kv_repeat=R, k_bits=kb, v_bits=vb)
    oargs = (q, kp, vp, ks, vs, kt, vt, kst, vst, kw, vw)
    ref = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, bf16_operands=True)
    ref_abs = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, bf16_operands=True, abs_v=True)
    _check(f"direct long prefix K{kb}V{vb}", out, ref, ref_abs)


@pytest.mark.parametrize("kb,vb", [(4, 4), (4, 2), (2, 4), (2, 2)])
def test_legacy_direct_matches_dequantise_first(kb, vb):
    """The direct path dequantises each tile in registers to the bf16 values
    legacy_dequantize writes (up to an exact power of two); decoding those
    bf16 rows through the hybrid kernel's bf16 path gives the same attention
    up to the order of the split-K sums (here within 2^-10 of the output
    scale)."""
    import hyquant_amd.d_stage_cache as L
    from hyquant_amd.decode_d_stage import _decode
    print(f"legacy direct vs dequantise-first K{kb}V{vb}", flush=True)
    rng = np.random.default_rng(404 + 10 * kb + vb)
    BHK, R, N, D, T, S, W = 4, 4, 3000, 128, 150, 9, 64
    kp, ks = _legacy_inputs(rng, BHK, N, D, kb)
    vp, vs = _legacy_inputs(rng, BHK, N, D, vb)
    f = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
    q = O.bf16_round(rng.standard_normal((BHK * R, D)).astype(np.float32))
    d = lambda a: to_dev_bf16(a, "cuda")
    u = lambda a: torch.from_numpy(a).cuda()
    direct = L.splitk_decode_attention_k4v4_mma(d(q).view(1, BHK * R, 1, D), u(kp), u(vp), u(ks), u(vs), d(kt),
                                                d(vt), d(kst), d(vst), d(kw), d(vw), kv_repeat=R, k_bits=kb, v_bits=vb)
    kf = torch.empty(BHK, N + T, D, dtype=torch.bfloat16, device="cuda")
    vf = torch.empty_like(kf)
    L.legacy_dequantize(u(kp), u(ks), D, kb, out=kf[:, :N])
    L.legacy_dequantize(u(vp), u(vs), D, vb, out=vf[:, :N])
    kf[:, N:].copy_(d(kt))
    vf[:, N:].copy_(d(vt))
    none8 = torch.empty(BHK, 0, D // 2, dtype=torch.int8, device="cuda")
    none16 = torch.empty(BHK, 0, dtype=torch.float16, device="cuda")
    first = _decode(d(q), none8, none8, none16, none16, kf, vf, d(kst), d(vst), d(kw), d(vw), 4, 4, R, None, 0,
                    None, None)
    a, b = direct.float().reshape(BHK * R, D), first.float()
    assert (a - b).abs().max().item() <= 2.0 ** -10 * max(1.0, b.abs().max().item())


def test_legacy_decode_config1_shape():
    """Config-1 shape (B=1, 32q/8kv, 8K prefix) through the legacy entry point."""
    import hyquant_amd.d_stage_cache as L
    print("legacy decode config-1 shape", flush=True)
    rng = np.random.default_rng(77)
    HKV, R, N, D, T, S, W = 8, 4, 7667, 128, 397, 64, 128
    kp, ks = _legacy_inputs(rng, HKV, N, D, 4)
    vp, vs = _legacy_inputs(rng, HKV, N, D, 4)
    f = lambda n: O.bf16_round(rng.standard_normal((HKV, n, D)).astype(np.float32))
    kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
    q = O.bf16_round(rng.standard_normal((HKV * R, D)).astype(np.float32))
    d = lambda a: to_dev_bf16(a, "cuda")
    u = lambda a: torch.from_numpy(a).cuda()
    out = L.fused_decode_attention_k4v4(d(q).view(1, HKV * R, 1, D), u(kp), u(vp), u(ks), u(vs), d(kt), d(vt),
                                        d(kst), d(vst), d(kw), d(vw), kv_repeat=R)
    oargs = (q, kp, vp, ks, vs, kt, vt, kst, vst, kw, vw)
    ref = O.legacy_decode_fp64(*oargs, kv_repeat=R, bf16_operands=True)
    ref_abs = O.legacy_decode_fp64(*oargs, kv_repeat=R, bf16_operands=True, abs_v=True)
    _check("config-1 shape", out, ref, ref_abs)
    # a second call gives the same bits
    out2 = L.fused_decode_attention_k4v4(d(q).view(1, HKV * R, 1, D), u(kp), u(vp), u(ks), u(vs), d(kt), d(vt),
                                         d(kst), d(vst), d(kw), d(vw), kv_repeat=R)
    assert torch.equal(out, out2)


def test_legacy_decode_empty_segments_and_no_prefix():
    import hyquant_amd.d_stage_cache as L
    rng = np.random.default_rng(5)
    BHK, R, D, W = 2, 4, 128, 32
    q = O.bf16_round(rng.standard_normal((BHK * R, D)).astype(np.float32))
    kw = O.bf16_round(rng.standard_normal((BHK, W, D)).astype(np.float32))
    vw = O.bf16_round(rng.standard_normal((BHK, W, D)).astype(np.float32))
    e8 = torch.empty(BHK, 0, D // 2, dtype=torch.uint8, device="cuda")
    es = torch.empty(BHK, 0, D, dtype=torch.float16, device="cuda")
    eb = torch.empty(BHK, 0, D, dtype=torch.bfloat16, device="cuda")
    d = lambda a: to_dev_bf16(a, "cuda")
    out = L.fused_decode_attention_k4v4(d(q).view(1, BHK * R, 1, D), e8, e8, es, es, eb, eb, eb, eb, d(kw), d(vw),
                                        kv_repeat=R)
    z8 = np.zeros((BHK, 0, D // 2), np.uint8)
    zs = np.zeros((BHK, 0, D), np.float16)
    zb = np.zeros((BHK, 0, D), np.float32)
    ref = O.legacy_decode_fp64(q, z8, z8, zs, zs, zb, zb, zb, zb, kw, vw, kv_repeat=R)
    ref_abs = O.legacy_decode_fp64(q, z8, z8, zs, zs, zb, zb, zb, zb, kw, vw, kv_repeat=R, abs_v=True)
    _check("window only", out, ref, ref_abs)


def test_d_stage_decode_attention_per_token_format():
    """Legacy path A: per-token int4 K (and int4 / int2 V) prefix dequantised
    to fp16 then bf16, one KV head per query head, [B, H, W, D] window."""
    from hyquant_amd.d_stage_cache import d_stage_decode_attention, decode_4seg_attention
    assert decode_4seg_attention is d_stage_decode_attention
    rng = np.random.default_rng(9)
    B, H, N, D, T, S, W = 2, 3, 400, 128, 20, 6, 48
    BH = B * H
    for vb in (4, 2):
        k = O.bf16_round(rng.standard_normal((BH, N, D)).astype(np.float32))
        v = O.bf16_round(rng.standard_normal((BH, N, D)).astype(np.float32))
        kp, ks = O.quantize_per_token(k, 4)
        vp, vs = O.quantize_per_token(v, vb)
        f = lambda n: O.bf16_round(rng.standard_normal((BH, n, D)).astype(np.float32))
        kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
        q = O.bf16_round(rng.standard_normal((BH, D)).astype(np.float32))
        d = lambda a: to_dev_bf16(a, "cuda")
        u = lambda a: torch.from_numpy(a).cuda()
        out = d_stage_decode_attention(d(q).view(B, H, 1, D), u(kp), u(vp), u(ks), u(vs), d(kt), d(vt), d(kst),
                                       d(vst), d(kw).view(B, H, W, D), d(vw).view(B, H, W, D), v_bits=vb)
        assert out.shape == (B, H, 1, D)
        # dequantize_k_int4_channel(...).to(bf16): fp16(code * scale) rounded to bf16
        kd = O.bf16_round(O.dequantize_per_token(kp, ks, 4).astype(np.float32))
        vd = O.bf16_round(O.dequantize_per_token(vp, vs, vb).astype(np.float32))
        e8 = np.zeros((BH, 0, D // 2), np.int8)
        e16 = np.zeros((BH, 0), np.float16)
        Kb = np.concatenate([kd, kt], 1)
        Vb = np.concatenate([vd, vt], 1)
        ref = O.decode_fp64(q, e8, e8, e16, e16, Kb, Vb, kst, vst, kw, vw)
        ref_abs = O.decode_fp64(q, e8, e8, e16, e16, Kb, Vb, kst, vst, kw, vw, abs_v=True)
        _check(f"d_stage_decode_attention V{vb}", out, ref, ref_abs)


def test_legacy_entry_points_reject_bad_arguments():
    import hyquant_amd.d_stage_cache as L
    D = 128
    q = torch.zeros(1, 4, 1, D, dtype=torch.bfloat16, device="cuda")
    kp = torch.zeros(1, 10, D // 2, dtype=torch.uint8, device="cuda")
    ks = torch.zeros(1, 1, D, dtype=torch.float16, device="cuda")
    eb = torch.zeros(1, 0, D, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(1, 4, D, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError):
        L.fused_decode_attention_k4v4(q.half(), kp, kp, ks, ks, eb, eb, eb, eb, w, w, kv_repeat=4)
    with pytest.raises(AssertionError):
        L.splitk_decode_attention_k4v4_mma(q, kp, kp, ks, ks, eb, eb, eb, eb, w, w, kv_repeat=4, k_bits=8)
    with pytest.raises(ValueError):       # too few scale groups for the prefix
        L.legacy_dequantize(torch.zeros(1, 200, D // 2, dtype=torch.uint8, device="cuda"), ks, D, 4)


@pytest.mark.parametrize("vb", [4, 2])
def test_legacy_direct_every_code_and_scale(vb):
    """The direct path's in-register dequantisation against the oracle for
    every V code (16 int4 or 4 int2 values) with every finite fp16 scale.
    Each head holds a one-token prefix and no bf16 rows, so its softmax
    weight is exactly 1 and its output row is the dequantised V row: heads x
    128 channels carry the codes x 63488 (code, scale) pairs.  Zeros are
    compared without their sign (the product with P = 1 accumulates onto
    +0).  K of the same width shares the code conversion."""
    import hyquant_amd.d_stage_cache as L
    print(f"legacy direct: every int{vb} code and finite fp16 scale", flush=True)
    D = 128
    ncode = 1 << vb
    b = np.arange(65536, dtype=np.uint32)
    fin = b[((b >> 10) & 0x1F) != 0x1F].astype(np.uint16)          # 63488 finite fp16
    BHK = fin.size * ncode // D
    p = np.arange(BHK * D).reshape(BHK, D)
    code = (p % ncode).astype(np.uint8)
    vs = fin[p // ncode].reshape(BHK, 1, D).view(np.float16)
    if vb == 4:
        vp = ((code[:, 0::2] << 4) | code[:, 1::2]).reshape(BHK, 1, D // 2)
    else:      # channel 4j + i in bits 7-2i..6-2i of byte j
        vp = ((code[:, 0::4] << 6) | (code[:, 1::4] << 4) | (code[:, 2::4] << 2) | code[:, 3::4]).reshape(BHK, 1, D // 4)
    rng = np.random.default_rng(9)
    kp = rng.integers(0, 256, (BHK, 1, D // 2), dtype=np.uint8)
    ks = np.ones((BHK, 1, D), np.float16)
    q = O.bf16_round(rng.standard_normal((BHK, D)).astype(np.float32))
    eb = torch.empty(BHK, 0, D, dtype=torch.bfloat16, device="cuda")
    u = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    out = L.splitk_decode_attention_k4v4_mma(to_dev_bf16(q, "cuda").view(1, BHK, 1, D), u(kp), u(vp), u(ks), u(vs),
                                             eb, eb, eb, eb, eb, eb, kv_repeat=1, k_bits=4, v_bits=vb)
    got = out.view(BHK, D).view(torch.int16).cpu().numpy().view(np.uint16)
    exp = O.legacy_dequant_bf16(vp, vs, vb)[:, 0, :]
    assert np.array_equal(np.where(got == 0x8000, 0, got), np.where(exp == 0x8000, 0, exp))


@pytest.mark.parametrize("kb,vb", [(4, 2), (2, 4)])
def test_legacy_direct_c_abi_group_and_strides(kb, vb):
    """hyq_decode_legacy through the C ABI with a 48-token scale group (the
    16-token tiles never cross a group; 512-token pieces start inside one),
    code rows and scale rows padded past their data, and a ragged 1000-token
    prefix, against the fp64 restatement with the same group."""
    import ctypes
    from hyquant_amd import _lib
    print(f"legacy direct C ABI group 48 K{kb}V{vb}", flush=True)
    L = _lib.lib()
    rng = np.random.default_rng(48 + kb)
    BHK, R, N, D, T, S, W, group = 3, 4, 1000, 128, 21, 5, 40, 48
    G = -(-N // group)
    kp, _ = _legacy_inputs(rng, BHK, N, D, kb)
    vp, _ = _legacy_inputs(rng, BHK, N, D, vb)
    ks = rng.uniform(-0.12, 0.12, (BHK, G, D)).astype(np.float16)
    vs = rng.uniform(-0.12, 0.12, (BHK, G, D)).astype(np.float16)
    kbuf = np.zeros((BHK, N, 16 * kb + 16), np.uint8)
    kbuf[:, :, :16 * kb] = kp
    vbuf = np.zeros((BHK, N, 16 * vb + 4), np.uint8)
    vbuf[:, :, :16 * vb] = vp
    ksbuf = np.zeros((BHK, G, D + 8), np.float16)
    ksbuf[:, :, :D] = ks
    vsbuf = np.zeros((BHK, G, D + 8), np.float16)
    vsbuf[:, :, :D] = vs
    f = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    kt, vt, kst, vst, kw, vw = f(T), f(T), f(S), f(S), f(W), f(W)
    q = O.bf16_round(rng.standard_normal((BHK * R, D)).astype(np.float32))
    u = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    d = lambda a: to_dev_bf16(a, "cuda")
    keep = [u(kbuf), u(vbuf), u(ksbuf), u(vsbuf), d(kt), d(vt), d(kst), d(vst), d(kw), d(vw), d(q)]
    out = torch.empty(BHK * R, D, dtype=torch.bfloat16, device="cuda")
    p = _lib.LegacyParams()
    p.q, p.q_stride = keep[10].data_ptr(), D
    p.out, p.out_stride = out.data_ptr(), D
    p.k_codes, p.kc_stride_bh, p.kc_stride_n = keep[0].data_ptr(), N * (16 * kb + 16), 16 * kb + 16
    p.v_codes, p.vc_stride_bh, p.vc_stride_n = keep[1].data_ptr(), N * (16 * vb + 4), 16 * vb + 4
    p.k_scale, p.ks_stride_bh, p.ks_stride_g = keep[2].data_ptr(), G * (D + 8), D + 8
    p.v_scale, p.vs_stride_bh, p.vs_stride_g = keep[3].data_ptr(), G * (D + 8), D + 8
    p.n, p.group, p.k_bits, p.v_bits = N, group, kb, vb
    for i, (sk, sv, n) in enumerate(((keep[4], keep[5], T), (keep[6], keep[7], S), (keep[8], keep[9], W))):
        p.seg_k[i], p.seg_v[i], p.seg_k_stride_bh[i], p.seg_v_stride_bh[i], p.seg_n[i] = (
            sk.data_ptr(), sv.data_ptr(), n * D, n * D, n)
    p.bh_kv, p.kv_repeat, p.head_dim, p.sm_scale = BHK, R, D, D ** -0.5
    need = L.hyq_decode_legacy_workspace_size(ctypes.byref(p))
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    st = L.hyq_decode_legacy(ctypes.byref(p), ws.data_ptr(), need, torch.cuda.current_stream().cuda_stream)
    assert st == 0, L.hyq_last_error()
    torch.cuda.synchronize()
    oargs = (q, kp, vp, ks, vs, kt, vt, kst, vst, kw, vw)
    ref = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, group=group, bf16_operands=True)
    ref_abs = O.legacy_decode_fp64(*oargs, k_bits=kb, v_bits=vb, kv_repeat=R, group=group, bf16_operands=True,
                                   abs_v=True)
    _check(f"C ABI group 48 K{kb}V{vb}", out, ref, ref_abs)
