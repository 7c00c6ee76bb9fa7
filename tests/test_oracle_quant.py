"""Pins for the oracle's per-token quantisation and int4/int2 packing
(src/ops/decode_d_stage.py:50-163): hand-computed known answers and exact
rational re-derivations, independent of the oracle's numpy code."""

from fractions import Fraction

import numpy as np
import pytest

from oracle import hyq_oracle as O
from tests._exact import fp16_bits, rint_half_even, to_fp16, to_fp32


def _bytes(a):
    return [int(b) & 0xFF for b in np.asarray(a).reshape(-1)]


def test_known_answer_unit_scale_and_nibble_order():
    # amax = 7 -> scale = fp16(1.0); codes = rint_half_even(x)
    x = np.array([[[7, -7, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5]]], np.float32)
    packed, scale = O.quantize_per_token(x, 4)
    assert scale.view(np.uint16)[0, 0] == 0x3C00
    # codes 7,-7 | 4,-4 | 0,2 | 2,0 ; even channel in the low nibble
    assert _bytes(packed) == [0x97, 0xC4, 0x20, 0x02]
    codes = O.unpack_int4(packed)
    assert codes.tolist() == [[[7, -7, 4, -4, 0, 2, 2, 0]]]


def test_known_answer_scale_rounding():
    # amax = 1 -> 1/7 in fp32 -> fp16 RNE = 0x3092 (1.142578125 * 2^-3)
    x = np.array([[[1.0, -0.5, 0.25, 0.0]]], np.float32)
    _, scale = O.quantize_per_token(x, 4)
    assert scale.view(np.uint16)[0, 0] == 0x3092


def test_known_answer_zero_token_subnormal_scale():
    x = np.zeros((1, 1, 8), np.float32)
    packed, scale = O.quantize_per_token(x, 4)
    # fp16(fp32(1e-5) / 7) = 24 * 2^-24 (subnormal)
    assert scale.view(np.uint16)[0, 0] == 0x0018
    assert _bytes(packed) == [0, 0, 0, 0]


def test_known_answer_overflowing_scale():
    # amax / 7 > 65504 -> fp16 +inf, every code 0 (x / inf = 0)
    x = np.array([[[999424.0, -5.0, 3.0, 1.0]]], np.float32)
    packed, scale = O.quantize_per_token(x, 4)
    assert scale.view(np.uint16)[0, 0] == 0x7C00
    assert _bytes(packed) == [0, 0]


def test_known_answer_int2():
    x = np.array([[[1.0, -1.0, 0.5, -0.5]]], np.float32)
    packed, scale = O.quantize_per_token(x, 2)
    assert scale.view(np.uint16)[0, 0] == 0x3C00
    assert _bytes(packed) == [0x0D]
    assert O.unpack_int2(packed).tolist() == [[[1, -1, 0, 0]]]


def test_int8_codes():
    x = np.array([[[127.0, -127.0, 63.5, 64.5]]], np.float32)
    codes, scale = O.quantize_per_token(x, 8)
    assert scale.view(np.uint16)[0, 0] == 0x3C00
    assert codes.tolist() == [[[127, -127, 64, 64]]]


def test_pack_all_nibble_pairs_roundtrip():
    a, b = np.meshgrid(np.arange(-8, 8), np.arange(-8, 8), indexing="ij")
    codes = np.stack([a.ravel(), b.ravel()], axis=-1).astype(np.int8)[None]
    packed = O.pack_int4(codes)
    # byte = (a & 15) | (b & 15) << 4 for every pair
    expect = [((int(p) & 15) | ((int(q) & 15) << 4)) for p, q in zip(a.ravel(), b.ravel())]
    assert _bytes(packed) == expect
    assert np.array_equal(O.unpack_int4(packed), codes)


def test_exact_rational_rederivation_random_tokens():
    """Every scale and code equals an exact rational evaluation of
    fp16(fp32(max(amax,1e-5)) / 7) and rint(x / scale) clamped."""
    rng = np.random.default_rng(1)
    x = O.bf16_round(rng.standard_normal((3, 5, 16)).astype(np.float32) * rng.uniform(0.01, 50, (3, 5, 1)).astype(np.float32))
    codes, scale = O.quantize_codes(x, 4)
    for i in range(3):
        for n in range(5):
            row = [Fraction(float(v)) for v in x[i, n]]
            amax = max(max(abs(v) for v in row), Fraction(float(np.float32(1e-5))))
            s32 = to_fp32(amax / 7)
            s16 = to_fp16(s32)
            assert scale[i, n].view(np.uint16) == fp16_bits(s16)
            for d, v in enumerate(row):
                c = min(7, max(-8, rint_half_even(to_fp32(v / s16))))
                assert codes[i, n, d] == c


def test_invariants_error_bound_and_code_range():
    rng = np.random.default_rng(2)
    x = O.bf16_round(rng.standard_normal((4, 64, 128)).astype(np.float32) * 3)
    packed, scale = O.quantize_per_token(x, 4)
    codes = O.unpack_int4(packed)
    assert codes.min() >= -7 and codes.max() <= 7  # -8 only in degenerate cases
    s = scale.astype(np.float64)[..., None]
    err = np.abs(codes * s - x.astype(np.float64))
    assert np.all(err <= s / 2 + 1e-12)
    # every token reaches |code| = 7 on its amax channel
    assert np.all(np.abs(codes).max(axis=-1) == 7)


def test_matches_torch_cpu_rounding():
    """numpy's fp16 conversion / rint agree with torch's on random bf16 data
    (the reference computes in torch)."""
    import torch
    rng = np.random.default_rng(3)
    x = O.bf16_round(rng.standard_normal((2, 33, 128)).astype(np.float32) * 2)
    codes, scale = O.quantize_codes(x, 4)
    xt = torch.from_numpy(x)
    st = (xt.abs().amax(dim=-1).clamp(min=1e-5) / 7).to(torch.float16)
    qt = (xt / st.float().unsqueeze(-1)).round().clamp(-8, 7).to(torch.int8)
    assert np.array_equal(st.numpy().view(np.uint16), scale.view(np.uint16))
    assert np.array_equal(qt.numpy(), codes)


def test_dequantize_fp16():
    x = np.array([[[7, -7, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5]]], np.float32)
    packed, scale = O.quantize_per_token(x, 4)
    deq = O.dequantize_per_token(packed, scale, 4)
    assert deq.tolist() == [[[7, -7, 4, -4, 0, 2, 2, 0]]]


def _fp16_rne_exact(v):
    """fp16 bits of the rational v, rounded to nearest even from first
    principles (normal and subnormal ranges, overflow to inf)."""
    import math
    from fractions import Fraction
    sign = 0x8000 if math.copysign(1.0, v) < 0 else 0        # -2 * 0.0 is -0.0
    v = Fraction(v)
    a = abs(v)
    if a == 0:
        return sign
    e = max(a.numerator.bit_length() - a.denominator.bit_length() + 1, -13)
    while Fraction(2) ** e <= a:       # normalise to 2^(e-1) <= a < 2^e (or the subnormal range)
        e += 1
    while e > -13 and Fraction(2) ** (e - 1) > a:
        e -= 1
    quantum = Fraction(2) ** (max(e, -13) - 11)                 # 11 significant bits; 2^-24 below 2^-14
    n = a / quantum
    r = n.numerator // n.denominator
    rem = n - r
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and r % 2 == 1):
        r += 1
    val = r * quantum
    if val >= 65520 or val > 65504:
        return sign | 0x7C00
    return sign | int(np.float16(float(val)).view(np.uint16))


def test_dequantize_against_exact_rounding_and_torch():
    """fp16(code * scale) for every code of 2, 4 and 8 bits and scales over the
    whole fp16 range (subnormal, normal, near overflow): against an exact
    rational round-to-nearest-even, and against the reference's own torch
    expression (q.float() * scale.float()).to(torch.float16)."""
    import torch
    rng = np.random.default_rng(21)
    scales = np.concatenate([np.exp(rng.uniform(np.log(6e-8), np.log(6.5e4), 60)),
                             [0.0, 6e-8, 6.1e-5, 65504.0, 1.0, 1 / 3]]).astype(np.float16)
    for nbits in (2, 4, 8):
        ncode = 2 ** nbits
        codes = np.arange(-(ncode // 2), ncode // 2, dtype=np.int8)
        D = max(8, ncode)
        reps = -(-D // len(codes))
        row = np.tile(codes, reps)[:D]
        c = np.broadcast_to(row, (1, len(scales), D)).astype(np.int8)
        if nbits == 4:
            packed = O.pack_int4(c)
        elif nbits == 2:
            packed = O.pack_int2(c)
        else:
            packed = c.copy()
        sc = scales[None, :]
        deq = O.dequantize_per_token(packed, sc, nbits).astype(np.float16).view(np.uint16)
        for i, s16 in enumerate(scales):
            for j in range(D):
                exp = _fp16_rne_exact(int(row[j]) * float(s16))
                assert deq[0, i, j] == exp, (nbits, float(s16), int(row[j]))
        qt = torch.from_numpy(O.unpack_codes(packed, nbits).astype(np.float32))
        ref = (qt * torch.from_numpy(sc).float().unsqueeze(-1)).to(torch.float16)
        assert np.array_equal(ref.numpy().view(np.uint16), deq)


def test_bad_bits():
    with pytest.raises(ValueError):
        O.quantize_per_token(np.zeros((1, 1, 8), np.float32), 3)


def test_bf16_round_ties_and_f64_single_rounding():
    # 1 + 2^-8 is a tie between 1 and 1 + 2^-7 -> even (1.0)
    assert O.bf16_round(np.array([1 + 2 ** -8], np.float32))[0] == 1.0
    assert O.bf16_round(np.array([1 + 3 * 2 ** -8], np.float32))[0] == 1 + 2 ** -6
    # f64 value just above a bf16 tie must round up although fp32 RNE would
    # land exactly on the tie (double-rounding trap)
    v = 1 + 2 ** -8 + 2 ** -40
    assert O.bf16_round_f64(np.array([v]))[0] == 1 + 2 ** -7
    assert O.bf16_round(np.array([v], np.float32))[0] == 1.0
