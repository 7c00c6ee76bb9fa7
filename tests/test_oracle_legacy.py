"""Pins of the oracle's legacy decode format (src/ops/d_stage_cache.py):
hand-decoded bytes, every byte value against per-bit arithmetic, the group
mapping of the [G, D] scales, and the legacy decode against the per-token
decode over the same values."""

import numpy as np

from oracle import hyq_oracle as O


def test_legacy_unpack_known_bytes():
    # int4: high nibble = even channel, value u - 8
    assert O.legacy_unpack(np.array([[0xA3]], np.uint8), 4).tolist() == [[2.0, -5.0]]
    assert O.legacy_unpack(np.array([[0x08, 0x80]], np.uint8), 4).tolist() == [[-8.0, 0.0, 0.0, -8.0]]
    assert O.legacy_unpack(np.array([[0xFF]], np.uint8), 4).tolist() == [[7.0, 7.0]]
    # int2: channel 4k+i in bits (7-2i, 6-2i), value u - 1.5
    assert O.legacy_unpack(np.array([[0xE4]], np.uint8), 2).tolist() == [[1.5, 0.5, -0.5, -1.5]]
    assert O.legacy_unpack(np.array([[0x1B]], np.uint8), 2).tolist() == [[-1.5, -0.5, 0.5, 1.5]]


def test_legacy_unpack_every_byte():
    b = np.arange(256, dtype=np.uint8)[:, None]
    v4 = O.legacy_unpack(b, 4)
    v2 = O.legacy_unpack(b, 2)
    for x in range(256):
        bits = [(x >> i) & 1 for i in range(8)]
        hi = bits[4] + 2 * bits[5] + 4 * bits[6] + 8 * bits[7]
        lo = bits[0] + 2 * bits[1] + 4 * bits[2] + 8 * bits[3]
        assert v4[x].tolist() == [hi - 8, lo - 8]
        crumbs = [bits[6] + 2 * bits[7], bits[4] + 2 * bits[5], bits[2] + 2 * bits[3], bits[0] + 2 * bits[1]]
        assert v2[x].tolist() == [c - 1.5 for c in crumbs]


def test_legacy_values_group_mapping():
    rng = np.random.default_rng(0)
    BH, N, D = 2, 300, 8
    packed = rng.integers(0, 256, (BH, N, D // 2), dtype=np.uint8)
    scale = rng.uniform(-2, 2, (BH, 3, D)).astype(np.float16)
    vals = O.legacy_values(packed, scale, 4)
    codes = O.legacy_unpack(packed, 4)
    for (h, n, d) in [(0, 0, 0), (1, 127, 7), (0, 128, 3), (1, 255, 0), (0, 256, 5), (1, 299, 6)]:
        assert vals[h, n, d] == float(codes[h, n, d]) * float(scale[h, n // 128, d])


def test_legacy_dequant_bf16_signs_and_rounding():
    # u = 8 (value 0) with a negative scale gives -0; odd products round to even
    packed = np.array([[[0x88, 0x9F]]], np.uint8)                 # values 0, 0, 1, 7
    scale = np.array([[[-1.0, 1.0, 1.0 + 2.0 ** -10, 3.0 + 2.0 ** -9]]], np.float16)
    bits = O.legacy_dequant_bf16(packed, scale, 4)
    assert bits[0, 0, 0] == 0x8000 and bits[0, 0, 1] == 0x0000
    # 1 * (1 + 2^-10): below half an ulp of bf16 at 1 -> 1.0
    assert bits[0, 0, 2] == 0x3F80
    # 7 * (3 + 2^-9) = 21 + 7 * 2^-9 = 21.013671875 -> bf16 ulp at 16..32 is 1/8: 21.0
    assert bits[0, 0, 3] == O.f32_to_bf16_bits(np.array([21.0], np.float32))[0]


def _segments(rng, BHK, T, S, W, D):
    f = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    return f(T), f(T), f(S), f(S), f(W), f(W)


def test_legacy_decode_equals_per_token_decode_on_the_same_values():
    """Unit scales: an int4 legacy prefix is the per-token prefix with codes
    u - 8 and scale 1; an int2 legacy prefix (values u - 1.5) is a per-token
    int4 prefix with codes 2u - 3 and scale 0.5."""
    rng = np.random.default_rng(1)
    BHK, R, N, D = 3, 4, 200, 16
    q = O.bf16_round(rng.standard_normal((BHK * R, D)).astype(np.float32))
    segs = _segments(rng, BHK, 5, 3, 8, D)
    ones = np.ones((BHK, 2, D), np.float16)
    for bits in (4, 2):
        packed = rng.integers(0, 256, (BHK, N, D * bits // 8), dtype=np.uint8)
        legacy = O.legacy_decode_fp64(q, packed, packed, ones, ones, *segs, k_bits=bits, v_bits=bits, kv_repeat=R)
        vals = O.legacy_unpack(packed, bits)
        if bits == 4:
            codes, sc = vals.astype(np.int8), np.ones((BHK, N), np.float16)
        else:
            codes, sc = (2 * vals).astype(np.int8), np.full((BHK, N), 0.5, np.float16)
        pt = O.pack_int4(codes)
        per_token = O.decode_fp64(q, pt, pt, sc, sc, *segs, k_bits=4, v_bits=4, kv_repeat=R)
        np.testing.assert_allclose(legacy, per_token, rtol=0, atol=1e-12)
