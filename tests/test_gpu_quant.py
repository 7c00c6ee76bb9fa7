"""GPU parity of per-token quantisation + packing (hyq_quant_pack) against the
CPU oracle: bit-exact codes, packed bytes and fp16 scales."""

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import to_dev_bf16

pytestmark = pytest.mark.gpu


def _special_tokens(D):
    rows = [
        np.zeros(D),                                  # subnormal scale, codes 0
        np.full(D, 999424.0),                         # scale overflows to +inf
        np.r_[7, -7, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5, np.zeros(D - 8)],  # ties
        np.r_[1e-30, np.zeros(D - 1)],                # below the 1e-5 clamp
        np.r_[-3.0, np.full(D - 1, 1.5)],             # negative amax
    ]
    return O.bf16_round(np.stack(rows).astype(np.float32))


@pytest.mark.parametrize("nbits", [4, 2, 8])
def test_quant_pack_bit_exact(nbits):
    rng = np.random.default_rng(100 + nbits)
    BH, N, D = 6, 77, 128
    x = O.bf16_round((rng.standard_normal((BH, N, D)) * rng.uniform(1e-3, 30, (BH, N, 1))).astype(np.float32))
    x[0, :5] = _special_tokens(D)
    print(f"quant nbits={nbits} shape={x.shape}", flush=True)
    import hyquant_amd as hq
    xd = to_dev_bf16(x, "cuda")
    packed, scale = hq.quantize_per_token(xd, nbits)
    torch.cuda.synchronize()
    rp, rs = O.quantize_per_token(x, nbits)
    assert np.array_equal(packed.cpu().numpy(), rp)
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.view(np.uint16))


def test_quant_pack_into_offset_window_and_strided_input():
    """Append semantics of the staging flush: write 128 tokens at an offset of a
    capacity buffer; input is a strided view of a wider ring."""
    import hyquant_amd as hq
    from hyquant_amd.decode_d_stage import quantize_into
    rng = np.random.default_rng(7)
    BH, D = 4, 128
    ring = O.bf16_round(rng.standard_normal((BH, 160, D)).astype(np.float32) * 2)
    ring_d = to_dev_bf16(ring, "cuda")
    cap = torch.full((BH, 1000, D // 2), 0x55, dtype=torch.int8, device="cuda")
    scl = torch.zeros(BH, 1000, dtype=torch.float16, device="cuda")
    quantize_into(ring_d[:, 16:144], 4, cap[:, 300:428], scl[:, 300:428])
    torch.cuda.synchronize()
    rp, rs = O.quantize_per_token(ring[:, 16:144], 4)
    assert np.array_equal(cap[:, 300:428].cpu().numpy(), rp)
    assert np.array_equal(scl[:, 300:428].cpu().numpy().view(np.uint16), rs.view(np.uint16))
    # nothing outside the window was touched
    assert bool((cap[:, :300] == 0x55).all()) and bool((cap[:, 428:] == 0x55).all())


def test_quant_config_inputs_bit_exact():
    """The benchmark distribution (outlier channels + planted lines), cfg0 size."""
    import hyquant_amd as hq
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, W=128, S=37, seed=0)
    for arr in (inp.keys, inp.values):
        x = arr.reshape(8, 1024, 128)
        packed, scale = hq.quantize_per_token(to_dev_bf16(x, "cuda"), 4)
        rp, rs = O.quantize_per_token(x, 4)
        assert np.array_equal(packed.cpu().numpy(), rp)
        assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("nbits", [4, 2, 8])
def test_quant_every_bf16_value_bit_exact(nbits):
    """Every bf16 value v with |v| <= amax, for 16 random token scales: all
    exact ties v / s = k + 1/2 and the values next to them are covered, so
    the kernel's quotient and rounding must agree with IEEE division and
    round-half-even everywhere."""
    rng = np.random.default_rng(70 + nbits)
    D = 128
    pos = (np.arange(0, 0x7F80, dtype=np.uint32) << 16).view(np.float32)   # finite bf16 >= 0
    amaxes = O.bf16_round(np.exp(rng.uniform(np.log(1e-4), np.log(1e3), 16)).astype(np.float32))
    toks = []
    for amax in amaxes:
        vals = pos[pos <= amax]
        vals = np.concatenate([vals, -vals])
        per = D - 1
        ntok = -(-len(vals) // per)
        body = np.zeros(ntok * per, np.float32)
        body[:len(vals)] = vals
        t = np.empty((ntok, D), np.float32)
        t[:, 0] = amax                                  # fixes the token's scale
        t[:, 1:] = body.reshape(ntok, per)
        toks.append(t)
    x = np.concatenate(toks)[None]
    print(f"quant exhaustive nbits={nbits} tokens={x.shape[1]}", flush=True)
    import hyquant_amd as hq
    packed, scale = hq.quantize_per_token(to_dev_bf16(x, "cuda"), nbits)
    torch.cuda.synchronize()
    rp, rs = O.quantize_per_token(x, nbits)
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(packed.cpu().numpy(), rp)


@pytest.mark.parametrize("nbits", [4, 2, 8])
@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
def test_quant_every_amax_bit_exact(nbits, dtype):
    """One token per positive finite 16-bit value a (every bf16, or every
    fp16 including subnormals), whose largest magnitude is a: the scale
    fp16(amax / qmax) and its reciprocal are formed without IEEE divisions
    in the kernel (a product with RN(1 / qmax), v_rcp_f32 with a Newton
    step), so every reachable amax and scale is compared with the oracle's
    IEEE arithmetic, codes included (the other channels are random values
    in [-a, a])."""
    rng = np.random.default_rng(500 + nbits + (dtype == "fp16"))
    D = 128
    if dtype == "bf16":
        a = (np.arange(1, 0x7F80, dtype=np.uint32) << 16).view(np.float32)
    else:
        a = np.arange(1, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    x = rng.uniform(-1.0, 1.0, (len(a), D)).astype(np.float32) * a[:, None]
    x[:, rng.integers(0, D)] = a
    x[::2, 0] = -a[::2]                                # negative amax on half of the tokens
    if dtype == "bf16":
        x = O.bf16_round(x)
        xd = to_dev_bf16(x[None], "cuda")
    else:
        x = x.astype(np.float16).astype(np.float32)
        xd = torch.from_numpy(x[None].astype(np.float16)).cuda()
    print(f"quant every amax nbits={nbits} {dtype} tokens={len(a)}", flush=True)
    import hyquant_amd as hq
    packed, scale = hq.quantize_per_token(xd, nbits)
    torch.cuda.synchronize()
    rp, rs = O.quantize_per_token(x[None], nbits)
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.view(np.uint16))
    assert np.array_equal(packed.cpu().numpy(), rp)


@pytest.mark.parametrize("nbits", [4, 2, 8])
def test_quant_pack_fp16_input_bit_exact(nbits):
    """quantize_per_token on fp16 tokens (src/ops/decode_d_stage.py:50-77
    takes bf16 or fp16: x.float() is exact for both): codes, bytes and scales
    bit-exact with the oracle on the same values, including fp16 subnormals
    and the largest finite fp16."""
    import hyquant_amd as hq
    rng = np.random.default_rng(300 + nbits)
    BH, N, D = 5, 93, 128
    x = (rng.standard_normal((BH, N, D)) * rng.uniform(1e-4, 300, (BH, N, 1))).astype(np.float16)
    x[0, 0] = 0
    x[0, 1, :] = np.float16(6.1e-5) * rng.integers(-3, 4, D)      # subnormal-scale tokens
    x[0, 2, 0] = np.float16(65504.0)
    x[0, 3, :8] = [7, -7, 3.5, -3.5, 0.5, 1.5, 2.5, -0.5]           # ties
    xf = x.astype(np.float32)
    packed, scale = hq.quantize_per_token(torch.from_numpy(x).cuda(), nbits)
    torch.cuda.synchronize()
    rp, rs = O.quantize_per_token(xf, nbits)
    assert np.array_equal(packed.cpu().numpy(), rp)
    assert np.array_equal(scale.cpu().numpy().view(np.uint16), rs.view(np.uint16))


@pytest.mark.parametrize("nbits", [4, 2, 8])
def test_dequant_bit_exact(nbits):
    """dequantize_per_token (hyq_dequant) against the oracle's fp16(code *
    scale) (src/ops/decode_d_stage.py:80-101): random packed bytes, so every
    code occurs (the most negative one too), and scales across the fp16
    range: subnormal, normal, products that overflow to inf and a zero."""
    import hyquant_amd as hq
    rng = np.random.default_rng(400 + nbits)
    BH, N, D = 7, 131, 128
    packed = rng.integers(-128, 128, size=(BH, N, 16 * nbits), dtype=np.int8)
    scale = np.exp(rng.uniform(np.log(1e-7), np.log(6e4), size=(BH, N))).astype(np.float16)
    scale[0, :4] = [0.0, np.float16(6e-8), np.float16(65504.0), np.float16(1.0)]
    codes = O.unpack_codes(packed, nbits)
    assert codes.min() == -(2 ** (nbits - 1)) and codes.max() == 2 ** (nbits - 1) - 1
    got = hq.dequantize_per_token(torch.from_numpy(packed).cuda(), torch.from_numpy(scale).cuda(), D, nbits)
    torch.cuda.synchronize()
    assert got.dtype == torch.float16 and tuple(got.shape) == (BH, N, D)
    exp = O.dequantize_per_token(packed, scale, nbits).astype(np.float16)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), exp.view(np.uint16))


def test_dequant_round_trip_of_quantised_cache():
    """quantize then dequantize on the device: |x - deq(x)| <= scale / 2 (plus
    the fp16 rounding of the product) on the benchmark distribution, and a
    strided (head-sliced) packed input gives the same bytes as a contiguous one."""
    import hyquant_amd as hq
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, W=128, S=37, seed=3)
    x = inp.keys.reshape(8, 1024, 128)
    xd = to_dev_bf16(x, "cuda")
    packed, scale = hq.quantize_per_token(xd, 4)
    deq = hq.dequantize_per_token(packed, scale, 128, 4).float().cpu().numpy()
    s = scale.float().cpu().numpy()[..., None]
    assert np.all(np.abs(x - deq) <= s / 2 + np.abs(deq) * 2.0 ** -11 + 1e-7)
    wide = torch.zeros(8, 1024, 96, dtype=torch.int8, device="cuda")
    wide[:, :, 16:80] = packed
    a = hq.dequantize_per_token(wide[:, :, 16:80], scale, 128, 4)
    b = hq.dequantize_per_token(packed, scale, 128, 4)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
