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
