"""CPU checks of bench.py's float32 references (the prefill / decode error
figures in the bench line): the chunked causal attention against torch's
float64 scaled_dot_product_attention, and error_vs on known answers."""

import math

import torch

import bench


def test_exact_attention_matches_float64_sdpa():
    g = torch.Generator().manual_seed(3)
    B, HQ, HKV, N, D = 1, 4, 2, 300, 128
    q = torch.randn(B, HQ, N, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, HKV, N, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, HKV, N, D, generator=g).to(torch.bfloat16)
    out = bench.exact_attention_fp32(q, k, v, chunk=128)          # chunks that do not divide N
    ke = k.double().repeat_interleave(HQ // HKV, dim=1)
    ve = v.double().repeat_interleave(HQ // HKV, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.double(), ke, ve, is_causal=True)
    assert float((out.double() - ref).abs().max()) < 1e-5
    # row 0 attends to key 0 alone
    assert torch.allclose(out[:, :, 0], v.float().repeat_interleave(2, dim=1)[:, :, 0], atol=1e-6)


def test_error_vs_known_answers():
    ref = torch.tensor([[1.0, -2.0], [0.5, 4.0]])
    out = ref + torch.tensor([[0.0, 0.1], [-0.3, 0.0]])
    e = bench.error_vs(out, ref)
    assert math.isclose(e["max_abs"], 0.3, rel_tol=1e-6)
    assert math.isclose(e["rel_max"], 0.3 / 4.0, rel_tol=1e-6)
    assert math.isclose(e["mse"], (0.01 + 0.09) / 4, rel_tol=1e-6)
    assert math.isclose(e["rel_l2"], math.sqrt(0.1) / math.sqrt(1 + 4 + 0.25 + 16), rel_tol=1e-6)
