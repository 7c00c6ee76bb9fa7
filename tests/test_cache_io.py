"""Round trips of the DStageKVCache file format (hyquant_amd.cache_io) on
CPU tensors: the layers are filled by hand with the shapes the freeze and
the staging ring produce, so no kernel runs."""

import json

import pytest
import torch

from hyquant_amd.cache_io import FORMAT_KEY, load_cache, save_cache
from hyquant_amd.d_stage_kv_cache import DStageKVCache, _PrefixStore

B, HKV, HQ, D = 2, 2, 8, 128


def _rand_bf16(g, *shape):
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def _fill_decode_layer(layer, g, nq=300, T=17, W=64, ptr=37):
    """A decode-phase layer with random codes, scales and rows."""
    BH = B * HKV
    layer.phase = "decode"
    layer._B, layer._H_KV, layer._D = B, HKV, D
    for attr, bits in (("_kstore", layer.k_bits), ("_vstore", layer.v_bits)):
        st = _PrefixStore(BH, D, bits, nq, "cpu")
        st.packed.copy_(torch.randint(-128, 128, st.packed.shape, generator=g, dtype=torch.int8))
        st.scale.copy_(torch.rand(st.scale.shape, generator=g).to(torch.float16))
        setattr(layer, attr, st)
    layer.k_topk, layer.v_topk = _rand_bf16(g, BH, T, D), _rand_bf16(g, BH, T, D)
    layer.topk_indices = torch.randint(0, 1000, (B, HKV, T), generator=g)
    layer.k_window, layer.v_window = _rand_bf16(g, BH, W, D), _rand_bf16(g, BH, W, D)
    layer._staging_buf_k = torch.zeros(BH, 128, D, dtype=torch.bfloat16)
    layer._staging_buf_v = torch.zeros(BH, 128, D, dtype=torch.bfloat16)
    layer._staging_buf_k[:, :ptr] = _rand_bf16(g, BH, ptr, D)
    layer._staging_buf_v[:, :ptr] = _rand_bf16(g, BH, ptr, D)
    layer._staging_ptr = ptr
    layer._seq_len = nq + T + W + ptr


def _make_cache(g):
    """Four layers: K4V2 and K4V4 in decode, one prefill layer with its
    query tail, one that has seen nothing."""
    cache = DStageKVCache(num_layers=4, k_bits=4, v_bits_fn=lambda i: 2 if i == 0 else 4, window_size=64)
    _fill_decode_layer(cache.get_layer(0), g)
    _fill_decode_layer(cache.get_layer(1), g, nq=0, T=0, ptr=0)
    l2 = cache.get_layer(2)
    l2.update_prefill(_rand_bf16(g, B, HKV, 90, D), _rand_bf16(g, B, HKV, 90, D))
    l2.save_query_tail(_rand_bf16(g, B, HQ, 90, D))
    cache._seen_tokens = 417
    return cache


def _same(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and torch.equal(a.view(torch.uint8) if a.dtype != torch.int64 else a,
                                                                     b.view(torch.uint8) if b.dtype != torch.int64 else b)


def test_round_trip_is_bit_identical(tmp_path):
    g = torch.Generator().manual_seed(5)
    cache = _make_cache(g)
    path = str(tmp_path / "cache.safetensors")
    cache.save(path)
    back = DStageKVCache.load(path, device="cpu")
    assert back.num_layers == 4 and back.window_size == 64 and back.seen_tokens == 417
    for i in range(4):
        a, b = cache.get_layer(i), back.get_layer(i)
        assert (a.phase, a.k_bits, a.v_bits, a.get_seq_length()) == (b.phase, b.k_bits, b.v_bits, b.get_seq_length())
        if a.phase == "decode":
            for name in ("k_quant_packed", "v_quant_packed", "k_scale", "v_scale", "k_topk", "v_topk",
                         "topk_indices", "k_window", "v_window"):
                assert _same(getattr(a, name), getattr(b, name)), name
            assert b._staging_ptr == a._staging_ptr
            assert _same(a._staging_buf_k[:, :a._staging_ptr], b._staging_buf_k[:, :b._staging_ptr])
            assert _same(a._staging_buf_v[:, :a._staging_ptr], b._staging_buf_v[:, :b._staging_ptr])
            assert b._staging_buf_k.shape[1] == 128        # the ring keeps its full size
            assert b._kstore.capacity >= b._kstore.n + 128  # room for the next flush
        elif a._keys is not None:
            assert _same(a._keys, b._keys) and _same(a._values, b._values)
            assert _same(a._query_tail, b._query_tail)
        else:
            assert b._keys is None


def test_only_live_lengths_are_stored(tmp_path):
    from safetensors import safe_open
    g = torch.Generator().manual_seed(6)
    cache = _make_cache(g)
    path = str(tmp_path / "c.safetensors")
    save_cache(cache, path)
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = json.loads(f.metadata()[FORMAT_KEY])
        assert meta["version"] == 1 and [m["phase"] for m in meta["layers"]] == ["decode", "decode", "prefill", "prefill"]
        assert tuple(f.get_tensor("layers.0.k_packed").shape) == (B * HKV, 300, 64)   # int4 K
        assert tuple(f.get_tensor("layers.0.v_packed").shape) == (B * HKV, 300, 32)   # int2 V
        assert tuple(f.get_tensor("layers.0.k_staging").shape) == (B * HKV, 37, D)
        assert not any(k.startswith("layers.3.") for k in f.keys())


def test_load_rejects_inconsistent_files(tmp_path):
    from safetensors.torch import save_file
    g = torch.Generator().manual_seed(7)
    cache = _make_cache(g)
    path = str(tmp_path / "c.safetensors")
    save_cache(cache, path)
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        tensors = {k: f.get_tensor(k) for k in f.keys()}
        meta = json.loads(f.metadata()[FORMAT_KEY])
    # a V code width that does not match the recorded bit width
    bad = dict(tensors)
    bad["layers.0.v_packed"] = torch.zeros(B * HKV, 300, 64, dtype=torch.int8)
    save_file(bad, str(tmp_path / "bad.safetensors"), metadata={FORMAT_KEY: json.dumps(meta)})
    with pytest.raises(ValueError, match="v_packed"):
        load_cache(str(tmp_path / "bad.safetensors"), device="cpu")
    # a missing segment
    bad = {k: v for k, v in tensors.items() if k != "layers.0.k_window"}
    save_file(bad, str(tmp_path / "bad2.safetensors"), metadata={FORMAT_KEY: json.dumps(meta)})
    with pytest.raises(ValueError, match="k_window"):
        load_cache(str(tmp_path / "bad2.safetensors"), device="cpu")
    # an unknown version and a file of another kind
    meta2 = dict(meta, version=2)
    save_file(tensors, str(tmp_path / "v2.safetensors"), metadata={FORMAT_KEY: json.dumps(meta2)})
    with pytest.raises(ValueError, match="version"):
        load_cache(str(tmp_path / "v2.safetensors"), device="cpu")
    save_file({"x": torch.zeros(1)}, str(tmp_path / "other.safetensors"))
    with pytest.raises(ValueError, match="not a DStageKVCache"):
        load_cache(str(tmp_path / "other.safetensors"), device="cpu")
