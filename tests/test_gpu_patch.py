"""The model-level drop-in: HF Llama-3 / Qwen3 attention patched with
hyquant_amd.patch (src/patch/patch_llama.py, patch_qwen.py), prefill and
greedy decode through DStageKVCache, on small random-initialised models
(head_dim 128, GQA 2) built from transformers' own model classes.

Checks: the patched "dense" mode reproduces the unpatched model bit for bit;
every hybrid / D-stage mode runs generate() end to end and its per-layer
attention outputs track the dense model's (cosine similarity of the
flattened outputs, which the int4 / int8 quantisation keeps close to 1 and
a wrong head mapping, segment or position would not); unsupported modes
raise."""

import pytest
import torch

pytestmark = pytest.mark.gpu

N_PROMPT = 700
W = 128


def _model(family, seed=0):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(seed)
    common = dict(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
                  num_key_value_heads=2, head_dim=128, vocab_size=256, max_position_embeddings=4096,
                  attn_implementation="eager")
    if family == "llama":
        cfg = transformers.LlamaConfig(**common)
        m = transformers.LlamaForCausalLM(cfg)
    else:
        cfg = transformers.Qwen3Config(**common)
        m = transformers.Qwen3ForCausalLM(cfg)
    return m.to(device="cuda", dtype=torch.bfloat16).eval()


def _capture(model):
    """Per-layer attention outputs of the last forward call (before o_proj)."""
    store = {}
    hooks = []
    for i, layer in enumerate(model.model.layers):
        def pre(mod, args, i=i):
            store[i] = args[0].detach().float()
        hooks.append(layer.self_attn.o_proj.register_forward_pre_hook(pre))
    return store, hooks


def _cos(a, b):
    a, b = a.flatten(), b.flatten()
    return float(torch.dot(a, b) / (a.norm() * b.norm()))


def _ids(seed=1, n=N_PROMPT):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (1, n), generator=g).cuda()


@pytest.mark.parametrize("family", ["llama", "qwen"])
def test_patched_dense_is_identical(family):
    from hyquant_amd.patch import patch_attention_forward_model
    ids = _ids()
    ref = _model(family)
    with torch.no_grad():
        want = ref(ids).logits
    m = patch_attention_forward_model(_model(family), mode="dense", window_size=W)
    with torch.no_grad():
        got = m(ids).logits
    assert torch.equal(got, want)


def _check_decode_against_oracle(cache):
    """Wrap every layer's decode_attention: each call's output is checked at
    once against the float64 oracle over that layer's four segments."""
    import numpy as np
    from oracle import hyq_oracle as O
    checked = []

    def wrap(layer):
        orig = layer.decode_attention

        def run(q, kv_repeat):
            out = orig(q, kv_repeat)
            B, HQ, _, D = q.shape
            npf = lambda t: t.float().cpu().numpy()
            npi = lambda t: t.cpu().numpy()
            ptr = layer._staging_ptr
            args = (npf(q.reshape(B * HQ, D)), npi(layer.k_quant_packed), npi(layer.v_quant_packed),
                    npi(layer.k_scale), npi(layer.v_scale), npf(layer.k_topk), npf(layer.v_topk),
                    npf(layer._staging_buf_k[:, :ptr]), npf(layer._staging_buf_v[:, :ptr]),
                    npf(layer.k_window), npf(layer.v_window))
            ref = O.decode_fp64(*args, k_bits=layer.k_bits, v_bits=layer.v_bits, kv_repeat=kv_repeat)
            ref_abs = O.decode_fp64(*args, k_bits=layer.k_bits, v_bits=layer.v_bits, kv_repeat=kv_repeat,
                                    abs_v=True)
            got = npf(out.reshape(B * HQ, D))
            bound = 2e-3 + 2.0 ** -9 * ref_abs + 2.0 ** -8 * np.abs(ref)
            assert np.all(np.abs(got - ref) <= bound), float(np.max(np.abs(got - ref)))
            checked.append(layer.layer_idx)
            return out
        layer.decode_attention = run

    for i in range(len(cache)):
        wrap(cache.get_layer(i))
    return checked


@pytest.mark.parametrize("family,mode,min_cos", [("llama", "hybrid_full", 0.98), ("llama", "hybrid_k4v2", 0.6),
                                                 ("llama", "d_k4v4", 0.98), ("llama", "d_k8v8", 0.98),
                                                 ("llama", "d_k2v4_vert", 0.6), ("qwen", "hybrid_full", 0.98)])
def test_generate_tracks_dense(family, mode, min_cos):
    """Every decode call matches the oracle over the cache's segments; the
    attention outputs track the dense model's (2-bit codes lose most of a
    value's precision, hence the lower floor for the K4V2 / K2V4 modes)."""
    from hyquant_amd.patch import create_cache_for_mode, patch_attention_forward_model
    print(f"generate {family} {mode}", flush=True)
    ids = _ids()
    dense = _model(family)
    model = patch_attention_forward_model(_model(family), mode=mode, window_size=W, top_ratio=0.05)
    cache = create_cache_for_mode(mode, num_layers=2, window_size=W, top_ratio=0.05)
    checked = _check_decode_against_oracle(cache)
    store, hooks = _capture(model)
    outs = []
    with torch.no_grad():
        # prefill, then 6 greedy decode steps, recording each step's attention outputs
        logits = model(ids, past_key_values=cache, use_cache=True).logits
        outs.append({i: t[:, -1:] for i, t in store.items()})
        seq = ids
        nxt = logits[:, -1:].argmax(-1)
        for _ in range(6):
            seq = torch.cat([seq, nxt], dim=1)
            logits = model(nxt, past_key_values=cache, use_cache=True).logits
            outs.append({i: t.clone() for i, t in store.items()})
            nxt = logits[:, -1:].argmax(-1)
    for h in hooks:
        h.remove()
    # the dense model over the same tokens (teacher forcing), all positions at once
    dstore, dhooks = _capture(dense)
    with torch.no_grad():
        dense(seq)
    for h in dhooks:
        h.remove()
    for step, o in enumerate(outs):
        pos = N_PROMPT - 1 + step
        for i in o:
            c = _cos(o[i], dstore[i][:, pos:pos + 1])
            print(f"  step {step} layer {i}: cos {c:.5f}", flush=True)
            assert c > min_cos, (step, i, c)
    assert checked == [0, 1] * 6
    assert cache.get_layer(0).phase == "decode"
    assert cache.get_seq_length() == N_PROMPT + 6


@pytest.mark.parametrize("mode", ["sage_w", "sage_w0"])
def test_window_only_modes(mode):
    """sage_w / sage_w0 (src/patch/patch_llama.py:211-221): the prefill runs
    sage_unified_attention, whose per-layer outputs track the dense model's;
    decode steps use the model's own attention and the HF cache."""
    from hyquant_amd.patch import patch_attention_forward_model
    ids = _ids(seed=5)
    dense = _model("llama")
    model = patch_attention_forward_model(_model("llama"), mode=mode, window_size=W)
    store, hooks = _capture(model)
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=3, do_sample=False)
        model(ids)
    for h in hooks:
        h.remove()
    dstore, dhooks = _capture(dense)
    with torch.no_grad():
        dense(ids)
    for h in dhooks:
        h.remove()
    for i in store:
        c = _cos(store[i], dstore[i])
        print(f"  {mode} prefill layer {i}: cos {c:.5f}", flush=True)
        assert c > 0.98, (i, c)
    assert out.shape == (1, N_PROMPT + 3)


def test_fp8_qk_prefill_switch(monkeypatch):
    """HYBRID_ATTN_PREFILL_KERNEL=fp8 routes a D-stage mode's prefill through
    the FP8-QK kernel (src/patch/patch_llama.py:160-190); the outputs still
    track the dense model."""
    from hyquant_amd.patch import create_cache_for_mode, patch_attention_forward_model
    monkeypatch.setenv("HYBRID_ATTN_PREFILL_KERNEL", "fp8")
    ids = _ids(seed=6)
    dense = _model("llama")
    model = patch_attention_forward_model(_model("llama"), mode="hybrid_full", window_size=W)
    cache = create_cache_for_mode("hybrid_full", num_layers=2, window_size=W)
    store, hooks = _capture(model)
    with torch.no_grad():
        model(ids, past_key_values=cache, use_cache=True)
    for h in hooks:
        h.remove()
    dstore, dhooks = _capture(dense)
    with torch.no_grad():
        dense(ids)
    for h in dhooks:
        h.remove()
    for i in store:
        c = _cos(store[i], dstore[i])
        print(f"  fp8-QK prefill layer {i}: cos {c:.5f}", flush=True)
        assert c > 0.98, (i, c)


def test_hf_generate_with_cache():
    """transformers' own generate() loop drives the cache (transformers 5.x API)."""
    from hyquant_amd.patch import create_cache_for_mode, patch_attention_forward_model
    ids = _ids(seed=3)
    model = patch_attention_forward_model(_model("llama"), mode="hybrid_full", window_size=W)
    cache = create_cache_for_mode("hybrid_full", num_layers=2, window_size=W)
    with torch.no_grad():
        out = model.generate(ids, past_key_values=cache, max_new_tokens=5, do_sample=False)
    assert out.shape == (1, N_PROMPT + 5)
    assert cache.get_seq_length() == N_PROMPT + 4     # the last token is sampled, not cached


def test_mode_errors():
    from hyquant_amd.patch import patch_attention_forward_model
    m = _model("llama")
    with pytest.raises(ValueError):
        patch_attention_forward_model(m, mode="nope")
    with pytest.raises(NotImplementedError):
        patch_attention_forward_model(m, mode="sparse_only")
    with pytest.raises(ValueError):
        patch_attention_forward_model(m, mode="hybrid_full", top_ratio=0.0)
