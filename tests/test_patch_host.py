"""Host-side behaviour of the model-level drop-in (hyquant_amd.patch) that
needs no GPU: the dense path's HF attention-backend resolution
(src/patch/_common.py:102-121) and a CPU forward of a patched "dense"
model under sdpa, which must match the unpatched model."""

import types

import pytest
import torch

from hyquant_amd.patch import resolve_attention_interface


def _eager(*args, **kwargs):
    raise AssertionError("not called")


def test_backend_resolution_rules():
    transformers = pytest.importorskip("transformers")
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    cfg = lambda impl: types.SimpleNamespace(_attn_implementation=impl)
    assert resolve_attention_interface(cfg("eager"), _eager) is _eager
    assert resolve_attention_interface(None, _eager) is _eager                      # no config: eager
    assert resolve_attention_interface(cfg(None), _eager) is _eager
    assert resolve_attention_interface(cfg("sdpa"), _eager) is ALL_ATTENTION_FUNCTIONS["sdpa"]
    # sdpa cannot return attention weights in some transformers versions
    assert resolve_attention_interface(cfg("sdpa"), _eager, output_attentions=True) is _eager
    assert resolve_attention_interface(cfg("no_such_backend"), _eager) is _eager
    assert transformers is not None


@pytest.mark.parametrize("family", ["llama", "qwen"])
def test_patched_dense_sdpa_matches_unpatched_cpu(family):
    transformers = pytest.importorskip("transformers")
    from hyquant_amd.patch import patch_attention_forward_model
    torch.manual_seed(0)
    common = dict(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                  num_key_value_heads=2, head_dim=128, vocab_size=128, max_position_embeddings=512,
                  attn_implementation="sdpa")
    if family == "llama":
        make = lambda: transformers.LlamaForCausalLM(transformers.LlamaConfig(**common))
    else:
        make = lambda: transformers.Qwen3ForCausalLM(transformers.Qwen3Config(**common))
    ref = make().eval()
    pat = make().eval()
    pat.load_state_dict(ref.state_dict())
    patch_attention_forward_model(pat, mode="dense")
    ids = torch.randint(0, 128, (1, 40), generator=torch.Generator().manual_seed(1))
    with torch.no_grad():
        a = ref(ids).logits
        b = pat(ids).logits
    assert torch.equal(a, b)
