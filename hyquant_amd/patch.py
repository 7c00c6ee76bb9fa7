"""Attention patches for Hugging Face Llama-3 and Qwen3 models on MI355X.

Drop-in for the reference's patch entry points:
  patch_attention_forward_model          src/patch/__init__.py:29-71
  patch_llama3_attention_forward_model   src/patch/patch_llama.py:265-298
  patch_qwen3_attention_forward_model    src/patch/patch_qwen.py (same shape)
  create_cache_for_mode                  src/ops/__init__.py:28-67
and the helpers of src/patch/_common.py (mode table, argument validation,
the D-stage cache hand-off of :198-228).

Each patched attention module keeps its projections, rotary embedding and
output projection and routes the attention itself by mode:
  dense                the model's own attention (cache updated as usual);
  D-stage modes        (d_k4v4 ... hybrid_k2v4, the mode table below) with a
                       DStageKVCache attached: prefill keeps the bf16 KV and
                       the last W queries, the first decode step freezes the
                       cache into its four segments, every decode step runs
                       the fused decode kernel over them; the prefill itself
                       runs the hybrid kernel ("vquant_vert" prefill) or exact
                       causal attention ("full" prefill);
  vquant_vert          hybrid prefill without a D-stage cache;
  sage_w, sage_w0      window-only INT8-QK prefill (sage_unified_attention)
                       with the window W, or with every key in int8;
  full_attention       exact causal attention for the prefill.
Decode steps of the prefill-only modes use the model's own attention, as in
the reference.  The sparse baselines (sparse_only, minference_sparse) are not
part of this build and raise NotImplementedError when a model is patched
with them.

Exact causal attention is the hybrid prefill kernel with the window covering
the whole sequence (every key tile in fp16, one softmax), so every prefill
runs on libhyq.so.
"""

from __future__ import annotations

import os

from types import MethodType
from typing import Any, Optional, Tuple

import torch

from .d_stage_kv_cache import DStageKVCache
from .decode_d_stage import _dequantize_by_bits, _quantize_by_bits
from .sage_unified import sage_vertical_attention_v2
from .vertical import compute_vertical_indices

# src/patch/_common.py:38-49: bit widths, vertical-line retention, prefill kernel
D_STAGE_MODES = {
    "d_k4v4": {"k_bits": 4, "v_bits": 4, "vert": False, "prefill_kernel": "full"},
    "d_k4v4_vert": {"k_bits": 4, "v_bits": 4, "vert": True, "prefill_kernel": "full"},
    "d_k8v8": {"k_bits": 8, "v_bits": 8, "vert": False, "prefill_kernel": "full"},
    "d_k4v2": {"k_bits": 4, "v_bits": 2, "vert": False, "prefill_kernel": "full"},
    "d_k4v2_vert": {"k_bits": 4, "v_bits": 2, "vert": True, "prefill_kernel": "full"},
    "d_k2v4": {"k_bits": 2, "v_bits": 4, "vert": False, "prefill_kernel": "full"},
    "d_k2v4_vert": {"k_bits": 2, "v_bits": 4, "vert": True, "prefill_kernel": "full"},
    "hybrid_full": {"k_bits": 4, "v_bits": 4, "vert": True, "prefill_kernel": "vquant_vert"},
    "hybrid_k4v2": {"k_bits": 4, "v_bits": 2, "vert": True, "prefill_kernel": "vquant_vert"},
    "hybrid_k2v4": {"k_bits": 2, "v_bits": 4, "vert": True, "prefill_kernel": "vquant_vert"},
}

VALID_MODES = {"dense", "full_attention", "sage_w", "sage_w0", "vquant_vert", "minference_sparse", "sparse_only",
               "d_stage", *D_STAGE_MODES}
_NOT_BUILT = {"sparse_only", "minference_sparse"}
_VALID_BITS = (2, 4, 8)


def validate_patch_args(mode: str, window_size: int, top_ratio: float, k_bits: Optional[int] = None,
                        v_bits: Optional[int] = None) -> str:
    """The reference's checks and messages (src/patch/_common.py:59-77)."""
    if mode not in VALID_MODES:
        raise ValueError(f"Unsupported mode '{mode}'. Expected one of: {sorted(VALID_MODES)}.")
    if window_size < 0:
        raise ValueError(f"window_size must be >= 0, got {window_size}.")
    if not (0.0 < top_ratio <= 1.0):
        raise ValueError(f"top_ratio must be in (0, 1], got {top_ratio}.")
    if mode == "d_stage":
        if k_bits not in _VALID_BITS:
            raise ValueError(f"k_bits must be in {sorted(_VALID_BITS)}, got {k_bits}.")
        if v_bits not in _VALID_BITS:
            raise ValueError(f"v_bits must be in {sorted(_VALID_BITS)}, got {v_bits}.")
    return mode


def is_d_stage_mode(mode: str) -> bool:
    return mode == "d_stage" or mode in D_STAGE_MODES


def is_d_stage_cache(past_key_values: Any) -> bool:
    """Duck-typed like the reference (src/patch/_common.py:194-196)."""
    return hasattr(past_key_values, "get_layer") and hasattr(past_key_values, "_layers")


def infer_kv_repeat(attn_module: torch.nn.Module) -> int:
    """Query heads per KV head of an attention module (src/patch/_common.py:90-99)."""
    groups = getattr(attn_module, "num_key_value_groups", None)
    if groups is not None:
        return max(int(groups), 1)
    if hasattr(attn_module, "num_heads") and hasattr(attn_module, "num_key_value_heads"):
        return max(int(attn_module.num_heads) // max(int(attn_module.num_key_value_heads), 1), 1)
    return 1


def create_cache_for_mode(mode: str, num_layers: int, head_dim: int = 128, k_bits: int = 4, v_bits: int = 4,
                          **kwargs) -> Optional[DStageKVCache]:
    """The D-stage cache a mode decodes against, or None (src/ops/__init__.py:28-67)."""
    if not is_d_stage_mode(mode):
        return None
    if mode == "d_stage":
        kb, vb, vert = k_bits, v_bits, True
    else:
        cfg = D_STAGE_MODES[mode]
        kb, vb, vert = cfg["k_bits"], cfg["v_bits"], cfg["vert"]
    return DStageKVCache(num_layers=num_layers, k_bits=kb, v_bits_fn=lambda i, _vb=vb: _vb,
                         window_size=kwargs.get("window_size", 256), top_ratio=kwargs.get("top_ratio", 0.05),
                         use_vert=vert)


def handle_d_stage_cache(layer_idx: int, past_key_values: Any, query_states: torch.Tensor,
                         key_states: torch.Tensor, value_states: torch.Tensor, attn_module: torch.nn.Module,
                         sin: torch.Tensor, cos: torch.Tensor,
                         cache_position: Optional[torch.LongTensor]) -> Tuple[torch.Tensor, torch.Tensor]:
    """Prefill: keep the query tail and accumulate bf16 KV; decode: freeze on
    the first step, then append to the staging ring (src/patch/_common.py:198-228)."""
    layer_cache = past_key_values.get_layer(layer_idx)
    if query_states.shape[2] > 1:
        layer_cache.save_query_tail(query_states)
        return past_key_values.update(key_states, value_states, layer_idx,
                                      {"sin": sin, "cos": cos, "cache_position": cache_position})
    if layer_cache.phase == "prefill":
        layer_cache.freeze(kv_repeat=infer_kv_repeat(attn_module))
    layer_cache.append_staging(key_states, value_states)
    return key_states, value_states


def resolve_attention_interface(config: Any, eager_fn, *, output_attentions: bool = False):
    """The HF attention backend the dense path calls (src/patch/_common.py:102-121):
    the model's `_attn_implementation` looked up in transformers' registry of
    attention functions, falling back to the family's eager forward when the
    implementation is eager, unknown or unavailable, or when attention
    weights are requested from sdpa (some transformers versions cannot
    return them)."""
    impl = getattr(config, "_attn_implementation", None) or "eager"
    if impl == "eager" or (impl == "sdpa" and output_attentions):
        return eager_fn
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS
    except Exception:
        return eager_fn
    return ALL_ATTENTION_FUNCTIONS.get(impl, eager_fn)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Exact causal attention, q [B, H_q, N, D], k/v [B, H_kv, N, D] (GQA-native):
    the hybrid kernel with every key inside the window (fp16 QK and P.V)."""
    B, H, N, _ = q.shape
    none = torch.empty((B, H, 0), dtype=torch.int64, device=q.device)
    return sage_vertical_attention_v2(q, k, v, none, window_size=N, smooth_k=False)


def _hybrid_prefill(q, k, v, window_size: int, top_ratio: float, kv_repeat: int, fp8_qk: bool = False) -> torch.Tensor:
    vidx = compute_vertical_indices(q, k, window_size, top_ratio, kv_repeat=kv_repeat)
    if fp8_qk:
        from .sage_unified import sage_vertical_attention_v2_fp8
        return sage_vertical_attention_v2_fp8(q, k, v, vidx, window_size=window_size, smooth_k=True)
    return sage_vertical_attention_v2(q, k, v, vidx, window_size=window_size, smooth_k=True)


def _quant_roundtrip_decode(q, k, v, mode: str, window_size: int, top_ratio: float, kv_repeat: int):
    """Decode without an attached D-stage cache: the reference's quantise /
    dequantise round trip of the whole KV, bf16 window and vertical lines
    kept (src/patch/patch_llama.py:113-152)."""
    cfg = D_STAGE_MODES.get(mode, {"k_bits": 4, "v_bits": 4, "vert": True})
    B, Hkv, N, D = k.shape
    kf = k.unsqueeze(2).expand(B, Hkv, kv_repeat, N, D).reshape(B, Hkv * kv_repeat, N, D)
    vf = v.unsqueeze(2).expand(B, Hkv, kv_repeat, N, D).reshape(B, Hkv * kv_repeat, N, D)
    H = kf.shape[1]
    kp, ks = _quantize_by_bits(kf.reshape(B * H, N, D).contiguous(), cfg["k_bits"])
    vp, vs = _quantize_by_bits(vf.reshape(B * H, N, D).contiguous(), cfg["v_bits"])
    kd = _dequantize_by_bits(kp, ks, D, cfg["k_bits"]).reshape(B, H, N, D).to(k.dtype)
    vd = _dequantize_by_bits(vp, vs, D, cfg["v_bits"]).reshape(B, H, N, D).to(v.dtype)
    if N > window_size:
        kd[:, :, N - window_size:] = kf[:, :, N - window_size:]
        vd[:, :, N - window_size:] = vf[:, :, N - window_size:]
        if cfg["vert"]:
            P = N - window_size
            idx = compute_vertical_indices(q, kf, window_size, top_ratio).unsqueeze(-1).expand(-1, -1, -1, D)
            kd[:, :, :P].scatter_(2, idx, kf[:, :, :P].gather(2, idx))
            vd[:, :, :P].scatter_(2, idx, vf[:, :, :P].gather(2, idx))
    scores = (q @ kd.transpose(-1, -2).contiguous()) * (D ** -0.5)
    return torch.softmax(scores.float(), dim=-1).to(vd.dtype) @ vd


def build_attention_forward(family: str, *, mode: str, window_size: int, top_ratio: float):
    """Patched forward of a Llama-3 ("llama") or Qwen3 ("qwen", q/k RMS norms)
    attention module (src/patch/patch_llama.py:27-259, src/patch/patch_qwen.py)."""
    if family == "llama":
        from transformers.models.llama.modeling_llama import apply_rotary_pos_emb, eager_attention_forward
    elif family == "qwen":
        from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb, eager_attention_forward
    else:
        raise ValueError(f"unknown model family '{family}'")
    d_mode = is_d_stage_mode(mode)

    def forward(self, hidden_states: torch.Tensor, position_embeddings: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
                attention_mask: Optional[torch.Tensor] = None, past_key_values: Optional[Any] = None,
                cache_position: Optional[torch.LongTensor] = None, **kwargs):
        output_attentions = bool(kwargs.pop("output_attentions", False))
        kwargs.pop("use_cache", None)
        kwargs.pop("position_ids", None)
        for alias in ("past_key_values", "past_key_value"):       # transformers 4.x / 5.x names
            if past_key_values is None and alias in kwargs:
                past_key_values = kwargs.pop(alias)
            kwargs.pop(alias, None)
        if position_embeddings is None:
            raise ValueError("position_embeddings are required for the patched attention.")
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape)
        k = self.k_proj(hidden_states).view(hidden_shape)
        if family == "qwen":
            q, k = self.q_norm(q), self.k_norm(k)
        q, k = q.transpose(1, 2), k.transpose(1, 2)
        v = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = apply_rotary_pos_emb(q, k, cos, sin)
        q_len = int(q.shape[2])
        kv_repeat = infer_kv_repeat(self)

        d_cache = d_mode and past_key_values is not None and is_d_stage_cache(past_key_values)
        if d_cache:
            k, v = handle_d_stage_cache(self.layer_idx, past_key_values, q, k, v, self, sin, cos, cache_position)
        elif past_key_values is not None:
            k, v = past_key_values.update(k, v, self.layer_idx, {"sin": sin, "cos": cos,
                                                                 "cache_position": cache_position})
        attn_weights = None
        if mode == "dense" or (q_len == 1 and not d_mode):
            if attention_mask is not None and attention_mask.ndim == 4:
                attention_mask = attention_mask[:, :, :, : k.shape[-2]]
            attend = resolve_attention_interface(getattr(self, "config", None), eager_attention_forward,
                                                 output_attentions=output_attentions)
            out, attn_weights = attend(
                self, q, k, v, attention_mask, dropout=0.0, scaling=getattr(self, "scaling", q.shape[-1] ** -0.5),
                sliding_window=getattr(self, "sliding_window", None), **kwargs)
        else:
            if q_len == 1 and d_cache:
                out = past_key_values.get_layer(self.layer_idx).decode_attention(q, kv_repeat)
            elif q_len == 1:
                out = _quant_roundtrip_decode(q, k, v, mode, window_size, top_ratio, kv_repeat)
            else:
                if k.shape[2] != q_len:
                    raise NotImplementedError("chunked prefill (keys longer than queries) is not supported")
                hybrid = mode == "vquant_vert" or mode == "d_stage" or (
                    d_mode and D_STAGE_MODES[mode]["prefill_kernel"] == "vquant_vert")
                if mode in ("sage_w", "sage_w0"):             # src/patch/patch_llama.py:211-221
                    from .sage_unified import sage_unified_attention
                    out = sage_unified_attention(q, k, v, window_size=window_size if mode == "sage_w" else 0,
                                                 smooth_k=True)
                elif hybrid:
                    # D-stage modes honour HYBRID_ATTN_PREFILL_KERNEL=fp8 (src/patch/patch_llama.py:160-190)
                    fp8_qk = d_mode and os.environ.get("HYBRID_ATTN_PREFILL_KERNEL", "int8").lower() == "fp8"
                    out = _hybrid_prefill(q, k, v, window_size, top_ratio, kv_repeat, fp8_qk)
                else:                                           # full_attention and the "full" D-stage modes
                    out = causal_attention(q, k, v)
            out = out.transpose(1, 2).to(hidden_states.dtype).contiguous()
        out = self.o_proj(out.reshape(*input_shape, -1).contiguous())
        return out, (attn_weights if output_attentions else None)

    return forward


def _patch(model: torch.nn.Module, family: str, cls, mode: str, window_size: int, top_ratio: float,
           k_bits: Optional[int], v_bits: Optional[int]) -> torch.nn.Module:
    mode = validate_patch_args(mode, window_size, top_ratio, k_bits, v_bits)
    if mode in _NOT_BUILT:
        raise NotImplementedError(f"mode '{mode}' (sparse baseline) is not part of this build; the attention "
                                  "modes are dense, full_attention, sage_w, sage_w0, vquant_vert, hybrid_* and d_*")
    fwd = build_attention_forward(family, mode=mode, window_size=window_size, top_ratio=top_ratio)
    patched = 0
    for module in model.modules():
        if isinstance(module, cls):
            if not hasattr(module, "_original_forward"):
                module._original_forward = module.forward
            module.forward = MethodType(fwd, module)
            patched += 1
    if patched == 0:
        raise RuntimeError(f"No {cls.__name__} modules were found to patch.")
    return model


def patch_llama3_attention_forward_model(model: torch.nn.Module, *, mode: str = "sage_w", window_size: int = 256,
                                         top_ratio: float = 0.05, k_bits: Optional[int] = None,
                                         v_bits: Optional[int] = None, report_stats: bool = False,
                                         use_vertical_indices: bool = True) -> torch.nn.Module:
    """Patch every LlamaAttention module in place (src/patch/patch_llama.py:265-298)."""
    del report_stats, use_vertical_indices
    from transformers.models.llama.modeling_llama import LlamaAttention
    return _patch(model, "llama", LlamaAttention, mode, window_size, top_ratio, k_bits, v_bits)


def patch_qwen3_attention_forward_model(model: torch.nn.Module, *, mode: str = "sage_w", window_size: int = 256,
                                        top_ratio: float = 0.05, k_bits: Optional[int] = None,
                                        v_bits: Optional[int] = None, report_stats: bool = False,
                                        use_vertical_indices: bool = True) -> torch.nn.Module:
    """Patch every Qwen3Attention module in place (src/patch/patch_qwen.py)."""
    del report_stats, use_vertical_indices
    from transformers.models.qwen3.modeling_qwen3 import Qwen3Attention
    return _patch(model, "qwen", Qwen3Attention, mode, window_size, top_ratio, k_bits, v_bits)


def _infer_patch_target(model) -> str:
    text = f"{getattr(getattr(model, 'config', None), 'model_type', '')} {model.__class__.__name__}".lower()
    if "glm" in text:
        return "glm4"
    if "qwen" in text:
        return "qwen"
    if "llama" in text:
        return "llama"
    raise ValueError(f"Unable to infer patch target from model '{model.__class__.__name__}'. "
                     "Please set patch_target explicitly to one of: qwen, llama, glm4.")


def patch_attention_forward_model(model, *, mode: str = "sage_w", window_size: int = 256, top_ratio: float = 0.05,
                                  report_stats: bool = False, use_vertical_indices: bool = True,
                                  patch_target: str = "auto"):
    """Patch qwen / llama attention with optional auto detection (src/patch/__init__.py:29-71)."""
    if patch_target == "auto":
        patch_target = _infer_patch_target(model)
    if patch_target == "qwen":
        return patch_qwen3_attention_forward_model(model, mode=mode, window_size=window_size, top_ratio=top_ratio)
    if patch_target == "llama":
        return patch_llama3_attention_forward_model(model, mode=mode, window_size=window_size, top_ratio=top_ratio)
    if patch_target == "glm4":
        raise NotImplementedError("the GLM-4 patch never reaches the hybrid kernels and is not part of this build")
    raise ValueError("Unsupported patch_target. Expected one of: auto, qwen, llama, glm4.")
