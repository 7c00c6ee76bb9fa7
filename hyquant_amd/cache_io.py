"""On-disk format of the decode-stage KV cache (DStageKVCache).

The reference cache (src/ops/d_stage_kv_cache.py:360-491) cannot be saved:
beam search and checkpointing raise or are absent (:466-472).  This module
gives the four-segment cache a file format, so a long prompt's frozen cache
can be written once and decoding resumed later, in another process or on
another GPU, with bit-identical results.

Format: one safetensors file (tensors plus a JSON string under the metadata
key "hyquant_amd.dstage_cache"; nothing in it is executed on load).  The JSON
holds the format version, the cache options (window_size, top_ratio,
use_vert, seen_tokens) and, per layer, its bit widths, phase and sizes.
Tensors are named "layers.<i>.<name>":

  decode phase   k_packed / v_packed  int8 [B*H_KV, n_quant, packed width]
                 k_scale / v_scale    fp16 [B*H_KV, n_quant]
                 k_topk / v_topk      [B*H_KV, T, D], topk_indices int64 [B, H_KV, T]
                 k_window / v_window  [B*H_KV, W, D]
                 k_staging / v_staging [B*H_KV, staging_ptr, D] (the live slots)
  prefill phase  keys / values [B, H_KV, N, D], query_tail [B, H_Q, W, D]
                 (absent for a layer that has seen no tokens)

Only the live lengths are stored (not the prefix's spare capacity or the
unused staging slots).  The packed bytes, scales and bf16 rows are the
cache's own tensors, so a loaded cache decodes exactly like the saved one.
"""

from __future__ import annotations

import json
from typing import Dict, Optional, Tuple, Union

import torch

from .decode_d_stage import GROUP_SIZE, _packed_dim

FORMAT_KEY = "hyquant_amd.dstage_cache"
FORMAT_VERSION = 1

_DECODE_TENSORS = ("k_packed", "v_packed", "k_scale", "v_scale", "k_topk", "v_topk", "topk_indices",
                   "k_window", "v_window", "k_staging", "v_staging")


def _layer_state(layer) -> Tuple[Dict[str, torch.Tensor], dict]:
    """Tensors and metadata of one DStageLayerCache."""
    meta = {"k_bits": layer.k_bits, "v_bits": layer.v_bits, "phase": layer.phase, "seq_len": layer._seq_len}
    tensors: Dict[str, torch.Tensor] = {}
    if layer.phase == "decode":
        kp, ks = layer._kstore.views()
        vp, vs = layer._vstore.views()
        ptr = layer._staging_ptr
        tensors = {
            "k_packed": kp, "v_packed": vp, "k_scale": ks, "v_scale": vs,
            "k_topk": layer.k_topk, "v_topk": layer.v_topk, "topk_indices": layer.topk_indices,
            "k_window": layer.k_window, "v_window": layer.v_window,
            "k_staging": layer._staging_buf_k[:, :ptr], "v_staging": layer._staging_buf_v[:, :ptr],
        }
        meta.update({"B": layer._B, "H_KV": layer._H_KV, "D": layer._D, "n_quant": int(kp.shape[1]),
                     "staging_ptr": ptr})
    elif layer._keys is not None:
        tensors = {"keys": layer._keys, "values": layer._values}
        if layer._query_tail is not None:
            tensors["query_tail"] = layer._query_tail
    return tensors, meta


def save_cache(cache, path: str) -> None:
    """Write a DStageKVCache to `path` (safetensors)."""
    from safetensors.torch import save_file

    tensors: Dict[str, torch.Tensor] = {}
    layers = []
    for i in range(cache.num_layers):
        t, meta = _layer_state(cache.get_layer(i))
        layers.append(meta)
        for name, x in t.items():
            tensors[f"layers.{i}.{name}"] = x.detach().to("cpu").contiguous()
    header = {
        "version": FORMAT_VERSION,
        "num_layers": cache.num_layers,
        "window_size": cache.window_size,
        "top_ratio": cache.top_ratio,
        "use_vert": cache.use_vert,
        "seen_tokens": cache.seen_tokens,
        "layers": layers,
    }
    save_file(tensors, path, metadata={FORMAT_KEY: json.dumps(header)})


def _check(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(f"load_cache: {msg}")


def _restore_layer(layer, meta: dict, t: Dict[str, torch.Tensor], device) -> None:
    from .d_stage_kv_cache import _PrefixStore

    layer.phase = meta["phase"]
    layer._seq_len = int(meta["seq_len"])
    if layer.phase == "prefill":
        if "keys" in t:
            _check("values" in t and t["keys"].shape == t["values"].shape, "prefill keys/values mismatch")
            layer._keys = t["keys"].to(device)
            layer._values = t["values"].to(device)
            layer._query_tail = t["query_tail"].to(device) if "query_tail" in t else None
            _check(layer._keys.shape[2] == layer._seq_len, "prefill length does not match seq_len")
        return
    _check(layer.phase == "decode", f"unknown phase {layer.phase!r}")
    missing = [n for n in _DECODE_TENSORS if n not in t]
    _check(not missing, f"decode layer {layer.layer_idx} lacks {missing}")
    B, H_KV, D = int(meta["B"]), int(meta["H_KV"]), int(meta["D"])
    BH = B * H_KV
    nq, ptr = int(meta["n_quant"]), int(meta["staging_ptr"])
    _check(0 <= ptr < GROUP_SIZE, "staging_ptr out of range")
    for name, bits in (("k", layer.k_bits), ("v", layer.v_bits)):
        p, s = t[f"{name}_packed"], t[f"{name}_scale"]
        _check(p.dtype == torch.int8 and tuple(p.shape) == (BH, nq, _packed_dim(D, bits)),
               f"{name}_packed shape {tuple(p.shape)} does not match {bits}-bit codes")
        _check(s.dtype == torch.float16 and tuple(s.shape) == (BH, nq), f"{name}_scale shape")
    T = int(t["k_topk"].shape[1])
    W = int(t["k_window"].shape[1])
    _check(tuple(t["topk_indices"].shape) == (B, H_KV, T), "topk_indices shape")
    for name, n in (("k_topk", T), ("v_topk", T), ("k_window", W), ("v_window", W),
                    ("k_staging", ptr), ("v_staging", ptr)):
        _check(tuple(t[name].shape) == (BH, n, D), f"{name} shape {tuple(t[name].shape)}")
    dtype = t["k_window"].dtype
    layer._B, layer._H_KV, layer._D = B, H_KV, D
    for attr, name, bits in (("_kstore", "k", layer.k_bits), ("_vstore", "v", layer.v_bits)):
        store = _PrefixStore(BH, D, bits, nq, device)
        store.packed[:, :nq].copy_(t[f"{name}_packed"])
        store.scale[:, :nq].copy_(t[f"{name}_scale"])
        setattr(layer, attr, store)
    layer.k_topk = t["k_topk"].to(device)
    layer.v_topk = t["v_topk"].to(device)
    layer.topk_indices = t["topk_indices"].to(device)
    layer.k_window = t["k_window"].to(device)
    layer.v_window = t["v_window"].to(device)
    layer._staging_buf_k = torch.zeros(BH, GROUP_SIZE, D, dtype=dtype, device=device)
    layer._staging_buf_v = torch.zeros(BH, GROUP_SIZE, D, dtype=dtype, device=device)
    layer._staging_buf_k[:, :ptr].copy_(t["k_staging"])
    layer._staging_buf_v[:, :ptr].copy_(t["v_staging"])
    layer._staging_ptr = ptr
    layer._keys = layer._values = layer._query_tail = None


def load_cache(path: str, device: Optional[Union[str, torch.device]] = None):
    """Read a file written by save_cache into a new DStageKVCache on
    `device` (default: the current GPU)."""
    from safetensors import safe_open

    from .d_stage_kv_cache import DStageKVCache

    if device is None:
        device = torch.device("cuda", torch.cuda.current_device())
    device = torch.device(device)
    with safe_open(path, framework="pt", device="cpu") as f:
        md = f.metadata() or {}
        _check(FORMAT_KEY in md, "not a DStageKVCache file")
        header = json.loads(md[FORMAT_KEY])
        _check(header.get("version") == FORMAT_VERSION, f"unsupported format version {header.get('version')}")
        metas = header["layers"]
        _check(len(metas) == header["num_layers"], "layer count mismatch")
        kb = [int(m["k_bits"]) for m in metas]
        vb = [int(m["v_bits"]) for m in metas]
        cache = DStageKVCache(num_layers=header["num_layers"], k_bits=lambda i: kb[i], v_bits_fn=lambda i: vb[i],
                              window_size=header["window_size"], top_ratio=header["top_ratio"],
                              use_vert=header["use_vert"])
        names = set(f.keys())
        for i, meta in enumerate(metas):
            prefix = f"layers.{i}."
            t = {n[len(prefix):]: f.get_tensor(n) for n in names if n.startswith(prefix)}
            _restore_layer(cache.get_layer(i), meta, t, device)
    cache._seen_tokens = int(header["seen_tokens"])
    return cache
