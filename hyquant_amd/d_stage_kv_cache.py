"""Quantised decode-stage KV cache on MI355X: drop-in for
src/ops/d_stage_kv_cache.py (DStageLayerCache, DStageKVCache).

Same phases and segment semantics as the reference:
  prefill: bf16 K/V accumulate; the last W queries are kept;
  freeze (first decode step): window = last W tokens (bf16); vertical lines =
    top-rho of [0, N - 2W) (F3) kept bf16 in score order; the remaining prefix
    quantised per token in ascending position order (F6);
  decode: new tokens go to a 128-slot bf16 staging ring; when it fills, it is
    quantised and appended to the prefix (F7: the current token is attended).
Differences (all internal): the freeze runs on the selector / reorganisation
kernels of libhyq.so, and the quantised prefix lives in a capacity buffer, so a
flush quantises 128 tokens in place instead of re-concatenating the whole
prefix (src/ops/d_stage_kv_cache.py:201-216, F10).  k_quant_packed etc. are
views of the live length.
"""

from __future__ import annotations

from typing import Any, Callable, Optional, Tuple

import torch

from . import _lib
from .decode_d_stage import (
    GROUP_SIZE,
    _packed_dim,
    _require_gpu,
    _stream,
    fused_d_stage_decode,
    quantize_into,
)
from .vertical import freeze_vertical_indices

try:
    from transformers.cache_utils import Cache as _HF_Cache
except Exception:  # transformers not available
    _HF_Cache = object

_CAPACITY_STEP = 1024          # prefix capacity grows in multiples of this many tokens


class _PrefixStore:
    """Capacity-allocated int4/int2/int8 prefix with its per-token scales."""

    def __init__(self, BH: int, D: int, bits: int, n: int, device, cap: Optional[int] = None):
        self.bits = bits
        self.D = D
        self.n = n
        cap = cap if cap is not None else ((n + GROUP_SIZE + _CAPACITY_STEP - 1) // _CAPACITY_STEP) * _CAPACITY_STEP
        self.packed = torch.empty(BH, max(cap, 1), _packed_dim(D, bits), dtype=torch.int8, device=device)
        self.scale = torch.empty(BH, max(cap, 1), dtype=torch.float16, device=device)

    @property
    def capacity(self) -> int:
        return self.packed.shape[1]

    def views(self) -> Tuple[torch.Tensor, torch.Tensor]:
        return self.packed[:, :self.n], self.scale[:, :self.n]

    def reserve(self, extra: int) -> None:
        if self.n + extra <= self.capacity:
            return
        cap = max(2 * self.capacity, ((self.n + extra + _CAPACITY_STEP - 1) // _CAPACITY_STEP) * _CAPACITY_STEP)
        packed = torch.empty(self.packed.shape[0], cap, self.packed.shape[2], dtype=torch.int8, device=self.packed.device)
        scale = torch.empty(self.scale.shape[0], cap, dtype=torch.float16, device=self.scale.device)
        packed[:, :self.n].copy_(self.packed[:, :self.n])
        scale[:, :self.n].copy_(self.scale[:, :self.n])
        self.packed, self.scale = packed, scale

    def append_quantized(self, x: torch.Tensor) -> None:
        """Quantise x [BH, m, D] bf16 into the next m slots."""
        m = x.shape[1]
        self.reserve(m)
        quantize_into(x, self.bits, self.packed[:, self.n:self.n + m], self.scale[:, self.n:self.n + m])
        self.n += m


class DStageLayerCache:
    """Per-layer KV cache with the prefill -> decode phase transition
    (src/ops/d_stage_kv_cache.py:36-357)."""

    def __init__(self, layer_idx: int, k_bits: int = 4, v_bits: int = 4, window_size: int = 256,
                 top_ratio: float = 0.05, use_vert: bool = True):
        self.layer_idx = layer_idx
        self.k_bits = k_bits
        self.v_bits = v_bits
        self.window_size = window_size
        self.top_ratio = top_ratio
        self.use_vert = use_vert
        self.phase: str = "prefill"
        self._seq_len: int = 0
        self._keys: Optional[torch.Tensor] = None
        self._values: Optional[torch.Tensor] = None
        self._query_tail: Optional[torch.Tensor] = None
        self._kstore: Optional[_PrefixStore] = None
        self._vstore: Optional[_PrefixStore] = None
        self.k_topk: Optional[torch.Tensor] = None
        self.v_topk: Optional[torch.Tensor] = None
        self.topk_indices: Optional[torch.Tensor] = None
        self._staging_buf_k: Optional[torch.Tensor] = None
        self._staging_buf_v: Optional[torch.Tensor] = None
        self._staging_ptr: int = 0
        self.k_window: Optional[torch.Tensor] = None
        self.v_window: Optional[torch.Tensor] = None
        self._B = self._H_KV = self._D = 0

    # --- prefill -------------------------------------------------------------

    def update_prefill(self, key_states: torch.Tensor, value_states: torch.Tensor):
        """Accumulate bf16 KV during prefill (src/ops/d_stage_kv_cache.py:82-95)."""
        if self._keys is None:
            self._keys = key_states
            self._values = value_states
        else:
            self._keys = torch.cat([self._keys, key_states], dim=2)
            self._values = torch.cat([self._values, value_states], dim=2)
        self._seq_len = self._keys.shape[2]
        return self._keys, self._values

    def save_query_tail(self, query_states: torch.Tensor):
        """Keep the last W queries for the freeze-time selector (:97-100)."""
        W = min(self.window_size, query_states.shape[2])
        self._query_tail = query_states[:, :, -W:, :].detach()

    # --- freeze ----------------------------------------------------------------

    @property
    def k_quant_packed(self):
        return None if self._kstore is None else self._kstore.views()[0]

    @property
    def v_quant_packed(self):
        return None if self._vstore is None else self._vstore.views()[0]

    @property
    def k_scale(self):
        return None if self._kstore is None else self._kstore.views()[1]

    @property
    def v_scale(self):
        return None if self._vstore is None else self._vstore.views()[1]

    def freeze(self, kv_repeat: int = 1):
        """Quantise the prefix, keep window + vertical lines bf16, release the
        bf16 KV (src/ops/d_stage_kv_cache.py:106-189)."""
        assert self.phase == "prefill" and self._keys is not None
        keys, values = self._keys, self._values
        _require_gpu(keys, "keys")
        B, H_KV, N, D = keys.shape
        self._B, self._H_KV, self._D = B, H_KV, D
        BH = B * H_KV
        W = min(self.window_size, N)
        prefix_len = N - W
        dev = keys.device
        dtype = keys.dtype
        if prefix_len > 0 and self.use_vert and self._query_tail is not None and kv_repeat >= 1:
            vidx = freeze_vertical_indices(self._query_tail, keys[:, :, :prefix_len, :], self.window_size,
                                           self.top_ratio, kv_repeat)
        else:
            vidx = torch.zeros(B, H_KV, 0, dtype=torch.int64, device=dev)
        T = int(vidx.shape[-1])
        self.topk_indices = vidx
        self._kstore = _PrefixStore(BH, D, self.k_bits, prefix_len - T, dev)
        self._vstore = _PrefixStore(BH, D, self.v_bits, prefix_len - T, dev)
        self.k_topk = torch.empty(BH, T, D, dtype=dtype, device=dev)
        self.v_topk = torch.empty(BH, T, D, dtype=dtype, device=dev)
        self.k_window = torch.empty(BH, W, D, dtype=dtype, device=dev)
        self.v_window = torch.empty(BH, W, D, dtype=dtype, device=dev)
        k = keys if keys.stride(-1) == 1 else keys.contiguous()
        v = values if values.stride(-1) == 1 else values.contiguous()
        L = _lib.lib()
        stream = _stream(dev)
        ws = torch.empty(max(L.hyq_freeze_workspace_size(BH, prefix_len), 256), dtype=torch.uint8, device=dev)
        kp, ks = self._kstore.packed, self._kstore.scale
        vp, vs = self._vstore.packed, self._vstore.scale
        vidx_flat = vidx.reshape(BH, T).contiguous()
        st = L.hyq_freeze_reorganise(
            k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), v.data_ptr(), v.stride(0), v.stride(1), v.stride(2),
            B, H_KV, N, D, W, vidx_flat.data_ptr(), T, self.k_bits, self.v_bits, int(dtype == torch.float16),
            kp.data_ptr(), kp.stride(0), kp.stride(1), vp.data_ptr(), vp.stride(0), vp.stride(1),
            ks.data_ptr(), ks.stride(0), vs.data_ptr(), vs.stride(0),
            self.k_topk.data_ptr(), self.k_topk.stride(0), self.k_topk.stride(1),
            self.v_topk.data_ptr(), self.v_topk.stride(0), self.v_topk.stride(1),
            self.k_window.data_ptr(), self.k_window.stride(0), self.k_window.stride(1),
            self.v_window.data_ptr(), self.v_window.stride(0), self.v_window.stride(1),
            ws.data_ptr(), ws.numel(), stream)
        _lib.check(st, "freeze")
        self._staging_buf_k = torch.zeros(BH, GROUP_SIZE, D, device=dev, dtype=dtype)
        self._staging_buf_v = torch.zeros(BH, GROUP_SIZE, D, device=dev, dtype=dtype)
        self._staging_ptr = 0
        self._keys = None
        self._values = None
        self._query_tail = None
        self.phase = "decode"

    # --- decode ----------------------------------------------------------------

    def append_staging(self, key_states: torch.Tensor, value_states: torch.Tensor):
        """Append decode token(s) to the staging ring, flushing every 128
        tokens (src/ops/d_stage_kv_cache.py:195-207)."""
        B, H_KV, S, D = key_states.shape
        BH = B * H_KV
        k = key_states.reshape(BH, S, D)
        v = value_states.reshape(BH, S, D)
        i = 0
        while i < S:
            n = min(S - i, GROUP_SIZE - self._staging_ptr)
            self._staging_buf_k[:, self._staging_ptr:self._staging_ptr + n].copy_(k[:, i:i + n])
            self._staging_buf_v[:, self._staging_ptr:self._staging_ptr + n].copy_(v[:, i:i + n])
            self._staging_ptr += n
            i += n
            if self._staging_ptr >= GROUP_SIZE:
                self._flush_staging_buffer()
        self._seq_len += S

    def _flush_staging_buffer(self):
        """Quantise the full ring and append it to the prefix (:209-217)."""
        self._kstore.append_quantized(self._staging_buf_k)
        self._vstore.append_quantized(self._staging_buf_v)
        self._staging_ptr = 0

    def decode_attention(self, query_states: torch.Tensor, kv_repeat: int) -> torch.Tensor:
        """q_len = 1 attention over the four segments (src/ops/d_stage_kv_cache.py:219-354).
        query_states [B, H_Q, 1, D] -> [B, H_Q, 1, D]."""
        B, H_KV, D = self._B, self._H_KV, self._D
        H_Q = H_KV * kv_repeat
        k_staging = self._staging_buf_k[:, :self._staging_ptr]
        v_staging = self._staging_buf_v[:, :self._staging_ptr]
        out = fused_d_stage_decode(
            query_states.reshape(B * H_Q, D), self.k_quant_packed, self.v_quant_packed,
            self.k_scale, self.v_scale, self.k_topk, self.v_topk, k_staging, v_staging,
            self.k_window, self.v_window, self.k_bits, self.v_bits, kv_repeat=kv_repeat)
        return out.reshape(B, H_Q, 1, D)

    def get_seq_length(self) -> int:
        return self._seq_len


def _per_layer(spec, layer_idx: int) -> int:
    """A bit width given as one int for every layer or as a function of the layer index."""
    return int(spec(layer_idx)) if callable(spec) else int(spec)


class DStageKVCache(_HF_Cache):
    """HF `Cache` of D-stage layers, the drop-in for src/ops/d_stage_kv_cache.py:360-491.

    Each layer is a `DStageLayerCache`: bf16 K/V while the prompt is
    prefilled, then (after its `freeze`) the four decode segments, with
    decode-step tokens appended to the bf16 staging segment.  The HF
    protocol surface is what `generate()` touches: `update`,
    `get_seq_length`, `get_mask_sizes`, `get_max_cache_shape`, `reset`,
    indexing and iteration per layer.  Beam search is not supported (its
    batch re-indexing methods raise), and `crop` leaves the cache as it is:
    the quantised segments are never shortened."""

    is_compileable = False

    def __init__(self, num_layers: int = 32, k_bits=4, v_bits_fn: Callable[[int], int] = lambda i: 4 if i == 0 else 2,
                 window_size: int = 256, top_ratio: float = 0.05, use_vert: bool = True):
        # transformers 5.x wants an explicit (here empty) layer list; 4.x takes
        # no arguments; without transformers the base is `object`
        for kwargs in ({"layers": []}, {}):
            try:
                super().__init__(**kwargs)
                break
            except TypeError:
                continue
        self.num_layers = num_layers
        self.window_size = window_size
        self.top_ratio = top_ratio
        self.use_vert = use_vert
        self._bits = [(_per_layer(k_bits, i), _per_layer(v_bits_fn, i)) for i in range(num_layers)]
        self._layers = [self._new_layer(i) for i in range(num_layers)]
        self._seen_tokens = 0

    def _new_layer(self, i: int) -> DStageLayerCache:
        kb, vb = self._bits[i]
        return DStageLayerCache(i, kb, vb, self.window_size, self.top_ratio, self.use_vert)

    # -- HF Cache protocol ---------------------------------------------------

    def update(self, key_states, value_states, layer_idx: int, cache_kwargs: Optional[dict[str, Any]] = None):
        layer = self._layers[layer_idx]
        if layer.phase == "prefill":
            out = layer.update_prefill(key_states, value_states)
        else:                           # a decode step: the token joins the bf16 staging segment
            layer.append_staging(key_states, value_states)
            out = (key_states, value_states)
        if layer_idx == 0:              # HF reads the running token count from layer 0
            self._seen_tokens = layer.get_seq_length()
        return out

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if 0 <= layer_idx < len(self._layers):
            return self._layers[layer_idx].get_seq_length()
        return 0

    def get_max_cache_shape(self) -> int:
        return -1                       # no fixed capacity

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> Tuple[int, int]:
        """(kv_length, kv_offset) for HF's causal-mask construction."""
        kv = self.get_seq_length(layer_idx)
        return (query_length, 0) if kv == 0 else (kv, max(0, kv - query_length))

    def reset(self):
        self._layers = [self._new_layer(i) for i in range(self.num_layers)]
        self._seen_tokens = 0

    def crop(self, max_length: int):
        pass

    def batch_repeat_interleave(self, repeats: int):
        raise NotImplementedError("beam search is not supported by DStageKVCache")

    def batch_select_indices(self, indices: torch.Tensor):
        raise NotImplementedError("beam search is not supported by DStageKVCache")

    def __len__(self) -> int:
        return self.num_layers

    def __getitem__(self, idx: int):
        """The bf16 prompt K/V of a layer still in prefill, else (None, None)."""
        layer = self._layers[idx]
        if layer.phase == "prefill" and layer._keys is not None:
            return layer._keys, layer._values
        return None, None

    def __iter__(self):
        return (self[i] for i in range(len(self._layers)))

    def __bool__(self) -> bool:
        return True                     # an empty cache is still a cache to generate()

    # -- this implementation -------------------------------------------------

    def get_layer(self, layer_idx: int) -> DStageLayerCache:
        return self._layers[layer_idx]

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    def save(self, path: str) -> None:
        """Write the cache (all four segments of every layer) to a safetensors
        file; see hyquant_amd.cache_io for the format."""
        from .cache_io import save_cache
        save_cache(self, path)

    @classmethod
    def load(cls, path: str, device=None) -> "DStageKVCache":
        """Read a file written by save() onto `device` (default: the current GPU)."""
        from .cache_io import load_cache
        return load_cache(path, device)


QuantizedKVCache = DStageKVCache
