"""Vertical-line selector on MI355X: drop-in for compute_vertical_indices
(src/patch/_common.py:144-190).

Definition (bit-exact with the CPU oracle): the query mean of the last
min(window, Q) queries is rounded once to bf16 (exact float64 sum), each score
is the exact dot product rounded once to bf16, and the top-k are returned in
(score desc, index asc) order; torch.topk leaves the order of ties unspecified
(src/patch/_common.py:189), this build breaks ties by the lower index.
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .decode_d_stage import _require_gpu, _stream

_ws_cache: dict = {}


def _scratch(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index, stream, "select")
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


def top_k_count(prefix_len: int, top_ratio: float) -> int:
    """min(max(1, ceil(P * rho)), P) exactly as src/patch/_common.py:187-188."""
    top_k = max(1, int(math.ceil(prefix_len * top_ratio)))
    return min(top_k, prefix_len)


def _rows_ok(t: torch.Tensor) -> torch.Tensor:
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any((s * 2) % 16 for s in t.stride()[:-1]):
        return t.contiguous()
    return t


def _select(q: torch.Tensor, group: int, k: torch.Tensor, prefix_len: int, tail: int, top_k: int) -> torch.Tensor:
    B, HQ, QL, D = q.shape
    HK = k.shape[1]
    if q.dtype not in (torch.bfloat16, torch.float16) or k.dtype != q.dtype:
        raise ValueError(f"compute_vertical_indices expects bf16 or fp16 queries and keys of one dtype, "
                         f"got {q.dtype} and {k.dtype}")
    q = q if q.stride(-1) == 1 else q.contiguous()
    k = _rows_ok(k)
    h_out = HQ // group
    out = torch.empty(B, h_out, top_k, dtype=torch.int64, device=q.device)
    if B == 0 or top_k == 0:
        return out
    L = _lib.lib()
    stream = _stream(q.device)
    need = L.hyq_vertical_select_workspace_size(B, h_out, prefix_len, top_k)
    if need == 0:
        raise ValueError(f"compute_vertical_indices: unsupported prefix length {prefix_len}")
    ws = _scratch(q.device, stream, need)
    st = L.hyq_vertical_select(q.data_ptr(), q.stride(0), q.stride(1), q.stride(2), QL, HQ, group,
                               k.data_ptr(), k.stride(0), k.stride(1), k.stride(2), HK, prefix_len, B, D,
                               tail, top_k, int(q.dtype == torch.float16), out.data_ptr(), ws.data_ptr(),
                               ws.numel(), stream)
    _lib.check(st, "compute_vertical_indices")
    return out


def compute_vertical_indices(query_states: torch.Tensor, key_states: torch.Tensor, window_size: int,
                             top_ratio: float, kv_repeat: int = 1) -> torch.Tensor:
    """query_states [B, H_Q, Q, D]; key_states [B, H, K, D] with H == H_Q or
    H == H_Q / kv_repeat (GQA-native).  Returns int64 [B, H_Q, top_k]."""
    _require_gpu(query_states, "query_states")
    batch, num_heads, query_len, head_dim = query_states.shape
    key_len = int(key_states.shape[2])
    prefix_len = max(0, key_len - window_size)
    if prefix_len == 0:
        return torch.empty((batch, num_heads, 0), device=query_states.device, dtype=torch.int64)
    tail_len = min(window_size, query_len)
    if tail_len == 0:          # x[:, :, -0:, :] is the whole tensor
        tail_len = query_len
    top_k = top_k_count(prefix_len, top_ratio)
    if not (kv_repeat <= 1 or key_states.shape[1] == num_heads):
        H_KV = key_states.shape[1]
        assert num_heads == H_KV * kv_repeat, (
            f"H_Q ({num_heads}) != H_KV ({H_KV}) * kv_repeat ({kv_repeat})")
    return _select(query_states, 1, key_states, prefix_len, tail_len, top_k)


def freeze_vertical_indices(query_tail: torch.Tensor, key_prefix: torch.Tensor, window_size: int,
                            top_ratio: float, kv_repeat: int) -> torch.Tensor:
    """The freeze-time call (src/ops/d_stage_kv_cache.py:131-136): the query
    tail [B, H_Q, W', D] is averaged over each GQA group, then the selector runs
    per KV head over key_prefix [B, H_KV, N - W, D] (whose own last
    window_size positions are excluded again, F3).  Returns [B, H_KV, top_k]."""
    B, HQ, WT, D = query_tail.shape
    HK = key_prefix.shape[1]
    key_len = int(key_prefix.shape[2])
    prefix_len = max(0, key_len - window_size)
    if prefix_len == 0:
        return torch.empty((B, HK, 0), device=query_tail.device, dtype=torch.int64)
    tail_len = min(window_size, WT)
    if tail_len == 0:
        tail_len = WT
    top_k = top_k_count(prefix_len, top_ratio)
    return _select(query_tail, kv_repeat, key_prefix, prefix_len, tail_len, top_k)
