"""Helpers shared by the GPU tests: move oracle arrays to the device."""

import numpy as np
import torch


def to_dev_bf16(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16).to(dev)


def state_to_device(st, dev) -> dict:
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    return dict(
        k_packed=t(st.k_packed), v_packed=t(st.v_packed),
        k_scale=t(st.k_scale), v_scale=t(st.v_scale),
        k_topk=to_dev_bf16(st.k_topk, dev), v_topk=to_dev_bf16(st.v_topk, dev),
        k_staging=to_dev_bf16(st.k_staging, dev), v_staging=to_dev_bf16(st.v_staging, dev),
        k_window=to_dev_bf16(st.k_window, dev), v_window=to_dev_bf16(st.v_window, dev),
    )


def gpu_prefill_inputs(B, HQ, HKV, N, W, seed, dev, q_len=None, plant_ratio=0.05, D=128):
    """The benchmark distribution at sizes too large to draw on the CPU,
    drawn on the GPU with a seeded device generator: q ~ N(0,1)
    [B, HQ, q_len, D] (q_len = N by default; the selector and the freeze read
    only the last W rows), k ~ N(0,1) plus a per-(KV head, channel) offset
    ~ N(0, 2), v ~ N(0,1); per (b, KV head) plant_ratio * N positions of the
    non-window prefix get key offset + 3 sqrt(D) u, u the unit mean direction
    of the KV group's last W queries.  Returns bf16 (q, k, v)."""
    import math
    g = torch.Generator(device=dev).manual_seed(seed)
    G = HQ // HKV
    QL = N if q_len is None else q_len
    q = torch.randn(B, HQ, QL, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, HKV, N, D, generator=g, device=dev)
    off = torch.randn(HKV, D, generator=g, device=dev) * math.sqrt(2.0)
    k += off[None, :, None, :]
    v = torch.randn(B, HKV, N, D, generator=g, device=dev).to(torch.bfloat16)
    n_plant = min(int(plant_ratio * N), max(0, N - W))
    if n_plant > 0:
        tail = q[:, :, -min(W, QL):].float().reshape(B, HKV, -1, D).mean(dim=2)        # [B, HKV, D]
        u = tail / tail.norm(dim=-1, keepdim=True)
        pos = torch.rand(B * HKV, N - W, generator=g, device=dev).argsort(dim=1)[:, :n_plant]
        line = (off[None] + 3.0 * math.sqrt(D) * u).reshape(B * HKV, 1, D)
        kf = k.view(B * HKV, N, D)
        kf.scatter_(1, pos[:, :, None].expand(-1, -1, D), line.expand(-1, n_plant, -1).contiguous())
    return q, k.to(torch.bfloat16), v


def np_f32(t: torch.Tensor) -> np.ndarray:
    """A bf16 / fp16 device tensor as float32 numpy values (exact)."""
    return t.float().cpu().numpy()


def layer_head_state(layer, heads):
    """The decode segments of a frozen DStageLayerCache for the KV heads
    `heads` (indices into B * H_KV) as an oracle DecodeState."""
    from oracle import hyq_oracle as O
    idx = torch.as_tensor(heads, device=layer.k_topk.device)
    take = lambda t: t.index_select(0, idx)
    D = layer.k_topk.shape[-1]
    st = O.DecodeState(
        take(layer.k_quant_packed).cpu().numpy(), take(layer.v_quant_packed).cpu().numpy(),
        take(layer.k_scale).cpu().numpy(), take(layer.v_scale).cpu().numpy(),
        np_f32(take(layer.k_topk)), np_f32(take(layer.v_topk)),
        np_f32(take(layer.k_window)), np_f32(take(layer.v_window)),
        np.zeros((len(heads), 128, D), np.float32), np.zeros((len(heads), 128, D), np.float32),
        0, layer.k_bits, layer.v_bits)
    ptr = layer._staging_ptr
    st.k_ring[:, :ptr] = np_f32(take(layer._staging_buf_k[:, :ptr]))
    st.v_ring[:, :ptr] = np_f32(take(layer._staging_buf_v[:, :ptr]))
    st.ring_ptr = ptr
    return st


def sample_heads(n, k=8, seed=0):
    """k distinct indices of range(n): the first, the last and k - 2 drawn at random."""
    if n <= k:
        return list(range(n))
    rng = np.random.default_rng(seed)
    mid = rng.choice(np.arange(1, n - 1), size=k - 2, replace=False)
    return sorted({0, n - 1, *(int(x) for x in mid)})


def exact_attention_gpu(qd, kd, vd, chunk=1024, sm_scale=None):
    """float32 causal attention on the GPU, chunked over queries, GQA by head
    index (a test reference; 2-D float32 products only)."""
    B, HQ, N, D = qd.shape
    G = HQ // kd.shape[1]
    sm = D ** -0.5 if sm_scale is None else sm_scale
    out = torch.empty(B, HQ, N, D, dtype=torch.float32, device=qd.device)
    for b in range(B):
        for h in range(HQ):
            kk = kd[b, h // G].float()
            vv = vd[b, h // G].float()
            for s in range(0, N, chunk):
                qq = qd[b, h, s:s + chunk].float()
                sc = (qq @ kk[: s + chunk].T.contiguous()) * sm
                i = torch.arange(s, s + qq.shape[0], device=qd.device)[:, None]
                j = torch.arange(sc.shape[1], device=qd.device)[None, :]
                sc = sc.masked_fill(j > i, float("-inf"))
                out[b, h, s:s + chunk] = torch.softmax(sc, dim=-1) @ vv[: s + chunk]
    return out


def bf16_bracket(out: np.ndarray, ref: np.ndarray, eps: np.ndarray) -> np.ndarray:
    """Elements where the bf16 output is NOT the bf16 rounding of some value
    within eps of ref, i.e. outside [bf16(ref - eps), bf16(ref + eps)] (RNE
    to bf16 is monotone).  Returns a boolean mask of violations."""
    from oracle import hyq_oracle as O
    lo = O.bf16_round_f64(np.asarray(ref, np.float64) - eps)
    hi = O.bf16_round_f64(np.asarray(ref, np.float64) + eps)
    return (out < lo) | (out > hi)


def cache_from_inputs(inp, k_bits=4, v_bits=4):
    """A DStageLayerCache fed the prefill of make_decode_inputs in two chunks, frozen."""
    from hyquant_amd.d_stage_kv_cache import DStageLayerCache
    layer = DStageLayerCache(0, k_bits=k_bits, v_bits=v_bits, window_size=inp.W, top_ratio=inp.rho)
    half = inp.N // 2
    kd, vd = to_dev_bf16(inp.keys, "cuda"), to_dev_bf16(inp.values, "cuda")
    layer.update_prefill(kd[:, :, :half], vd[:, :, :half])      # two prefill chunks
    layer.update_prefill(kd[:, :, half:], vd[:, :, half:])
    layer.save_query_tail(to_dev_bf16(inp.query_tail, "cuda"))
    layer.freeze(kv_repeat=inp.HQ // inp.HKV)
    return layer


def check_layer_state(layer, st):
    """A frozen layer's segments equal the oracle state bit for bit."""
    np_ = lambda t: t.cpu().numpy()
    assert np.array_equal(np_(layer.topk_indices), st.topk_idx)
    assert np.array_equal(np_(layer.k_quant_packed), st.k_packed)
    assert np.array_equal(np_(layer.v_quant_packed), st.v_packed)
    assert np.array_equal(np_(layer.k_scale).view(np.uint16), st.k_scale.view(np.uint16))
    assert np.array_equal(np_(layer.v_scale).view(np.uint16), st.v_scale.view(np.uint16))
    assert np.array_equal(np_(layer.k_topk.float()), st.k_topk)
    assert np.array_equal(np_(layer.v_topk.float()), st.v_topk)
    assert np.array_equal(np_(layer.k_window.float()), st.k_window)
    assert np.array_equal(np_(layer.v_window.float()), st.v_window)
    assert layer._staging_ptr == st.ring_ptr
    assert np.array_equal(np_(layer._staging_buf_k[:, :st.ring_ptr].float()), st.k_staging)


def _randn_bf16(rng, shape, scale=1.0):
    from oracle import hyq_oracle as O
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def first_tile_max_inputs(rng, B, HQ, HKV, N, W, T):
    """Inputs whose rows attain their maximum score at key 0, the first key
    of the first rest tile: channel 0 of every query is 3, key 0 is
    (26, 0, ..., 0) and channel 0 of every other key is 0, so key 0 scores
    about 10 (log2 units) against about 2.2 (std) for the others, while the
    others still carry most of the softmax weight.  Vertical indices avoid 0."""
    q = _randn_bf16(rng, (B, HQ, N, 128))
    q[..., 0] = 3.0
    k = _randn_bf16(rng, (B, HKV, N, 128), 1.5)
    k[..., 0] = 0.0
    k[:, :, 0, :] = 0.0
    k[:, :, 0, 0] = 26.0
    v = _randn_bf16(rng, (B, HKV, N, 128))
    P = max(0, N - W)
    vidx = np.stack([np.stack([1 + rng.permutation(P - 1)[:T] for _ in range(HQ)]) for _ in range(B)])
    return q, k, v, vidx.astype(np.int64).reshape(B, HQ, T)
