"""Decode-stage operators on MI355X: per-token quantisation and the fused
four-segment hybrid decode attention.

Drop-in for the reference's `src/ops/decode_d_stage.py`: same function names,
argument meaning, output allocation and exceptions.  Every call runs the HIP
kernels of libhyq.so on the current HIP stream of the input's device.
"""

from __future__ import annotations

import ctypes
import math
import struct
import threading
from typing import Optional, Tuple

import torch

from . import _lib

GROUP_SIZE = 128  # staging flush threshold (src/ops/decode_d_stage.py:19)
_LOG2_E = 1.44269504

# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(device: torch.device) -> int:
    """The current HIP stream of `device` as a pointer value (torch's raw
    accessor when it has one: the Stream object costs microseconds a call)."""
    if _raw_stream is not None and device.index is not None:
        return _raw_stream(device.index)
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor (no CPU implementation)")


def _inner_contig(t: torch.Tensor) -> torch.Tensor:
    """The kernels take any head stride (a multiple of 16 bytes) but need each
    head's rows packed back to back (token stride = row length) and 16-byte
    aligned; anything else gets a contiguous copy."""
    es = t.element_size()
    if t.is_contiguous() and t.data_ptr() % 16 == 0 and (t.shape[-1] * es) % 16 == 0:
        return t                       # the common case, decided in three calls
    if t.numel() == 0:
        return t
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and (t.dim() < 3 or t.stride(-2) == t.shape[-1])
          and all((s * es) % 16 == 0 for s in t.stride()[:-1]))
    return t if ok else t.contiguous()


_ws_lock = threading.Lock()
_ws_cache: dict = {}
_ws_raw: dict = {}          # (device, stream) -> (pointer, bytes) of the cached workspace


def _workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    """Split-K workspace (arrival counters + partials), cached per (device,
    stream) like the reference's split-K buffers
    (src/ops/decode_d_stage.py:797-811).  It is zero-filled once when
    allocated (the counters must start at zero; every call leaves them at
    zero).  Calls on one stream are ordered; different streams get their own
    buffer."""
    key = (device.index, stream)
    with _ws_lock:
        buf = _ws_cache.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
            _ws_cache[key] = buf
            _ws_raw[key] = (buf.data_ptr(), buf.numel())
        return buf


def _packed_dim(D: int, bits: int) -> int:
    return D // 4 if bits == 2 else D // 2 if bits == 4 else D


# ---------------------------------------------------------------------------
# quantisation (src/ops/decode_d_stage.py:50-163)
# ---------------------------------------------------------------------------


_HALF = (torch.bfloat16, torch.float16)


def quantize_per_token(x: torch.Tensor, nbits: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-token symmetric quantisation.

    x: [BH, N, D] bf16 or fp16 -> (packed int8 [BH, N, D*nbits/8], scale fp16 [BH, N]).
    Bit-exact with src/ops/decode_d_stage.py:50-77.
    """
    if nbits not in (2, 4, 8):
        raise ValueError(f"nbits must be 2, 4, or 8, got {nbits}")
    _require_gpu(x, "x")
    if x.dtype not in _HALF:
        raise ValueError(f"quantize_per_token expects bf16 or fp16 input, got {x.dtype}")
    BH, N, D = x.shape
    packed = torch.empty(BH, N, _packed_dim(D, nbits), dtype=torch.int8, device=x.device)
    scale = torch.empty(BH, N, dtype=torch.float16, device=x.device)
    quantize_into(x, nbits, packed, scale)
    return packed, scale


def quantize_into(x: torch.Tensor, nbits: int, packed: torch.Tensor, scale: torch.Tensor) -> None:
    """Quantise x [BH, N, D] into preallocated (possibly strided) outputs, e.g.
    the tail of a capacity-allocated prefix store (staging flush)."""
    BH, N, D = x.shape
    if BH * N == 0:
        return
    x = _inner_contig(x)
    if x.stride(-1) != 1:
        x = x.contiguous()
    if packed.stride(-1) != 1 or scale.stride(-1) != 1:
        raise ValueError("packed/scale outputs must be contiguous in the last dim")
    if x.dtype not in _HALF:
        raise ValueError(f"quantize_per_token expects bf16 or fp16 input, got {x.dtype}")
    st = _lib.lib().hyq_quant_pack(
        x.data_ptr(), int(x.dtype == torch.float16), BH, N, D, x.stride(0), x.stride(1), nbits,
        packed.data_ptr(), packed.stride(0), packed.stride(1),
        scale.data_ptr(), scale.stride(0), _stream(x.device))
    _lib.check(st, "quantize_per_token")


def _unpack_int4(packed: torch.Tensor, D: int) -> torch.Tensor:
    x = packed.to(torch.int32) & 0xFF
    lo = ((x & 0x0F) << 28) >> 28
    hi = (((x >> 4) & 0x0F) << 28) >> 28
    return torch.stack([lo, hi], dim=-1).reshape(*packed.shape[:-1], D).float()


def _unpack_int2(packed: torch.Tensor, D: int) -> torch.Tensor:
    x = packed.to(torch.int32) & 0xFF
    parts = [(((x >> (2 * j)) & 0x03) << 30) >> 30 for j in range(4)]
    return torch.stack(parts, dim=-1).reshape(*packed.shape[:-1], D).float()


def dequantize_per_token(packed: torch.Tensor, scale: torch.Tensor, D: int, nbits: int) -> torch.Tensor:
    """[BH, N, D_packed] + [BH, N] -> fp16 [BH, N, D] = fp16(code * scale)
    (src/ops/decode_d_stage.py:80-101), by the hyq_dequant kernel.  The fused
    decode never calls it (it dequantises in registers); the eager decode
    path and the bf16 round trip of a quantised cache do."""
    if nbits not in (2, 4, 8):
        raise ValueError(f"nbits must be 2, 4, or 8, got {nbits}")
    _require_gpu(packed, "packed")
    BH, N, DP = packed.shape
    if DP != _packed_dim(D, nbits):
        raise ValueError(f"packed rows hold {DP} bytes, expected {_packed_dim(D, nbits)} for D={D}, {nbits} bits")
    if packed.dtype != torch.int8 or scale.dtype != torch.float16 or tuple(scale.shape) != (BH, N):
        raise ValueError("dequantize_per_token expects int8 packed [BH, N, D_packed] and fp16 scale [BH, N]")
    out = torch.empty(BH, N, D, dtype=torch.float16, device=packed.device)
    if BH * N == 0:
        return out
    if packed.stride(-1) != 1:
        packed = packed.contiguous()
    if scale.stride(-1) != 1:
        scale = scale.contiguous()
    st = _lib.lib().hyq_dequant(packed.data_ptr(), BH, N, D, packed.stride(0), packed.stride(1), nbits,
                                scale.data_ptr(), scale.stride(0), out.data_ptr(), out.stride(0), out.stride(1),
                                _stream(packed.device))
    _lib.check(st, "dequantize_per_token")
    return out


def _quantize_by_bits(x: torch.Tensor, bits: int):
    """Alias kept for drop-in compatibility (src/ops/decode_d_stage.py:156-158)."""
    return quantize_per_token(x, bits)


def _dequantize_by_bits(packed, scale, D, bits):
    return dequantize_per_token(packed, scale, D, bits)


# ---------------------------------------------------------------------------
# fused decode (src/ops/decode_d_stage.py:916-1005)
# ---------------------------------------------------------------------------


def _fill_segment(p: _lib.DecodeParams, i: int, k: torch.Tensor, v: torch.Tensor) -> list:
    keep = []
    n = k.shape[1]
    p.seg_n[i] = n
    if n == 0:
        p.seg_k[i] = None
        p.seg_v[i] = None
        return keep
    k = _inner_contig(k)
    v = _inner_contig(v)
    keep += [k, v]
    p.seg_k[i] = k.data_ptr()
    p.seg_v[i] = v.data_ptr()
    p.seg_k_stride_bh[i], p.seg_k_stride_n[i] = k.stride(0), k.stride(1)
    p.seg_v_stride_bh[i], p.seg_v_stride_n[i] = v.stride(0), v.stride(1)
    return keep


def fused_d_stage_decode(
    q: torch.Tensor,                        # [BH_Q, D]
    k_quant_packed: torch.Tensor,           # [BH_KV, N_quant, D*k_bits/8] int8
    v_quant_packed: torch.Tensor,
    k_scale: torch.Tensor,                  # [BH_KV, N_quant] fp16
    v_scale: torch.Tensor,
    k_topk: torch.Tensor,                   # [BH_KV, N_topk, D] bf16
    v_topk: torch.Tensor,
    k_staging: torch.Tensor,                # [BH_KV, N_staging, D]
    v_staging: torch.Tensor,
    k_window: torch.Tensor,                 # [BH_KV, N_window, D]
    v_window: torch.Tensor,
    k_bits: int,
    v_bits: int,
    kv_repeat: int = 1,
    sm_scale: Optional[float] = None,
    split_tokens: int = 0,
) -> torch.Tensor:
    """Fused four-segment decode: quantised prefix (K and V codes of 2, 4 or 8
    bits) + top-k + staging + window under one online softmax.  Returns a new
    [BH_Q, D] tensor of q.dtype.  q and the segments may be bf16 or fp16
    (one dtype for the segments): fp16 values are rounded to bf16 before the
    products, as the reference's kernels do (src/ops/decode_d_stage.py:537-541),
    and the fp32 result is rounded once to q.dtype (:866)."""
    fx = _FX if _FX is not None else _load_fast_ext()
    if fx:
        dev = q.get_device() if isinstance(q, torch.Tensor) else -1
        if dev >= 0:
            stream = _raw_stream(dev) if _raw_stream is not None else torch.cuda.current_stream(dev).cuda_stream
            w = _ws_raw.get((dev, stream), _NO_WS)
            try:
                st, out = fx.decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging,
                                    v_staging, k_window, v_window, k_bits, v_bits, kv_repeat,
                                    _NAN if sm_scale is None else sm_scale, split_tokens, stream, w[0], w[1])
            except TypeError:
                st = -1
            if st == 0:
                return out
    out = _fast_decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging, v_staging,
                       k_window, v_window, k_bits, v_bits, kv_repeat, sm_scale, split_tokens)
    if out is not None:
        return out
    return _decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging, v_staging,
                   k_window, v_window, k_bits, v_bits, kv_repeat, sm_scale, split_tokens, None, None)


# ---------------------------------------------------------------------------
# the per-call host path
# ---------------------------------------------------------------------------
# A decode call is a few microseconds of GPU time, so the host side of an
# eager call matters (once per layer per token in HF generate()).  The fast
# path reads each tensor's data pointer, stride tuple and shape once, packs
# every field of hyq_decode_params with one precompiled struct.pack_into into
# a per-thread parameter block, and makes one library call, which validates
# (alignment, strides, sizes) and launches.  Whatever the fast path does not
# take (a non-unit channel stride, mixed segment dtypes, a bad argument the
# library rejects with EINVAL) goes through the checked path (_decode), which
# copies, or raises the reference's errors; a rejected call launches nothing.


def _params_struct() -> struct.Struct:
    """struct.Struct of hyq_decode_params in field order, built from the
    ctypes mirror's offsets (little-endian, explicit padding)."""
    codes = {ctypes.c_void_p: "Q", ctypes.c_int64: "q", ctypes.c_int32: "i", ctypes.c_float: "f"}
    fmt, pos = "<", 0
    for name, ctype in _lib.DecodeParams._fields_:
        off = getattr(_lib.DecodeParams, name).offset
        if off > pos:
            fmt += f"{off - pos}x"
        base, count = (ctype._type_, ctype._length_) if hasattr(ctype, "_length_") else (ctype, 1)
        fmt += (str(count) if count > 1 else "") + codes[base]
        pos = off + ctypes.sizeof(ctype)
    size = ctypes.sizeof(_lib.DecodeParams)
    if size > pos:
        fmt += f"{size - pos}x"
    st = struct.Struct(fmt)
    assert st.size == size, (st.size, size)
    return st


_PSTRUCT = None
_HYB = None
# The C++ form of the fast path (hyquant_amd/_hyq_fast.so, built by
# build.build_fast_ext): the same checks and the same parameter block, with
# the tensors' metadata read natively (about 3 us less host time per call).
# A status other than 0 (not taken, workspace missing or too small, a
# rejected argument) falls through to the Python fast path and then to the
# checked path, which handle each case.  None: not loaded yet; False: absent
# or built for a different parameter layout.
_FX = None
_NAN = float("nan")
_NO_WS = (0, 0)


def _load_fast_ext():
    global _FX
    import importlib.util
    import os
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_hyq_fast.so")
    mod = False
    if os.path.exists(path):
        spec = importlib.util.spec_from_file_location("hyquant_amd._hyq_fast", path)
        m = importlib.util.module_from_spec(spec)
        try:
            spec.loader.exec_module(m)
        except (ImportError, OSError):
            # built against another torch: the Python paths take every call
            _FX = False
            return False
        P = _lib.DecodeParams
        if m.layout() == (ctypes.sizeof(P), P.seg_n.offset, P.dtype_flags.offset):
            m.set_entry(ctypes.cast(_lib.lib().hyq_decode_hybrid, ctypes.c_void_p).value)
            mod = m
    _FX = mod
    return mod
_tls = threading.local()
_BF16, _FP16 = torch.bfloat16, torch.float16


def _seg(k, v):
    """(k pointer, k head stride, k token stride, v pointer, v head stride,
    v token stride, tokens, dtype) of one bf16 segment, or None when the
    segment needs the checked path (channels not contiguous, K and V of
    different lengths or dtypes)."""
    n = k.shape[1]
    if n == 0:
        return (0, 0, 0, 0, 0, 0, 0, None)
    a, b = k.stride(), v.stride()
    d = k.dtype
    if a[2] != 1 or b[2] != 1 or v.shape[1] != n or v.dtype is not d or (d is not _BF16 and d is not _FP16):
        return None
    return (k.data_ptr(), a[0], a[1], v.data_ptr(), b[0], b[1], n, d)


def _fast_decode(q, kp, vp, ks, vs, kt, vt, kst, vst, kw, vw, k_bits, v_bits, kv_repeat, sm_scale, split_tokens):
    """The eager fast path of fused_d_stage_decode; None when the call must
    take the checked path (nothing was launched then).  Tensors of the wrong
    rank fail an index or unpacking here and take the checked path too."""
    global _PSTRUCT, _HYB
    try:
        qdt = q.dtype
        if qdt is _BF16:
            flags = 0
        elif qdt is _FP16:
            flags = 5                                  # HYQ_DT_Q_FP16 | HYQ_DT_OUT_FP16
        else:
            return None
        BH_Q, D = q.shape
        qs = q.stride()
        if qs[1] != 1 or kv_repeat < 1 or BH_Q % kv_repeat or not q.is_cuda:
            return None
        s0, s1, s2 = _seg(kt, vt), _seg(kst, vst), _seg(kw, vw)
        if s0 is None or s1 is None or s2 is None:
            return None
        dts = {s0[7], s1[7], s2[7]}
        dts.discard(None)
        if len(dts) > 1:
            return None
        if _FP16 in dts:
            flags |= 2                                 # HYQ_DT_SEG_FP16
        nq = kp.shape[1]
        if nq > 0:
            a, b, c, e = kp.stride(), vp.stride(), ks.stride(), vs.stride()
            if a[2] != 1 or b[2] != 1 or c[1] != 1 or e[1] != 1:
                return None
            kpp, vpp, ksp, vsp = kp.data_ptr(), vp.data_ptr(), ks.data_ptr(), vs.data_ptr()
        else:
            a = b = c = e = (0, 0, 0)
            kpp = vpp = ksp = vsp = 0
    except (IndexError, ValueError, TypeError, AttributeError):
        return None
    out = torch.empty_like(q, memory_format=torch.contiguous_format)
    t = _tls
    p = getattr(t, "p", None)
    if p is None:
        if _PSTRUCT is None:
            _PSTRUCT = _params_struct()
            _HYB = _lib.lib().hyq_decode_hybrid
        p = t.p = _lib.DecodeParams()
        t.ref = ctypes.byref(p)
    _PSTRUCT.pack_into(
        p, 0, q.data_ptr(), qs[0], out.data_ptr(), D, kpp, a[0], a[1], vpp, b[0], b[1], ksp, c[0], vsp, e[0], nq,
        s0[0], s1[0], s2[0], s0[1], s1[1], s2[1], s0[2], s1[2], s2[2],
        s0[3], s1[3], s2[3], s0[4], s1[4], s2[4], s0[5], s1[5], s2[5],
        s0[6], s1[6], s2[6], BH_Q // kv_repeat, kv_repeat, D, k_bits, v_bits,
        D ** -0.5 if sm_scale is None else float(sm_scale), int(split_tokens), 0, 0, flags)
    dev = q.get_device()
    stream = _raw_stream(dev) if _raw_stream is not None else torch.cuda.current_stream(dev).cuda_stream
    ws = _ws_cache.get((dev, stream))
    st = _HYB(t.ref, ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, stream)
    if st == _lib.HYQ_ENOSPC:
        L = _lib.lib()
        ws = _workspace(q.device, stream, L.hyq_decode_workspace_size(t.ref))
        st = _HYB(t.ref, ws.data_ptr(), ws.numel(), stream)
    if st == _lib.HYQ_EINVAL:
        return None
    _lib.check(st, "fused_d_stage_decode")
    return out


def _decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging, v_staging,
            k_window, v_window, k_bits, v_bits, kv_repeat, sm_scale, split_tokens, lens_q, lens_s0):
    p, keep, out = decode_params(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging,
                                 v_staging, k_window, v_window, k_bits, v_bits, kv_repeat, sm_scale, split_tokens,
                                 lens_q, lens_s0)
    L = _lib.lib()
    need = L.hyq_decode_workspace_size(p)
    if need == 0:
        _lib.check(L.hyq_decode_hybrid(p, None, 0, None), "fused_d_stage_decode")
    stream = _stream(q.device)
    ws = _workspace(q.device, stream, need)
    st = L.hyq_decode_hybrid(p, ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, "fused_d_stage_decode")
    return out


def decode_params(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_topk, v_topk, k_staging, v_staging,
                  k_window, v_window, k_bits, v_bits, kv_repeat=1, sm_scale=None, split_tokens=0, lens_q=None,
                  lens_s0=None):
    """The hyq_decode_params of a fused_d_stage_decode call: returns (params,
    tensors that must stay alive while the call runs, the output tensor)."""
    _require_gpu(q, "q")
    if q.dtype not in _HALF:
        raise ValueError(f"fused_d_stage_decode expects bf16 or fp16 q, got {q.dtype}")
    segs = (k_topk, v_topk, k_staging, v_staging, k_window, v_window)
    seg_dtypes = {t.dtype for t in segs if t.shape[1] > 0}
    if not seg_dtypes <= set(_HALF) or len(seg_dtypes) > 1:
        raise ValueError(f"the top-k / staging / window segments must share one dtype, bf16 or fp16; "
                         f"got {sorted(str(d) for d in seg_dtypes)}")
    # an fp16 model: q and the segments are rounded to bf16 inside the kernel
    # (the reference's .to(tl.bfloat16) of its loads) and the result is fp16
    flags = 0
    if q.dtype == torch.float16:
        flags |= _lib.HYQ_DT_Q_FP16 | _lib.HYQ_DT_OUT_FP16
    if torch.float16 in seg_dtypes:
        flags |= _lib.HYQ_DT_SEG_FP16
    if k_bits not in (2, 4, 8) or v_bits not in (2, 4, 8):
        raise ValueError(f"k_bits and v_bits must be 2, 4, or 8, got {k_bits}, {v_bits}")
    BH_Q, D = q.shape
    if BH_Q % kv_repeat:
        raise ValueError(f"BH_Q ({BH_Q}) is not a multiple of kv_repeat ({kv_repeat})")
    BH_KV = BH_Q // kv_repeat
    if sm_scale is None:
        sm_scale = D ** -0.5
    out = torch.empty(BH_Q, D, device=q.device, dtype=q.dtype)
    q = _inner_contig(q)
    p = _lib.DecodeParams()
    keep = [q]
    p.q, p.q_stride = q.data_ptr(), q.stride(0)
    p.out, p.out_stride = out.data_ptr(), out.stride(0)
    n_quant = k_quant_packed.shape[1]
    p.n_quant = n_quant
    if n_quant > 0:
        kp = _inner_contig(k_quant_packed)
        vp = _inner_contig(v_quant_packed)
        ks = k_scale if k_scale.stride(-1) == 1 else k_scale.contiguous()
        vs = v_scale if v_scale.stride(-1) == 1 else v_scale.contiguous()
        keep += [kp, vp, ks, vs]
        p.k_packed, p.kp_stride_bh, p.kp_stride_n = kp.data_ptr(), kp.stride(0), kp.stride(1)
        p.v_packed, p.vp_stride_bh, p.vp_stride_n = vp.data_ptr(), vp.stride(0), vp.stride(1)
        p.k_scale, p.ks_stride_bh = ks.data_ptr(), ks.stride(0)
        p.v_scale, p.vs_stride_bh = vs.data_ptr(), vs.stride(0)
    for i, (k, v) in enumerate(((k_topk, v_topk), (k_staging, v_staging), (k_window, v_window))):
        keep += _fill_segment(p, i, k, v)
    p.bh_kv, p.kv_repeat, p.head_dim = BH_KV, kv_repeat, D
    p.k_bits, p.v_bits = k_bits, v_bits
    p.sm_scale = float(sm_scale)
    p.split_tokens = int(split_tokens)
    p.dtype_flags = flags
    if lens_q is not None:
        keep += [lens_q, lens_s0]
        p.seq_lens_quant, p.seq_lens_seg0 = lens_q.data_ptr(), lens_s0.data_ptr()
    return p, keep, out


# the reference's split-K entry point is the same operator here
fused_d_stage_decode_splitk = fused_d_stage_decode


def fused_d_stage_decode_batched(
    q: torch.Tensor,                        # [total_BH_Q, D]
    k_quant_packed: torch.Tensor,           # [total_BH_KV, max_N_quant, D*k_bits/8]
    v_quant_packed: torch.Tensor,
    k_scale: torch.Tensor,                  # [total_BH_KV, max_N_quant]
    v_scale: torch.Tensor,
    k_bf16: torch.Tensor,                   # [total_BH_KV, max_N_bf16, D]
    v_bf16: torch.Tensor,
    seq_lens_quant: torch.Tensor,           # [total_BH_KV] valid prefix tokens per head
    seq_lens_bf16: torch.Tensor,            # [total_BH_KV] valid bf16 tokens per head
    k_bits: int,
    v_bits: int,
    kv_repeat: int = 1,
    sm_scale: Optional[float] = None,
) -> torch.Tensor:
    """Several sequences of different lengths in one call
    (src/ops/decode_d_stage.py:1008-1129): the heads of all sequences are
    stacked along BH, each padded to the longest prefix / bf16 segment, and
    the per-head lengths bound what is attended.  The bf16 segment is the
    concatenated top-k / staging / window part of each head."""
    _require_gpu(q, "q")
    BH_KV = q.shape[0] // max(kv_repeat, 1)
    for name, t in (("seq_lens_quant", seq_lens_quant), ("seq_lens_bf16", seq_lens_bf16)):
        if t.numel() != BH_KV:
            raise ValueError(f"{name} must hold one length per KV head ({BH_KV}), got {t.numel()}")
    lq = seq_lens_quant.to(device=q.device, dtype=torch.int32).contiguous()
    lb = seq_lens_bf16.to(device=q.device, dtype=torch.int32).contiguous()
    e = k_bf16[:, :0]
    return _decode(q, k_quant_packed, v_quant_packed, k_scale, v_scale, k_bf16, v_bf16, e, e, e, e,
                   k_bits, v_bits, kv_repeat, sm_scale, 0, lq, lb)


def decode_bf16_full(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_repeat: int = 1,
                     sm_scale: Optional[float] = None) -> torch.Tensor:
    """Full-precision comparator: q [BH_Q, D], k/v [BH_KV, N, D] bf16."""
    _require_gpu(q, "q")
    BH_Q, D = q.shape
    BH_KV, N, _ = k.shape
    if sm_scale is None:
        sm_scale = D ** -0.5
    q = _inner_contig(q)
    k = _inner_contig(k)
    v = _inner_contig(v)
    out = torch.empty(BH_Q, D, device=q.device, dtype=q.dtype)
    L = _lib.lib()
    need = L.hyq_decode_bf16_workspace_size(BH_KV, kv_repeat, N, D)
    stream = _stream(q.device)
    ws = _workspace(q.device, stream, max(need, 1))
    st = L.hyq_decode_bf16(q.data_ptr(), q.stride(0), out.data_ptr(), out.stride(0),
                           k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
                           N, BH_KV, kv_repeat, D, float(sm_scale), ws.data_ptr(), ws.numel(), stream)
    _lib.check(st, "decode_bf16_full")
    return out
