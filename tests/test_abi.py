"""CPU checks of the C ABI: libhyq.so loads, exports every symbol that
include/hyq.h declares, and rejects bad arguments on the host side before any
GPU work (no compute calls are made here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hyq.h")


def _declared():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"\b(hyq_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_symbols():
    from hyquant_amd import _lib
    assert _declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    from hyquant_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhyq.so not built")
    lib = ctypes.CDLL(_lib.LIB_PATH)
    for name in _declared():
        assert hasattr(lib, name), name


def _L():
    from hyquant_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("libhyq.so not built")
    return _lib, _lib.lib()


def test_abi_version_and_error_strings():
    _lib, L = _L()
    assert L.hyq_abi_version() == _lib.ABI_VERSION == 7
    st = L.hyq_quant_pack(None, 0, 1, 1, 128, 0, 0, 3, None, 0, 0, None, 0, None)
    assert st == _lib.HYQ_EINVAL
    assert b"nbits must be 2, 4, or 8" in L.hyq_last_error()
    with pytest.raises(ValueError, match="nbits"):
        _lib.check(st, "quantize_per_token")


def test_quant_pack_host_validation():
    _lib, L = _L()
    assert L.hyq_quant_pack(None, 0, 1, 1, 100, 0, 0, 4, None, 0, 0, None, 0, None) == _lib.HYQ_ENOTSUP
    assert L.hyq_quant_pack(None, 1, -1, 1, 128, 0, 0, 4, None, 0, 0, None, 0, None) == _lib.HYQ_EINVAL
    # empty input is a no-op
    assert L.hyq_quant_pack(None, 0, 0, 5, 128, 0, 0, 4, None, 0, 0, None, 0, None) == _lib.HYQ_OK
    # misaligned x
    assert L.hyq_quant_pack(8, 0, 1, 1, 128, 128, 128, 4, 16, 64, 64, 16, 1, None) == _lib.HYQ_EINVAL


def test_dequant_host_validation():
    _lib, L = _L()
    assert L.hyq_dequant(None, 1, 1, 128, 0, 0, 3, None, 0, None, 0, 0, None) == _lib.HYQ_EINVAL
    assert L.hyq_dequant(None, 1, 1, 100, 0, 0, 4, None, 0, None, 0, 0, None) == _lib.HYQ_ENOTSUP
    # empty input is a no-op
    assert L.hyq_dequant(None, 0, 7, 128, 0, 0, 4, None, 0, None, 0, 0, None) == _lib.HYQ_OK
    # misaligned fp16 output rows (8 is not 16-byte aligned)
    assert L.hyq_dequant(16, 1, 1, 128, 64, 64, 4, 16, 1, 8, 128, 128, None) == _lib.HYQ_EINVAL


def test_legacy_dequant_host_validation():
    _lib, L = _L()
    # 8 bits is not a legacy format width; head dim 100 is unsupported
    assert L.hyq_legacy_dequant(None, 1, 1, 128, 0, 0, 8, None, 0, 0, 128, None, 0, 0, None) == _lib.HYQ_EINVAL
    assert L.hyq_legacy_dequant(None, 1, 1, 100, 0, 0, 4, None, 0, 0, 128, None, 0, 0, None) == _lib.HYQ_ENOTSUP
    assert L.hyq_legacy_dequant(None, 1, 1, 128, 0, 0, 4, None, 0, 0, 0, None, 0, 0, None) == _lib.HYQ_EINVAL
    # empty input is a no-op
    assert L.hyq_legacy_dequant(None, 0, 7, 128, 0, 0, 4, None, 0, 0, 128, None, 0, 0, None) == _lib.HYQ_OK
    # scale rows must be 16-byte aligned (8 is not)
    assert L.hyq_legacy_dequant(16, 1, 1, 128, 64, 64, 4, 8, 128, 128, 128, 256, 128, 128, None) == _lib.HYQ_EINVAL


def _params(_lib, **kw):
    p = _lib.DecodeParams()
    p.q, p.q_stride, p.out, p.out_stride = 256, 128, 512, 128
    p.bh_kv, p.kv_repeat, p.head_dim, p.k_bits, p.v_bits = 8, 4, 128, 4, 4
    p.sm_scale = 128 ** -0.5
    p.seg_n[2] = 128
    p.seg_k[2] = 1024
    p.seg_v[2] = 2048
    p.seg_k_stride_bh[2] = p.seg_v_stride_bh[2] = 128 * 128
    p.seg_k_stride_n[2] = p.seg_v_stride_n[2] = 128
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_decode_host_validation():
    _lib, L = _L()
    p = _params(_lib)
    assert L.hyq_decode_workspace_size(p) > 0
    for bits in ((2, 4), (8, 8), (4, 2)):       # every {2, 4, 8} pair is accepted
        assert L.hyq_decode_workspace_size(_params(_lib, k_bits=bits[0], v_bits=bits[1])) > 0
    for bad, code in ((dict(head_dim=64), _lib.HYQ_ENOTSUP), (dict(k_bits=3), _lib.HYQ_EINVAL),
                      (dict(v_bits=16), _lib.HYQ_EINVAL),
                      (dict(kv_repeat=17), _lib.HYQ_ENOTSUP), (dict(q=258), _lib.HYQ_EINVAL),
                      (dict(bh_kv=-1), _lib.HYQ_EINVAL)):
        p = _params(_lib, **bad)
        assert L.hyq_decode_workspace_size(p) == 0
        assert L.hyq_decode_hybrid(p, None, 0, None) == code, bad
    # too-small workspace is refused before launch
    p = _params(_lib)
    assert L.hyq_decode_hybrid(p, 4096, 16, None) == _lib.HYQ_ENOSPC
    assert b"workspace" in L.hyq_last_error()
    # prefix pointers must be present when n_quant > 0
    p = _params(_lib, n_quant=512)
    assert L.hyq_decode_hybrid(p, 4096, 1 << 30, None) == _lib.HYQ_EINVAL
    # packed rows must be 16 * bits bytes apart
    p = _params(_lib, n_quant=512, k_bits=2, v_bits=4, k_packed=4096, v_packed=8192, k_scale=4096, v_scale=4096,
                kp_stride_bh=512 * 64, kp_stride_n=64, vp_stride_bh=512 * 64, vp_stride_n=64)
    assert L.hyq_decode_hybrid(p, 4096, 1 << 30, None) == _lib.HYQ_EINVAL
    assert b"16 * bits" in L.hyq_last_error()


def test_dtype_flags_host_validation():
    """The fp16-model switches: unknown dtype_flags bits, and is_fp16 /
    dtype_fp16 values other than 0 and 1, are EINVAL before any launch."""
    _lib, L = _L()
    ok = _lib.HYQ_DT_Q_FP16 | _lib.HYQ_DT_SEG_FP16 | _lib.HYQ_DT_OUT_FP16
    assert L.hyq_decode_workspace_size(_params(_lib, dtype_flags=ok)) > 0
    p = _params(_lib, dtype_flags=8)
    assert L.hyq_decode_workspace_size(p) == 0
    assert L.hyq_decode_hybrid(p, None, 0, None) == _lib.HYQ_EINVAL
    assert b"dtype_flags" in L.hyq_last_error()
    assert L.hyq_vertical_select(None, 0, 0, 0, 4, 2, 1, None, 0, 0, 0, 2, 10, 1, 128, 4, 3, 2,
                                 None, None, 0, None) == _lib.HYQ_EINVAL
    assert b"is_fp16" in L.hyq_last_error()
    args = [None, 0, 0, 0, None, 0, 0, 0, 1, 1, 64, 128, 16, None, 0, 4, 4, 5] + [None, 0, 0] * 2 + \
        [None, 0] * 2 + [None, 0, 0] * 4 + [None, 0, None]
    assert L.hyq_freeze_reorganise(*args) == _lib.HYQ_EINVAL
    assert b"is_fp16" in L.hyq_last_error()
    pp = _lib.PrefillParams()
    pp.batch, pp.hq, pp.hkv, pp.head_dim, pp.n, pp.t, pp.window, pp.dtype_fp16 = 1, 1, 1, 128, 64, 0, 16, 2
    assert L.hyq_prefill_hybrid(ctypes.byref(pp), None, 0, None) == _lib.HYQ_EINVAL
    assert b"dtype_fp16" in L.hyq_last_error()


def test_decode_noalloc_host_validation():
    """hyq_decode_hybrid_noalloc validates like hyq_decode_hybrid and refuses,
    before touching the device, a call whose workspace exceeds its 16 MiB
    scratch (16384 KV heads x 16 query heads: 128 MiB of partials)."""
    _lib, L = _L()
    assert L.hyq_decode_hybrid_noalloc(_params(_lib, k_bits=3), None) == _lib.HYQ_EINVAL
    assert L.hyq_decode_hybrid_noalloc(_params(_lib, bh_kv=0), None) == _lib.HYQ_OK
    p = _params(_lib, bh_kv=16384, kv_repeat=16)
    assert L.hyq_decode_workspace_size(p) > 16 << 20
    assert L.hyq_decode_hybrid_noalloc(p, None) == _lib.HYQ_ENOSPC
    assert b"scratch" in L.hyq_last_error()


def test_prefill_unified_host_validation():
    """hyq_prefill_unified takes no vertical indices: t != 0 is EINVAL
    before anything is launched."""
    from hyquant_amd import _lib
    L = _lib.lib()
    p = _lib.PrefillParams()
    p.batch, p.hq, p.hkv, p.head_dim, p.n, p.t, p.window = 1, 1, 1, 128, 64, 3, 0
    assert L.hyq_prefill_unified(ctypes.byref(p), None, 0, None) == _lib.HYQ_EINVAL
    assert b"t must be 0" in L.hyq_last_error()
    p.t = 0
    assert L.hyq_prefill_unified(ctypes.byref(p), None, 0, None) == _lib.HYQ_EINVAL    # null tensors


def test_prefill_length_limit():
    """The prefill kernels address a head's 256-byte fp16 rows with 32-bit
    byte offsets: a sequence longer than 2^24 (or that many prefix positions
    or vertical indices) is ENOTSUP before anything is launched; 2^24 itself
    passes the size checks and fails later on the null tensors."""
    from hyquant_amd import _lib
    L = _lib.lib()
    for fn in (L.hyq_prefill_hybrid, L.hyq_prefill_hybrid_fp8qk):
        p = _lib.PrefillParams()
        p.batch, p.hq, p.hkv, p.head_dim, p.n, p.t, p.window = 1, 1, 1, 128, (1 << 24) + 1, 8, 128
        assert fn(ctypes.byref(p), None, 0, None) == _lib.HYQ_ENOTSUP
        assert b"2^24" in L.hyq_last_error()
        p.n = 1 << 24
        assert fn(ctypes.byref(p), None, 0, None) == _lib.HYQ_EINVAL
        p.n, p.t = 4096, (1 << 24) + 1
        assert fn(ctypes.byref(p), None, 0, None) == _lib.HYQ_ENOTSUP
    p = _lib.PrefillParams()
    p.batch, p.hq, p.hkv, p.head_dim, p.n, p.t, p.window = 1, 1, 1, 128, (1 << 24) + 1, 0, 0
    assert L.hyq_prefill_unified(ctypes.byref(p), None, 0, None) == _lib.HYQ_ENOTSUP
    assert L.hyq_prefill_lists(None, 0, 0, 0, 1, 1, (1 << 24) + 1, 8, 0, None, None, None, None, None,
                               None, 0, None) == _lib.HYQ_ENOTSUP


def test_select_top_k_limit():
    """The selector's sort size is the power of two above top_k, kept in an
    int: top_k above 2^30 is ENOTSUP before anything is launched."""
    _lib, L = _L()
    st = L.hyq_vertical_select(16, 0, 0, 128, 1, 1, 1, 16, 0, 0, 128, 1, (1 << 31) - 1, 1, 128, 1,
                               (1 << 30) + 1, 0, 16, None, 0, None)
    assert st == _lib.HYQ_ENOTSUP
    assert b"2^30" in L.hyq_last_error()
    assert L.hyq_vertical_select_workspace_size(1, 1, (1 << 31) - 1, (1 << 30) + 1) == 0


def test_bf16_workspace_size():
    _lib, L = _L()
    assert L.hyq_decode_bf16_workspace_size(8, 4, 8192, 128) > 8 * 4 * 128 * 4
    assert L.hyq_decode_bf16_workspace_size(8, 4, 8192, 64) == 0


def test_python_layer_rejects_cpu_tensors():
    import torch
    import hyquant_amd as hq
    with pytest.raises(ValueError, match="GPU"):
        hq.quantize_per_token(torch.zeros(1, 1, 128, dtype=torch.bfloat16), 4)
    with pytest.raises(ValueError, match="nbits"):
        hq.quantize_per_token(torch.zeros(1, 1, 128, dtype=torch.bfloat16), 5)


def _legacy_params(_lib, **kw):
    p = _lib.LegacyParams()
    p.q, p.q_stride, p.out, p.out_stride = 256, 128, 512, 128
    p.k_codes, p.kc_stride_bh, p.kc_stride_n = 4096, 1000 * 64, 64
    p.v_codes, p.vc_stride_bh, p.vc_stride_n = 8192, 1000 * 64, 64
    p.k_scale, p.ks_stride_bh, p.ks_stride_g = 16384, 8 * 128, 128
    p.v_scale, p.vs_stride_bh, p.vs_stride_g = 32768, 8 * 128, 128
    p.n, p.group = 1000, 128
    p.k_bits = p.v_bits = 4
    p.seg_n[0] = 37
    p.seg_k[0], p.seg_v[0] = 65536, 131072
    p.seg_k_stride_bh[0] = p.seg_v_stride_bh[0] = 37 * 128
    p.bh_kv, p.kv_repeat, p.head_dim = 8, 4, 128
    p.sm_scale = 128 ** -0.5
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_legacy_host_validation():
    """hyq_decode_legacy's checks run on the host before any launch: a valid
    parameter block gets a workspace size (arrival counters, then the (m, l)
    table and partials of its pieces); each invalid one gets size 0
    and its status, and a valid call without a workspace is refused.  Code
    rows are checked against the loads of their bit width: a 4*k_bits-byte K
    load and v_bits-byte V loads per lane, rows of at least 16*bits bytes."""
    _lib, L = _L()
    p = _legacy_params(_lib)
    need = L.hyq_decode_legacy_workspace_size(p)
    assert need > 2 << 20
    assert L.hyq_decode_legacy(p, None, 0, None) == _lib.HYQ_ENOSPC
    # 2-bit rows: 32-byte strides, K rows 8-byte and V rows 2-byte aligned
    for kw in (dict(k_bits=2, kc_stride_n=32, k_codes=4104), dict(v_bits=2, vc_stride_n=32, v_codes=8194),
               dict(k_bits=2, v_bits=2, kc_stride_n=40, vc_stride_n=34)):
        p = _legacy_params(_lib, **kw)
        assert L.hyq_decode_legacy_workspace_size(p) > 0, kw
        assert L.hyq_decode_legacy(p, None, 0, None) == _lib.HYQ_ENOSPC, kw
    bad = ((dict(head_dim=64), _lib.HYQ_ENOTSUP), (dict(kv_repeat=17), _lib.HYQ_ENOTSUP),
           (dict(k_bits=3), _lib.HYQ_ENOTSUP), (dict(v_bits=8), _lib.HYQ_ENOTSUP),
           (dict(group=100), _lib.HYQ_EINVAL), (dict(kc_stride_n=48), _lib.HYQ_EINVAL),
           (dict(k_codes=4100), _lib.HYQ_EINVAL), (dict(v_codes=8194), _lib.HYQ_EINVAL),
           (dict(k_bits=2, kc_stride_n=32, k_codes=4100), _lib.HYQ_EINVAL),
           (dict(k_bits=2, kc_stride_n=24), _lib.HYQ_EINVAL),
           (dict(v_bits=2, vc_stride_n=32, v_codes=8193), _lib.HYQ_EINVAL),
           (dict(v_bits=2, vc_stride_n=30), _lib.HYQ_EINVAL),
           (dict(ks_stride_g=120), _lib.HYQ_EINVAL), (dict(q=258), _lib.HYQ_EINVAL),
           (dict(n=(1 << 24) + 1), _lib.HYQ_ENOTSUP), (dict(bh_kv=16385), _lib.HYQ_ENOTSUP))
    for kw, code in bad:
        p = _legacy_params(_lib, **kw)
        assert L.hyq_decode_legacy_workspace_size(p) == 0, kw
        assert L.hyq_decode_legacy(p, None, 0, None) == code, kw
    p = _legacy_params(_lib, n=0)
    p.seg_n[0] = 0
    assert L.hyq_decode_legacy(p, None, 0, None) == _lib.HYQ_EINVAL
    assert b"zero key tokens" in L.hyq_last_error()
