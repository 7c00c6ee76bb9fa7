"""CPU checks of the decode call's host path: the precompiled parameter
packing writes exactly the fields of hyq_decode_params, and calls the fast
path cannot take (CPU tensors, mixed segment dtypes, non-unit channel
strides) fall through to the checked path."""

import ctypes
import re

import torch

from hyquant_amd import _lib
from hyquant_amd import decode_d_stage as dd


def test_packed_params_match_the_ctypes_layout():
    st = dd._params_struct()
    assert st.size == ctypes.sizeof(_lib.DecodeParams)
    kinds = "".join(m.group(2) * int(m.group(1) or 1) for m in re.finditer(r"(\d*)([Qqif])", st.format))
    vals = [float(i) + 0.5 if c == "f" else i * 1000003 for i, c in enumerate(kinds, 1)]
    p = _lib.DecodeParams()
    st.pack_into(p, 0, *vals)
    got = []
    for name, _ in _lib.DecodeParams._fields_:
        x = getattr(p, name)
        got += list(x) if hasattr(x, "__len__") else [x]
    assert got == vals


def test_fast_path_declines_what_it_cannot_take():
    bf = torch.bfloat16
    q = torch.zeros(32, 128, dtype=bf)
    kp = torch.zeros(8, 16, 64, dtype=torch.int8)
    ks = torch.zeros(8, 16, dtype=torch.float16)
    seg = lambda n, dt=bf: torch.zeros(8, n, 128, dtype=dt)
    args = [q, kp, kp, ks, ks, seg(4), seg(4), seg(2), seg(2), seg(8), seg(8), 4, 4, 4, None, 0]
    assert dd._fast_decode(*args) is None                     # CPU tensors
    # a transposed segment (channel stride != 1) and mixed segment dtypes are
    # declined before anything else (no device needed to decide)
    t = args.copy()
    t[5] = seg(128).transpose(1, 2)
    assert dd._seg(t[5], t[6]) is None
    assert dd._seg(seg(4), seg(4, torch.float16)) is None
    assert dd._seg(seg(4), seg(5)) is None
    assert dd._seg(seg(0), seg(0))[6] == 0


def test_fast_extension_layout_and_declines():
    """The C++ form of the fast path (built by build.build_fast_ext) sees the
    same parameter layout as the ctypes mirror, and declines (status -1,
    nothing launched) what it cannot take: CPU tensors, a wrong rank, a
    transposed segment, mixed segment dtypes."""
    import os
    import pytest
    path = os.path.join(os.path.dirname(dd.__file__), "_hyq_fast.so")
    if not os.path.exists(path):
        pytest.skip("hyquant_amd/_hyq_fast.so not built (python -m hyquant_amd.build)")
    fx = dd._load_fast_ext()
    assert fx, "the extension was built for a different hyq_decode_params layout"
    P = _lib.DecodeParams
    assert fx.layout() == (ctypes.sizeof(P), P.seg_n.offset, P.dtype_flags.offset)
    bf = torch.bfloat16
    q = torch.zeros(32, 128, dtype=bf)
    kp = torch.zeros(8, 16, 64, dtype=torch.int8)
    ks = torch.zeros(8, 16, dtype=torch.float16)
    seg = lambda n, dt=bf: torch.zeros(8, n, 128, dtype=dt)
    base = [q, kp, kp, ks, ks, seg(4), seg(4), seg(2), seg(2), seg(8), seg(8), 4, 4, 4, float("nan"), 0, 0, 0, 0]
    assert fx.decode(*base)[0] == -1                          # CPU tensors
    for i, bad in ((0, torch.zeros(32, 128, 1, dtype=bf)), (5, seg(128).transpose(1, 2)),
                   (7, seg(2, torch.float16)), (1, torch.zeros(8, 16, dtype=torch.int8))):
        t = list(base)
        t[i] = bad
        if i == 7:
            t[8] = seg(2, torch.float16)
        assert fx.decode(*t)[0] == -1, i
