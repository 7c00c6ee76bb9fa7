"""Build recipe for libhyq.so (hipcc, gfx950 only).

Run `python -m hyquant_amd.build` or call `build()`; the library is written
next to this file so that it travels with the source tree.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libhyq.so")

SOURCES = ["status.hip", "quant.hip", "decode.hip", "select.hip", "prefill.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # packed-fp32 VALU forms are kept out of every kernel
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # IEEE-correct fp32 division (quantisation scales / codes are bit-exact)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-ffp-contract=off",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    return os.path.join(rocm, "bin", "hipcc")


# the phase-trace build of the decode kernel (s_memrealtime stamps per
# workgroup, read back with hyq_phase_trace_read; see bench.py --phase-trace)
TRACE_LIB = os.path.join(HERE, "libhyq_trace.so")


# the eager fast path of fused_d_stage_decode: a host-only Python extension
# (g++ against torch's headers; it calls libhyq.so through an address the
# Python side hands it, so it has no link dependency on the library)
FAST_EXT = os.path.join(HERE, "_hyq_fast.so")


def build_fast_ext(verbose: bool = False) -> str:
    import sysconfig

    import torch.utils.cpp_extension as ce
    inc = ce.include_paths() + [sysconfig.get_paths()["include"]]
    libs = ce.library_paths()
    import torch
    abi = int(bool(torch._C._GLIBCXX_USE_CXX11_ABI))
    tmp = FAST_EXT + ".tmp"
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-DTORCH_EXTENSION_NAME=_hyq_fast",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}", *[f"-I{i}" for i in inc],
           os.path.join(CSRC, "fastpath.cpp"), *[f"-L{d}" for d in libs], *[f"-Wl,-rpath,{d}" for d in libs],
           "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed ({proc.returncode}):\n{' '.join(cmd)}\n{proc.stderr}")
    if verbose and proc.stderr.strip():
        print(proc.stderr, file=sys.stderr)
    os.replace(tmp, FAST_EXT)
    return FAST_EXT


def build(verbose: bool = False, trace: bool = False) -> str:
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    out = TRACE_LIB if trace else LIB
    tmp = out + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, *(["-DHYQ_PHASE_TRACE"] if trace else []), "-o", tmp, *srcs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True, trace="--trace" in sys.argv[1:]))
    if "--trace" not in sys.argv[1:]:
        print(build_fast_ext(verbose=True))
