"""The decode kernel's asynchronous kernel-argument loads (CPU, compiles the
device code to assembly).

decode_kernel issues the scalar loads of its epilogue argument block (output,
partials, (m, l) table, counters) early, inside an asm statement the compiler
does not see as pending, and waits for them with an explicit lgkmcnt wait once
the stream is done.  That is correct only while the compiler neither reads nor
copies those SGPRs before the wait: a spill (v_writelane) or a move of the
destination registers in between would copy stale values that later serve as
pointers.  This test compiles decode.hip for gfx950 and checks, in every
decode_kernel instance, that no instruction between such a load and the next
lgkmcnt wait reads its destination registers."""

import os
import re
import subprocess
import tempfile

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "..", "hyquant_amd", "csrc", "decode.hip")


def _regs(text):
    out = set()
    for a, b in re.findall(r"\bs\[(\d+):(\d+)\]", text):
        out |= set(range(int(a), int(b) + 1))
    out |= {int(x) for x in re.findall(r"\bs(\d+)\b", text)}
    return out


def test_epilogue_argument_loads_are_not_read_before_their_wait():
    from hyquant_amd.build import HIPCC_FLAGS, hipcc
    if not os.path.exists(hipcc()):
        pytest.skip("hipcc not available")
    flags = [f for f in HIPCC_FLAGS if f not in ("-shared", "-fPIC")]
    with tempfile.TemporaryDirectory() as d:
        asm = os.path.join(d, "decode.s")
        proc = subprocess.run([hipcc(), *flags, "--cuda-device-only", "-S", "-o", asm, SRC],
                              capture_output=True, text=True)
        assert proc.returncode == 0, proc.stderr[-2000:]
        lines = open(asm).read().split("\n")
    kernel, checked, bad = None, 0, []
    for i, line in enumerate(lines):
        if re.match(r"^_Z\S*decode_kernel\S*:", line):
            kernel = line.split(":")[0]
        m = re.search(r"s_load_dwordx(?:8|4) (s\[\d+:\d+\]), s\[\d+:\d+\], 0x(?:c0|e0)\b", line)
        if not m or kernel is None:
            continue
        dst = _regs(m.group(1))
        checked += 1
        for j in range(i + 1, len(lines)):
            t = lines[j].split(";")[0].strip()
            if not t:
                continue
            if "s_waitcnt" in t and "lgkmcnt" in t:
                break
            if re.search(r"s_load\S* .*0x(?:c0|e0)\b", t):
                continue
            parts = t.split(None, 1)
            if len(parts) > 1 and _regs(parts[1]) & dst:
                bad.append((kernel, j + 1, t))
    assert checked >= 2, "no epilogue argument loads found: the test no longer matches the kernel"
    assert not bad, bad[:5]
