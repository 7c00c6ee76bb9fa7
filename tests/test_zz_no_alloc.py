"""GPU test of hyq_decode_hybrid_noalloc, the decode entry point that
allocates nothing (its workspace is the library's 16 MiB device array):
through the C ABI, two calls in a row, the second on a smaller input, each
bit-identical to hyq_decode_hybrid on the same parameters and within the
decode tolerance of the float64 oracle."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import state_to_device, to_dev_bf16

pytestmark = pytest.mark.gpu


def _both(st, q, G):
    """(noalloc output, workspace-entry output) for one decode state."""
    import hyquant_amd as hq
    from hyquant_amd import _lib
    from hyquant_amd.decode_d_stage import decode_params
    args = (q, st["k_packed"], st["v_packed"], st["k_scale"], st["v_scale"], st["k_topk"], st["v_topk"],
            st["k_staging"], st["v_staging"], st["k_window"], st["v_window"], 4, 4)
    p, keep, out = decode_params(*args, kv_repeat=G)
    L = _lib.lib()
    assert L.hyq_decode_workspace_size(p) <= 16 << 20
    rc = L.hyq_decode_hybrid_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "hyq_decode_hybrid_noalloc")
    ref = hq.fused_d_stage_decode(*args, kv_repeat=G)
    torch.cuda.synchronize()
    del keep
    return out, ref


def test_noalloc_decode_matches_workspace_entry_on_two_calls():
    dev = torch.device("cuda")
    runs = [dict(B=1, HQ=32, HKV=8, N=8192, S=64, seed=0),      # config 1
            dict(B=1, HQ=32, HKV=8, N=1024, S=37, seed=0)]      # config 0: a smaller second call
    for cfg in runs:
        print(f"noalloc decode {cfg}", flush=True)
        inp = O.make_decode_inputs(W=128, **cfg)
        st = O.build_decode_state(inp)
        q = to_dev_bf16(inp.q_dec, dev)
        out, ref = _both(state_to_device(st, dev), q, 4)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"{cfg}: outputs differ"
        err = float(np.max(np.abs(out.float().cpu().numpy() - O.decode_fp64_state(inp.q_dec, st, 4))))
        print(f"  bit-identical to hyq_decode_hybrid; max-abs vs fp64 oracle {err:.3e}", flush=True)
        assert err <= 2e-3


def test_noalloc_decode_wide_batch_then_small():
    """A many-head call (B=16, 8K prefix: 128 KV heads, the counters of the
    whole table in use) followed by a one-head call: the counters the first
    call used must be back at zero for the second."""
    import math
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(5)
    for B, N in ((16, 8192), (1, 300)):
        print(f"noalloc decode B={B} N={N}", flush=True)
        D, HKV = 128, 8
        T = max(1, math.ceil((N - 256) * 0.05))
        nq = N - 128 - T
        kv = lambda n: torch.randn(B * HKV, n, D, generator=g, device=dev).to(torch.bfloat16)
        import hyquant_amd as hq
        kp, ks = hq.quantize_per_token(kv(nq), 4)
        vp, vs = hq.quantize_per_token(kv(nq), 4)
        st = dict(k_packed=kp, v_packed=vp, k_scale=ks, v_scale=vs, k_topk=kv(T), v_topk=kv(T),
                  k_staging=kv(64), v_staging=kv(64), k_window=kv(128), v_window=kv(128))
        q = torch.randn(B * 32, D, generator=g, device=dev).to(torch.bfloat16)
        out, ref = _both(st, q, 4)
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


_CAPTURE_CHILD = r'''
import ctypes, math, sys
import torch
sys.path.insert(0, sys.argv[1])
import hyquant_amd as hq
from hyquant_amd import _lib
from hyquant_amd.decode_d_stage import decode_params

dev = torch.device("cuda")
g = torch.Generator(device=dev).manual_seed(7)
L = _lib.lib()


def state(B, N):
    D, HKV = 128, 8
    T = max(1, math.ceil((N - 256) * 0.05))
    nq = N - 128 - T
    kv = lambda n: torch.randn(B * HKV, n, D, generator=g, device=dev).to(torch.bfloat16)
    kp, ks = hq.quantize_per_token(kv(nq), 4)
    vp, vs = hq.quantize_per_token(kv(nq), 4)
    q = torch.randn(B * 32, D, generator=g, device=dev).to(torch.bfloat16)
    return (q, kp, vp, ks, vs, kv(T), kv(T), kv(64), kv(64), kv(128), kv(128), 4, 4)


calls = [state(1, 8192), state(1, 2048), state(2, 4096)]
params = [decode_params(*a, kv_repeat=4) for a in calls]
torch.cuda.synchronize()
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    # the process's first hyq_decode_hybrid_noalloc calls: the scratch lookup
    # and its clear happen inside the capture
    for p, keep, out in params:
        _lib.check(L.hyq_decode_hybrid_noalloc(ctypes.byref(p), torch.cuda.current_stream().cuda_stream),
                   "hyq_decode_hybrid_noalloc")
for replay in range(4):
    for _, _, out in params:
        out.fill_(0)
    graph.replay()
    # eager work between replays: the workspace entry point on the same inputs
    refs = [hq.fused_d_stage_decode(*a, kv_repeat=4) for a in calls]
    torch.cuda.synchronize()
    for i, ((_, _, out), ref) in enumerate(zip(params, refs)):
        if not torch.equal(out.view(torch.int16), ref.view(torch.int16)):
            print(f"replay {replay} call {i}: outputs differ", flush=True)
            sys.exit(1)
    print(f"replay {replay}: 3 captured calls bit-identical to hyq_decode_hybrid", flush=True)
print("OK", flush=True)
'''


def test_noalloc_first_call_inside_graph_capture():
    """The entry point is meant for code under HIP graph capture: in a fresh
    process (so that its first-ever call, with the scratch address lookup
    and the counter clear, is the captured one) three calls of different
    shapes are captured, and four replays, with eager calls of the
    workspace entry point between them, are each compared bit for bit with
    hyq_decode_hybrid on the same inputs."""
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc capture child: config-1, 2K and B=2 4K calls", flush=True)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True, text=True, timeout=240)
    print(r.stdout[-2000:], flush=True)
    assert r.returncode == 0, r.stderr[-3000:]
    assert "OK" in r.stdout
