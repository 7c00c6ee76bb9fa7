"""Benchmark of the fused hybrid decode attention on one MI355X.

Headline workload (benchmark config 1): one decode step of one attention
layer, B=1, 32 query / 8 KV heads, head_dim 128, prefix 8192 tokens frozen into
the four segments (int4 K4V4 prefix of 7667 tokens, 397 bf16 vertical lines,
64 bf16 staging tokens, 128 bf16 window tokens).  A "step" is one
fused_d_stage_decode call over that cache.

Timing: inputs are resident in HBM; R copies of the cache (R chosen so the
copies exceed 1 GiB, i.e. four times the 256 MiB Infinity Cache) are used in
rotation so every step streams its bytes from HBM.  W untimed steps, then
the steps are captured in ceil(R / K) HIP graphs of K steps, graph j over
copies jK .. jK + K - 1, replayed in turn so that a copy comes back only after
all R were streamed (whatever K is); each replay is bracketed by two HIP
events on the stream the kernels run on and by synchronisations, and the
median of five replays gives the per-step time (the same K steps issued as
Python calls one by one are reported as eager_us_per_step).

Output: one JSON line (rank 0), with the roofline of the decode kernel, the
CPU baseline (the reference's bf16 eager decode math run by torch on the host
CPU on config 1), the prefix sweep of config 2 beside a bf16 full-KV
split-K decode of the same shape, and the other configs' workloads measured
in the same run: config 3 (wide-GQA decode at B=32, 16K prefix; the vertical
line selector, the freeze reorganisation and the staging flush) and config 4
(hybrid prefill: int8 or fp8 QK, fp16 or fp8 P.V, and the window-only kernel;
TFLOP/s, MFMA utilisation and the output error against float32 exact
attention).  `accuracy` gives the config-1 decode error (max-abs, relative)
against float32 attention over the same quantised cache.

`--pmc` runs a fixed, short workload for hardware-counter passes instead (a
256 MiB device copy, the calibration of FETCH_SIZE / WRITE_SIZE, 20 eager
config-1 decode steps over distinct cache copies, three config-4 prefill
calls at N = 32768) and prints nothing; `--pmc-decode-shapes` runs four eager
decode steps at each of three shapes (B=16 32K, and the Qwen3-32B and
GLM-4-9B shapes of config 3) for SQ counter passes.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "hybrid decode-attn µs/step + HBM GB/s (% peak), 32q/8kv d128, 1K–32K prefix"
HBM_PEAK_GBS = 8000.0
D = 128


def top_k_count(prefix_len: int, rho: float) -> int:
    t = max(1, int(math.ceil(prefix_len * rho)))
    return min(t, prefix_len)


def seg_sizes(N: int, W: int = 128, S: int = 64, rho: float = 0.05):
    """Decode-time segment sizes after freeze (T from [0, N-2W))."""
    T = top_k_count(max(0, N - 2 * W), rho) if N - 2 * W > 0 else 0
    Nq = N - W - T
    return Nq, T, S, W


def algorithmic_bytes(B, HQ, HKV, N, W=128, S=64, rho=0.05, kb=4, vb=4):
    Nq, T, S, W = seg_sizes(N, W, S, rho)
    return B * HKV * (Nq * (16 * kb + 16 * vb + 2 + 2) + (T + S + W) * 2 * D * 2) + B * HQ * D * 2 * 2


def bf16_bytes(B, HQ, HKV, N, S=64):
    return B * HKV * (N + S) * 2 * D * 2 + B * HQ * D * 2 * 2


def make_state(B, HQ, HKV, N, dev, seed, W=128, S=64, rho=0.05, kb=4, vb=4):
    """Synthetic decode cache on the GPU: Gaussian K (per-channel N(0,2)
    offsets) and V, quantised by the library's own quantiser."""
    import hyquant_amd as hq
    Nq, T, S, W = seg_sizes(N, W, S, rho)
    BH = B * HKV
    g = torch.Generator(device=dev).manual_seed(seed)
    off = torch.randn(HKV, D, generator=g, device=dev) * math.sqrt(2.0)
    off_bh = off.repeat(B, 1)[:, None, :]
    bf = torch.bfloat16

    def kv(n, is_k):
        x = torch.randn(BH, n, D, generator=g, device=dev)
        if is_k:
            x += off_bh
        return x.to(bf)

    kp, ks = hq.quantize_per_token(kv(Nq, True), kb)
    vp, vs = hq.quantize_per_token(kv(Nq, False), vb)
    st = dict(k_packed=kp, v_packed=vp, k_scale=ks, v_scale=vs, bits=(kb, vb),
              k_topk=kv(T, True), v_topk=kv(T, False),
              k_staging=kv(S, True), v_staging=kv(S, False),
              k_window=kv(W, True), v_window=kv(W, False))
    q = torch.randn(B * HQ, D, generator=g, device=dev).to(bf)
    return q, st


def run_decode(q, st, G):
    import hyquant_amd as hq
    return hq.fused_d_stage_decode(q, st["k_packed"], st["v_packed"], st["k_scale"], st["v_scale"],
                                   st["k_topk"], st["v_topk"], st["k_staging"], st["v_staging"],
                                   st["k_window"], st["v_window"], st["bits"][0], st["bits"][1], kv_repeat=G)


REPLAYS = 5


def time_rotating(fn, states, warmup, steps, replays=REPLAYS):
    """ms per step over `steps` steps cycling through `states`.

    The steps are captured into ceil(R / K) HIP graphs of K steps each, graph
    j covering copies jK .. jK + K - 1 (mod R), and the graphs are replayed in
    turn, so a copy is streamed again only after every other copy was: R
    copies of >= 1 GiB together (four times the 256 MiB Infinity Cache) put
    at least that much traffic between two uses of a copy whatever K is.
    Each replay (K steps, no host work between launches) is bracketed by HIP
    events on the stream, and the median replay gives the per-step time.
    Returns (graph_ms_per_step, eager_ms_per_step) where the eager figure
    times max(K, 200) Python calls issued one by one (steady state: a short
    burst after an idle GPU also times the clocks ramping up)."""
    n = len(states)
    for i in range(max(warmup, 20)):
        fn(states[i % n])
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    ne = max(steps, 200)
    e0.record()
    for i in range(ne):
        fn(states[i % n])
    e1.record()
    torch.cuda.synchronize()
    eager = e0.elapsed_time(e1) / ne
    graphs = []
    for j in range(max(1, -(-n // steps))):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            for i in range(steps):
                fn(states[(j * steps + i) % n])
        graphs.append(g)
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    per = []
    for r in range(replays):
        e0.record()
        graphs[r % len(graphs)].replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / steps)
    per.sort()
    del graphs
    return per[len(per) // 2], eager


def copies_for(nbytes, cap=2048):
    return int(max(1, min(cap, math.ceil((1 << 30) / max(nbytes, 1)))))


def bench_hybrid(B, HQ, HKV, N, dev, warmup, steps, seed=0, kb=4, vb=4):
    nbytes = algorithmic_bytes(B, HQ, HKV, N, kb=kb, vb=vb)
    R = copies_for(nbytes)
    assert R * nbytes >= (1 << 30), "the rotated copies must cover 1 GiB"
    states = [make_state(B, HQ, HKV, N, dev, seed + r, kb=kb, vb=vb) for r in range(R)]
    G = HQ // HKV
    ms, eager = time_rotating(lambda s: run_decode(s[0], s[1], G), states, warmup, steps)
    del states
    return ms, nbytes, R, eager


def bench_bf16(B, HQ, HKV, N, dev, warmup, steps, seed=0):
    import hyquant_amd as hq
    nbytes = bf16_bytes(B, HQ, HKV, N)
    R = copies_for(nbytes, cap=64)
    g = torch.Generator(device=dev).manual_seed(seed)
    mk = lambda: torch.randn(B * HKV, N + 64, D, generator=g, device=dev).to(torch.bfloat16)
    states = [(torch.randn(B * HQ, D, generator=g, device=dev).to(torch.bfloat16), mk(), mk()) for _ in range(R)]
    G = HQ // HKV
    ms, eager = time_rotating(lambda s: hq.decode_bf16_full(s[0], s[1], s[2], kv_repeat=G), states, warmup, steps)
    del states
    return ms, nbytes, R, eager


def cpu_threads():
    """Threads for the CPU baseline: os.cpu_count(), capped by the CPUs this
    process may run on and by OMP_NUM_THREADS when the environment sets it
    (the GPU box gives one GPU's job a 16-CPU share and sets
    OMP_NUM_THREADS=16; more threads than that share oversubscribe it)."""
    n = os.cpu_count() or 1
    try:
        n = min(n, len(os.sched_getaffinity(0)))
    except (AttributeError, OSError):
        pass
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(N=8192, S=64, min_steps=20, budget_s=20.0):
    """The reference's eager decode math (bf16 dequant + SDPA on torch CPU,
    src/ops/d_stage_kv_cache.py:309-354) on config 1 (or config 0 with N=1024,
    S=37), timed on the host CPU."""
    from oracle import hyq_oracle as O
    cores = cpu_threads()
    torch.set_num_threads(cores)
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=N, W=128, S=S, seed=0)
    st = O.build_decode_state(inp)
    es = O.prepare_eager_state(st)
    q = torch.from_numpy(inp.q_dec)
    O.decode_bf16_eager_torch(q, es, 4, 1)
    times = []
    t_start = time.perf_counter()
    while len(times) < min_steps or (time.perf_counter() - t_start < 2.0 and len(times) < 200):
        t0 = time.perf_counter()
        O.decode_bf16_eager_torch(q, es, 4, 1)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    name = "config 1" if N == 8192 else "config 0" if N == 1024 else f"prefix {N}"
    return {"value": round(med * 1e6, 1), "unit": "us/step", "cores": cores, "kind": "port",
            "sample": f"{name} (B=1, 32q/8kv, prefix {N}, {S} staging tokens), median of {len(times)} steps "
                      f"of the bf16 eager dequant+SDPA decode on torch CPU, {cores} threads "
                      f"(os.cpu_count() {os.cpu_count()}, capped by the process's CPU set and "
                      f"OMP_NUM_THREADS); host CPU: {model}"}


# MI355X dense peaks (TFLOP/s or TOP/s)
PEAK_INT8 = 5000.0
PEAK_FP16 = 2500.0
PEAK_FP8 = 5000.0


def time_calls(fn, warmup=2, iters=5):
    """ms per call of fn, eager, HIP events on the current stream."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(iters):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / iters


def time_graph(fn, iters=50, replays=REPLAYS):
    """ms per call of fn: iters calls captured in one HIP graph, the median of
    `replays` replays bracketed by HIP events (no host launch cost inside the
    timed region, for calls shorter than a launch)."""
    for _ in range(3):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(iters):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    per = []
    for _ in range(replays):
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        per.append(e0.elapsed_time(e1) / iters)
    per.sort()
    del g
    return per[len(per) // 2]


def exact_attention_fp32(q, k, v, chunk=1024):
    """Causal softmax(q k^T / sqrt(D)) v in float32 on the GPU, chunked over
    queries, GQA by head index (the reference for the prefill error figures;
    2-D float32 products only)."""
    B, HQ, N, Dh = q.shape
    G = HQ // k.shape[1]
    out = torch.empty(B, HQ, N, Dh, dtype=torch.float32, device=q.device)
    for b in range(B):
        for h in range(HQ):
            kk = k[b, h // G].float()
            vv = v[b, h // G].float()
            for s0 in range(0, N, chunk):
                qq = q[b, h, s0:s0 + chunk].float()
                sc = (qq @ kk[: s0 + chunk].T.contiguous()) * Dh ** -0.5
                i = torch.arange(s0, s0 + qq.shape[0], device=q.device)[:, None]
                j = torch.arange(sc.shape[1], device=q.device)[None, :]
                sc = sc.masked_fill(j > i, float("-inf"))
                out[b, h, s0:s0 + chunk] = torch.softmax(sc, dim=-1) @ vv[: s0 + chunk]
    return out


def error_vs(out, ref):
    """max-abs, relative (max-abs / max |ref|), relative L2 and MSE of out
    against a float32 reference."""
    d = out.float() - ref
    return {"max_abs": float(d.abs().max()), "rel_max": float(d.abs().max() / ref.abs().max()),
            "rel_l2": float(d.norm() / ref.norm()), "mse": float((d * d).mean())}


def decode_error(dev):
    """Config-1 decode output against float32 attention over the same
    quantised cache on the GPU: the int4 codes times their fp16 scales (exact
    in float32), the top-k / staging / window rows, softmax(q k^T / sqrt(D)) v
    per query head with query head h on KV head h // 4."""
    from hyquant_amd.decode_d_stage import _unpack_int4
    q, st = make_state(1, 32, 8, 8192, dev, 99)
    out = run_decode(q, st, 4).float()
    kq = _unpack_int4(st["k_packed"], D) * st["k_scale"].float()[..., None]
    vq = _unpack_int4(st["v_packed"], D) * st["v_scale"].float()[..., None]
    K = torch.cat([kq, st["k_topk"].float(), st["k_staging"].float(), st["k_window"].float()], 1)
    V = torch.cat([vq, st["v_topk"].float(), st["v_staging"].float(), st["v_window"].float()], 1)
    ref = torch.empty(32, D, dtype=torch.float32, device=dev)
    for h in range(32):
        p = torch.softmax((K[h // 4] @ q[h].float()) * D ** -0.5, dim=0)
        ref[h] = p @ V[h // 4]
    e = error_vs(out, ref)
    e["reference"] = "float32 attention over the dequantised four-segment cache (GPU, torch)"
    e["bound"] = "max_abs <= 2e-3"
    return e


PREFILL_NS = (8192, 16384, 32768)
# (name, kernel kind, QK operand, P.V operand, QK peak, P.V peak)
PREFILL_VARIANTS = (
    ("hybrid int8/fp16", "hybrid", "int8", "fp16", PEAK_INT8, PEAK_FP16),
    ("hybrid int8/fp8", "hybrid", "int8", "fp8", PEAK_INT8, PEAK_FP8),
    ("hybrid fp8/fp16", "hybrid", "fp8", "fp16", PEAK_FP8, PEAK_FP16),
    ("window_only int8/fp16", "window_only", "int8", "fp16", PEAK_INT8, PEAK_FP16),
)
PREFILL_CALLS = 14          # per variant and N: 3 warm-up, 10 timed, 1 for the error figures


def bench_prefill(dev):
    """Config 4: hybrid prefill, B=1, 32q/8kv, d128, causal, W=128, rho=5%,
    with int8 or e4m3 QK on the rest tiles and fp16 or e4m3 P.V, and the
    window-only kernel (sage_w).  Each timing is the whole operator (K
    statistics, conversion, lists, gather and the attention kernel).  FLOPs
    counted as 2*B*H_Q*N^2*D (QK and PV over the causal half).  MFMA
    utilisation = achieved / the peak of the dtype mix, each of QK and PV half
    of the FLOPs."""
    from hyquant_amd.sage_unified import (sage_unified_attention, sage_vertical_attention_v2,
                                          sage_vertical_attention_v2_fp8)
    from hyquant_amd.vertical import compute_vertical_indices
    g = torch.Generator(device=dev).manual_seed(4)
    rows = []
    for N in PREFILL_NS:
        B, HQ, HKV, W = 1, 32, 8, 128
        q = torch.randn(B, HQ, N, D, generator=g, device=dev).to(torch.bfloat16)
        k = (torch.randn(B, HKV, N, D, generator=g, device=dev) +
             math.sqrt(2.0) * torch.randn(B, HKV, 1, D, generator=g, device=dev)).to(torch.bfloat16)
        v = torch.randn(B, HKV, N, D, generator=g, device=dev).to(torch.bfloat16)
        vidx = compute_vertical_indices(q, k, W, 0.05, kv_repeat=HQ // HKV)
        exact = exact_attention_fp32(q, k, v)
        flops = 2.0 * B * HQ * N * N * D
        fns = {
            "hybrid int8/fp16": lambda: sage_vertical_attention_v2(q, k, v, vidx, window_size=W),
            "hybrid int8/fp8": lambda: sage_vertical_attention_v2(q, k, v, vidx, window_size=W, pv_mode="fp8"),
            "hybrid fp8/fp16": lambda: sage_vertical_attention_v2_fp8(q, k, v, vidx, window_size=W),
            "window_only int8/fp16": lambda: sage_unified_attention(q, k, v, window_size=W),
        }
        for name, kind, qk, pv, qk_peak, pv_peak in PREFILL_VARIANTS:
            fn = fns[name]
            ms = time_calls(fn, warmup=PREFILL_CALLS - 11, iters=10)
            tf = flops / (ms * 1e-3) / 1e12
            peak = 2.0 / (1.0 / qk_peak + 1.0 / pv_peak)
            err = error_vs(fn(), exact)
            rows.append({"seq_len": N, "kernel": kind, "qk": qk, "pv": pv, "ms": round(ms, 3),
                         "tflops": round(tf, 1), "mfma_peak_tflops": round(peak, 1),
                         "mfma_util": round(tf / peak, 4), "n_vertical": int(vidx.shape[-1]) if kind == "hybrid" else 0,
                         "mse_vs_exact_fp32": float("%.3e" % err["mse"]),
                         "max_abs_vs_exact_fp32": float("%.3e" % err["max_abs"]),
                         "rel_l2_vs_exact_fp32": float("%.3e" % err["rel_l2"])})
            print(f"# prefill {rows[-1]}", file=sys.stderr, flush=True)
        del q, k, v, vidx, exact
        torch.cuda.empty_cache()
    return rows


def bench_boundary(dev):
    """Config 3 boundary ops at B=32, prefix 16384 (Llama shape 32q/8kv):
    the prefill-time vertical-line selector (W=256, rho=5%), the freeze
    (freeze-time selector + reorganisation into the four segments) and a staging
    flush (128 bf16 tokens of every KV head quantised to int4; timed as 50
    calls in a HIP graph, since one call is shorter than a host launch)."""
    from hyquant_amd.decode_d_stage import quantize_into
    from hyquant_amd.d_stage_kv_cache import DStageLayerCache
    from hyquant_amd.vertical import compute_vertical_indices
    g = torch.Generator(device=dev).manual_seed(3)
    B, HQ, HKV, N, W = 32, 32, 8, 16384, 256
    q = torch.randn(B, HQ, N, D, generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn(B, HKV, N, D, generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn(B, HKV, N, D, generator=g, device=dev).to(torch.bfloat16)
    out = {}
    ms = time_calls(lambda: compute_vertical_indices(q, k, W, 0.05, kv_repeat=HQ // HKV))
    by = B * HKV * (N - W) * D * 2 + B * HQ * W * D * 2
    out["select"] = {"us": round(ms * 1e3, 1), "gbs": round(by / (ms * 1e-3) / 1e9, 1),
                     "algorithmic_bytes": by, "n_selected": int(math.ceil((N - W) * 0.05))}

    def freeze_once():
        c = DStageLayerCache(0, 4, 4, window_size=W)
        c.update_prefill(k, v)
        c.save_query_tail(q[:, :, -W:, :])
        c.freeze(kv_repeat=HQ // HKV)
        return c
    ms = time_calls(freeze_once, warmup=1, iters=3)
    T = int(math.ceil((N - 2 * W) * 0.05))
    nq = N - W - T
    fb = (B * HKV * (N - 2 * W) * D * 2 + B * HQ * W * D * 2            # freeze-time selector reads
          + B * HKV * (N - W) * D * 2 * 2                               # K and V read by the reorganisation
          + B * HKV * (nq * 132 + (T + W) * D * 2 * 2))                 # segments written
    out["freeze"] = {"us": round(ms * 1e3, 1), "gbs": round(fb / (ms * 1e-3) / 1e9, 1), "algorithmic_bytes": fb}
    x = torch.randn(B * HKV, 128, D, generator=g, device=dev).to(torch.bfloat16)
    packed = torch.empty(B * HKV, 128, D // 2, dtype=torch.int8, device=dev)
    scale = torch.empty(B * HKV, 128, dtype=torch.float16, device=dev)
    ms = time_graph(lambda: quantize_into(x, 4, packed, scale), iters=50)
    by = B * HKV * 128 * (D * 2 + D // 2 + 2)
    out["flush"] = {"us": round(ms * 1e3, 2), "gbs": round(by / (ms * 1e-3) / 1e9, 1), "algorithmic_bytes": by}
    print(f"# boundary {out}", file=sys.stderr, flush=True)
    return out


def bench_wide_gqa(dev):
    """Config 3 decode shapes at B=32, prefix 16384: Qwen3-32B (64q/8kv) and
    GLM-4-9B (32q/2kv, GQA 16)."""
    rows = []
    for name, HQ, HKV in (("Qwen3-32B", 64, 8), ("GLM-4-9B", 32, 2)):
        ms, nb, _, _ = bench_hybrid(32, HQ, HKV, 16384, dev, 5, 50)
        rows.append({"model": name, "batch": 32, "q_heads": HQ, "kv_heads": HKV, "prefix": 16384,
                     "us_per_step": round(ms * 1e3, 2), "gbs": round(nb / (ms * 1e-3) / 1e9, 1),
                     "frac_peak": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
        print(f"# wide-gqa {rows[-1]}", file=sys.stderr, flush=True)
    return rows


def bench_modes(dev):
    """The other cache modes of the reference's mode table (src/patch/_common.py:38-49):
    K4V2, K2V4 and K8V8 prefixes, at config 1 and at B=16 with a 32K prefix."""
    rows = []
    for kb, vb in ((4, 2), (2, 4), (8, 8)):
        for B, N in ((1, 8192), (16, 32768)):
            ms, nb, _, _ = bench_hybrid(B, 32, 8, N, dev, 10, 100, kb=kb, vb=vb)
            rows.append({"mode": f"K{kb}V{vb}", "batch": B, "prefix": N, "us_per_step": round(ms * 1e3, 3),
                         "gbs": round(nb / (ms * 1e-3) / 1e9, 1),
                         "frac_peak": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
            print(f"# mode {rows[-1]}", file=sys.stderr, flush=True)
    return rows


def pmc_workload(dev):
    """Fixed workload for rocprofv3 --pmc passes: a 256 MiB device copy (the
    FETCH_SIZE / WRITE_SIZE calibration: it reads and writes 256 MiB), then 20
    eager config-1 decode steps, each over its own cache copy, then three
    config-4 hybrid prefill calls at N = 32768 (int8 QK, fp16 P.V), two with
    fp8 P.V and two with fp8 QK."""
    src_t = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst_t = torch.empty_like(src_t)
    for _ in range(3):
        dst_t.copy_(src_t)
    torch.cuda.synchronize()
    del src_t, dst_t
    states = [make_state(1, 32, 8, 8192, dev, s) for s in range(20)]
    torch.cuda.synchronize()
    for q, st in states:
        run_decode(q, st, 4)
    torch.cuda.synchronize()
    del states
    from hyquant_amd.sage_unified import sage_vertical_attention_v2, sage_vertical_attention_v2_fp8
    from hyquant_amd.vertical import compute_vertical_indices
    g = torch.Generator(device=dev).manual_seed(4)
    N, HQ, HKV, W = 32768, 32, 8, 128
    q = torch.randn(1, HQ, N, D, generator=g, device=dev).to(torch.bfloat16)
    k = (torch.randn(1, HKV, N, D, generator=g, device=dev) +
         math.sqrt(2.0) * torch.randn(1, HKV, 1, D, generator=g, device=dev)).to(torch.bfloat16)
    v = torch.randn(1, HKV, N, D, generator=g, device=dev).to(torch.bfloat16)
    vidx = compute_vertical_indices(q, k, W, 0.05, kv_repeat=HQ // HKV)
    for _ in range(3):
        sage_vertical_attention_v2(q, k, v, vidx, window_size=W)
    for _ in range(2):
        sage_vertical_attention_v2(q, k, v, vidx, window_size=W, pv_mode="fp8")
    for _ in range(2):
        sage_vertical_attention_v2_fp8(q, k, v, vidx, window_size=W)
    torch.cuda.synchronize()


# decode counter shapes: the 12 config-2 sweep points (Llama-3.1-8B,
# 32q/8kv), then the config-3 Qwen3-32B and GLM-4-9B shapes
PMC_SHAPES = tuple((b, 32, 8, n) for b in (1, 16) for n in (1024, 2048, 4096, 8192, 16384, 32768)) + \
    ((32, 64, 8, 16384), (32, 32, 2, 16384))


def pmc_copies(B, HQ, HKV, N):
    """Cache copies (one eager decode step each) per counter shape: enough
    to span more than the 256 MiB last-level cache, at most 64."""
    return int(max(4, min(64, math.ceil((384 << 20) / algorithmic_bytes(B, HQ, HKV, N)))))


def pmc_decode_shapes_workload(dev):
    """Fixed workload for counter passes over the decode kernel: a 256 MiB
    device copy (the FETCH_SIZE / WRITE_SIZE calibration) three times, then
    for each shape of PMC_SHAPES one eager step over each of pmc_copies()
    cache copies, in that order (a summary maps the decode_kernel dispatches
    back to the shapes by their order)."""
    src_t = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst_t = torch.empty_like(src_t)
    for _ in range(3):
        dst_t.copy_(src_t)
    torch.cuda.synchronize()
    del src_t, dst_t
    for (B, HQ, HKV, N) in PMC_SHAPES:
        R = pmc_copies(B, HQ, HKV, N)
        states = [make_state(B, HQ, HKV, N, dev, s) for s in range(R)]
        torch.cuda.synchronize()
        for q, st in states:
            run_decode(q, st, HQ // HKV)
        torch.cuda.synchronize()
        print(f"# pmc shape B={B} {HQ}q/{HKV}kv N={N}: {R} decode steps", file=sys.stderr, flush=True)
        del states
        torch.cuda.empty_cache()


def _counter_rows(path, counter):
    """(kernel name, dispatch id, value) of one counter from a rocprofv3
    counter_collection.csv, in dispatch order (values summed over the
    counter's instances)."""
    import csv
    vals = {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        key = int(r["Dispatch_Id"])
        name, v = vals.get(key, (r["Kernel_Name"], 0.0))
        vals[key] = (name, v + float(r["Counter_Value"]))
    return [(vals[k][0], k, vals[k][1]) for k in sorted(vals)]


def pmc_decode_summary(fetch_csv, write_csv, sq_csv=None):
    """Per-shape HBM bytes per decode launch from the FETCH_SIZE and
    WRITE_SIZE passes over --pmc-decode-shapes: the copy kernel's counters
    give the calibration (it reads and writes 256 MiB), the decode_kernel
    dispatches are mapped to PMC_SHAPES by order, and each shape reports the
    median over its launches.  An optional third pass (SQ / GRBM counters)
    adds each counter's per-shape median and the derived busy and wait
    fractions (GRBM_GUI_ACTIVE summed over 8 XCDs, 1024 SIMDs, VALU issue
    counted as 4 cycles per wave64 instruction)."""
    import numpy as np
    out = {"workload": "bench.py --pmc-decode-shapes", "shapes": []}
    cal = {}
    per = {}
    for counter, path in (("FETCH_SIZE", fetch_csv), ("WRITE_SIZE", write_csv)):
        rows = _counter_rows(path, counter)
        copy = [v for (n, _, v) in rows if "copyBuffer" in n][:3]
        dec = [v for (n, _, v) in rows if "decode_kernel" in n]
        if not copy or not dec:
            raise RuntimeError(f"{path}: no copy or decode_kernel dispatches for {counter}")
        raw = float(np.median(copy))
        scale = (256 << 10) / raw
        cal[counter] = {"copy_kib_raw": round(raw, 2), "scale": round(scale, 4)}
        per[counter] = (dec, scale)
    i = {"FETCH_SIZE": 0, "WRITE_SIZE": 0}
    for (B, HQ, HKV, N) in PMC_SHAPES:
        R = pmc_copies(B, HQ, HKV, N)
        row = {"batch": B, "q_heads": HQ, "kv_heads": HKV, "prefix": N, "launches": R,
               "algorithmic_bytes_per_launch": algorithmic_bytes(B, HQ, HKV, N)}
        for counter, key in (("FETCH_SIZE", "fetch_bytes_per_launch"), ("WRITE_SIZE", "write_bytes_per_launch")):
            dec, scale = per[counter]
            vals = dec[i[counter]: i[counter] + R]
            if len(vals) != R:
                raise RuntimeError(f"{counter}: {len(dec)} decode dispatches, fewer than the workload's")
            i[counter] += R
            row[key] = int(round(float(np.median(vals)) * 1024 * scale))
        row["traffic_bytes_per_launch"] = row["fetch_bytes_per_launch"] + row["write_bytes_per_launch"]
        row["traffic_over_algorithmic"] = round(row["traffic_bytes_per_launch"] / row["algorithmic_bytes_per_launch"], 4)
        out["shapes"].append(row)
    if sq_csv:
        import csv
        per_disp = {}
        for r in csv.DictReader(open(sq_csv)):
            if "decode_kernel" not in r["Kernel_Name"]:
                continue
            d = per_disp.setdefault(int(r["Dispatch_Id"]), {})
            d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
        disp = [per_disp[k] for k in sorted(per_disp)]
        j = 0
        for row in out["shapes"]:
            cs = disp[j: j + row["launches"]]
            j += row["launches"]
            if len(cs) != row["launches"]:
                raise RuntimeError(f"{sq_csv}: fewer decode dispatches than the workload's")
            med = {c: float(np.median([d.get(c, 0.0) for d in cs])) for c in sorted({c for d in cs for c in d})}
            row["sq"] = {c: float("%.4g" % v) for c, v in med.items()}
            cyc = med.get("GRBM_GUI_ACTIVE", 0.0) / 8
            der = {}
            if cyc > 0 and "SQ_ACTIVE_INST_VALU" in med:
                der["valu_busy"] = round(4 * med["SQ_ACTIVE_INST_VALU"] / 1024 / cyc, 3)
            if cyc > 0 and "SQ_VALU_MFMA_BUSY_CYCLES" in med:
                der["mfma_busy"] = round(med["SQ_VALU_MFMA_BUSY_CYCLES"] / 1024 / cyc, 3)
            if med.get("SQ_WAVE_CYCLES"):
                for c, key in (("SQ_WAIT_ANY", "wave_time_waiting_on_counters"),
                               ("SQ_WAIT_INST_ANY", "wave_time_waiting_to_issue")):
                    if c in med:
                        der[key] = round(med[c] / med["SQ_WAVE_CYCLES"], 3)
            if med.get("SQ_INSTS_VMEM_RD"):
                der["fetch_bytes_per_vmem_read"] = round(row["fetch_bytes_per_launch"] / med["SQ_INSTS_VMEM_RD"], 1)
            if med.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in med:
                der["valu_per_mfma"] = round((med["SQ_INSTS_VALU"] - med["SQ_INSTS_MFMA"]) / med["SQ_INSTS_MFMA"], 2)
            row["derived"] = der
    out["calibration"] = cal
    return out


def sweep_traffic_record():
    """{(batch, prefix): traffic bytes per launch} of the 32q/8kv decode
    shapes from profiles/decode_sweep_traffic.json, or {}."""
    path = os.path.join(ROOT, "profiles", "decode_sweep_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return {}
    return {(r["batch"], r["prefix"]): r["traffic_bytes_per_launch"] for r in rec.get("shapes", [])
            if r.get("q_heads") == 32 and r.get("kv_heads") == 8}


def prefill_trace_summary(trace_csv):
    """Per-kernel durations of `bench.py --prefill-only` from a rocprofv3
    kernel trace (run_kernel_trace.csv): the calls are told apart by their
    prefill_main_kernel dispatch (one per call; the auxiliary kernels of a
    call precede it) and mapped to (N, variant) by order: for each N of
    bench_prefill, for each variant, 3 warm-up + 10 timed calls + 1 error
    call.  Reports the median over the 14 calls, in microseconds."""
    import csv
    import numpy as np
    rows = list(csv.DictReader(open(trace_csv)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    calls, cur = [], {}
    short = lambda n: n.replace("void ", "").replace("hyq::(anonymous namespace)::", "").split("(")[0]
    ours = ("prefill_main_kernel", "kv_stats_kernel", "kv_final_kernel", "kv_convert_kernel", "gather_kernel",
            "per_block_int8_kernel", "zero_counts_kernel", "lists_kernel")
    for r in rows:
        n = short(r["Kernel_Name"])
        if not any(o in n for o in ours):
            continue
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        cur[n] = cur.get(n, 0.0) + d
        if "prefill_main_kernel" in n:
            calls.append(cur)
            cur = {}
    variants = [v[0] for v in PREFILL_VARIANTS]
    per = len(variants) * PREFILL_CALLS
    if len(calls) != len(PREFILL_NS) * per:
        raise RuntimeError(f"{len(calls)} prefill calls in the trace, expected {len(PREFILL_NS) * per}")
    table = []
    for ni, N in enumerate(PREFILL_NS):
        for vi, v in enumerate(variants):
            cs = calls[ni * per + vi * PREFILL_CALLS: ni * per + (vi + 1) * PREFILL_CALLS]
            names = sorted({k for c in cs for k in c})
            med = {k: round(float(np.median([c.get(k, 0.0) for c in cs])), 1) for k in names}
            table.append({"seq_len": N, "variant": v, "kernels_us": med,
                          "total_us": round(float(np.median([sum(c.values()) for c in cs])), 1)})
    return table


def bench_legacy(dev):
    """The legacy decode format (src/ops/d_stage_cache.py): the direct path
    (hyq_decode_legacy: codes and [G, D] group scales read in the decode)
    against the dequantise-first route (legacy_dequantize into bf16 rows, then
    the fused decode's bf16 path), eager calls, kv_repeat 4, bf16 top-k N/20,
    staging 64, window 128.  The calls rotate over copies of the inputs that
    cover at least 1 GiB together, so that every call streams its bytes from
    HBM (not from the 256 MiB Infinity Cache).  Time: best of three runs of
    50 calls after 5 warm-up calls, events around each run.  Bytes:
    16*(k_bits + v_bits) + 4 per prefix token and key head (codes and group
    scales) plus 512 per bf16 row."""
    import hyquant_amd.d_stage_cache as L
    from hyquant_amd.decode_d_stage import GROUP_SIZE, _decode
    def timed(fn, n):
        for _ in range(5):
            fn()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(3):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(n):
                fn()
            e1.record()
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) / n * 1e3)
        return best
    rows = []
    shapes = [(4, 4, 8, 7667), (4, 4, 32, 31000), (4, 4, 128, 31000), (4, 4, 128, 62000),
              (4, 2, 128, 31000), (2, 4, 128, 31000), (2, 2, 128, 31000)]
    for kb, vb, BHK, N in shapes:
        R, T, S, W, D = 4, N // 20, 64, 128, 128
        G = -(-N // GROUP_SIZE)
        nb = BHK * N * (16 * (kb + vb) + 4) + BHK * (T + S + W) * 512
        torch.manual_seed(0)

        def inputs():
            return (torch.randint(0, 256, (BHK, N, 16 * kb), dtype=torch.uint8, device=dev),
                    torch.randint(0, 256, (BHK, N, 16 * vb), dtype=torch.uint8, device=dev),
                    (torch.rand(BHK, G, D, device=dev) * 0.24 - 0.12).half(),
                    (torch.rand(BHK, G, D, device=dev) * 0.24 - 0.12).half(),
                    [torch.randn(BHK, n, D, device=dev).bfloat16() for n in (T, T, S, S, W, W)],
                    torch.randn(1, BHK * R, 1, D, device=dev).bfloat16())
        copies = [inputs() for _ in range(copies_for(nb))]
        it = [0]

        def nxt():
            c = copies[it[0] % len(copies)]
            it[0] += 1
            return c

        def direct(c=None):
            kp, vp, ks, vs, seg, q = c or nxt()
            return L.splitk_decode_attention_k4v4_mma(q, kp, vp, ks, vs, *seg, kv_repeat=R, k_bits=kb, v_bits=vb)
        kf = torch.empty(BHK, N + T, D, dtype=torch.bfloat16, device=dev)
        vf = torch.empty_like(kf)
        n8 = torch.empty(BHK, 0, D // 2, dtype=torch.int8, device=dev)
        n16 = torch.empty(BHK, 0, dtype=torch.float16, device=dev)

        def first(c=None):
            kp, vp, ks, vs, seg, q = c or nxt()
            L.legacy_dequantize(kp, ks, D, kb, out=kf[:, :N])
            L.legacy_dequantize(vp, vs, D, vb, out=vf[:, :N])
            kf[:, N:].copy_(seg[0])
            vf[:, N:].copy_(seg[1])
            return _decode(q.reshape(BHK * R, D), n8, n8, n16, n16, kf, vf, seg[2], seg[3], seg[4], seg[5],
                           4, 4, R, None, 0, None, None)
        diff = (direct(copies[0]).float().reshape(BHK * R, D) - first(copies[0]).float()).abs().max().item()
        td, tf = timed(direct, 50), timed(first, 20)
        rows.append({"k_bits": kb, "v_bits": vb, "kv_heads": BHK, "prefix": N, "direct_us": round(td, 1),
                     "direct_gbs": round(nb / (td * 1e-6) / 1e9, 1), "dequantise_first_us": round(tf, 1),
                     "max_abs_diff": float(f"{diff:.3g}"), "input_copies": len(copies)})
        print(f"# legacy {rows[-1]}", file=sys.stderr, flush=True)
        del copies, kf, vf
        torch.cuda.empty_cache()
    return rows


def kernel_trace_summary(trace_csv):
    """Median duration per kernel (name without its argument list) and grid
    size (work-items in x, then "x" and the y extent when it is above 1) over
    every dispatch of a rocprofv3 kernel trace (run_kernel_trace.csv), this
    library's kernels only, in microseconds."""
    import csv
    import numpy as np
    d = {}
    for r in csv.DictReader(open(trace_csv)):
        n = r["Kernel_Name"].replace("void ", "").replace("hyq::(anonymous namespace)::", "")
        if not n.startswith(("score", "topk", "qmean", "mark", "zero_words", "compact_quant", "gather_rows",
                             "quant_pack", "decode_kernel", "dequant", "prefill", "kv_", "lists", "per_block",
                             "legacy")):
            continue
        grid = r.get("Grid_Size_X", r.get("Grid_Size", ""))
        if r.get("Grid_Size_Y", "1") not in ("", "1"):
            grid += "x" + r["Grid_Size_Y"]
        d.setdefault((n.split("(")[0], grid), []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    return [{"kernel": k, "grid": g, "dispatches": len(v), "median_us": round(float(np.median(v)), 1)}
            for (k, g), v in sorted(d.items())]


PHASES = ("entry", "arguments", "Q", "first K/V", "stream done", "LDS merge", "partial acked",
          "counter", "merge (m,l) in", "merge summed", "merge stored", "merge entered",
          "merge loads issued")


def phase_trace(dev, steps=100, shape=(1, 32, 8, 8192)):
    """Per-phase timeline of a decode step (config 1 unless `shape` = (B, HQ,
    HKV, N) says otherwise) under HIP-graph replay,
    from the phase-trace build (libhyq_trace.so: s_memrealtime stamps of every
    wavefront, 100 MHz).  Two workloads: the bench's rotation over >= 1 GiB
    of cache copies, and one cache copy replayed (translations and caches
    warm).  For each of the last launches of a replay: the launch start t0 is
    the earliest wavefront entry; every phase is reported as the median and
    the maximum over wavefronts of (stamp - t0) in microseconds (the merge
    phases over the merging wavefronts only); `end` is the last merge store
    acknowledged, `gap` the time from a launch's end to the next launch's t0,
    `wave_spread` the median over workgroups of the spread of their four
    wavefronts' stream-done stamps; `entry_pct` and `stream_done_pct` the
    10/50/90/100th percentiles over wavefronts of their entry and stream-done
    stamps, `stream_us_pct` those of each wavefront's own stream (first K/V
    to stream done) — for shapes with more workgroups than slots these show
    the rounds and the tail."""
    import ctypes
    import numpy as np
    from hyquant_amd import _lib
    L = _lib.lib()
    if not hasattr(L, "hyq_phase_trace_read"):
        raise RuntimeError("phase trace needs the trace build: python -m hyquant_amd.build --trace, "
                           "then HYQ_LIBRARY=hyquant_amd/libhyq_trace.so")
    slots, maxw, nph = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
    L.hyq_phase_trace_geometry(ctypes.byref(slots), ctypes.byref(maxw), ctypes.byref(nph))
    S, MW, NP = slots.value, maxw.value, nph.value
    B, HQ, HKV, N = shape
    G = HQ // HKV
    out = {"shape": {"batch": B, "q_heads": HQ, "kv_heads": HKV, "prefix": N}}
    for mode in ("rotated", "one_copy"):
        nb = algorithmic_bytes(B, HQ, HKV, N)
        R = copies_for(nb) if mode == "rotated" else 1
        states = [make_state(B, HQ, HKV, N, dev, r) for r in range(R)]
        ms, _ = time_rotating(lambda s: run_decode(s[0], s[1], G), states, 10, steps)
        buf = np.zeros(S * MW * NP, dtype=np.uint64)
        nl = ctypes.c_uint32()
        rc = L.hyq_phase_trace_read(buf.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(buf.nbytes), ctypes.byref(nl))
        if rc != 0:
            raise RuntimeError("hyq_phase_trace_read failed")
        tr = buf.reshape(S, MW, NP).astype(np.int64)
        launches = []
        for s in range(S):
            idx = np.nonzero(tr[s][:, 0] > 0)[0]
            if len(idx) == 0:
                continue
            launches.append((int(tr[s][idx[0], NP - 1]), tr[s][: idx.max() + 1]))
        launches.sort(key=lambda x: x[0])
        launches = launches[-min(len(launches), steps, S):]
        med, mx, gaps, ends, spread = [], [], [], [], []
        pct = {"entry": [], "stream_done": [], "stream": []}
        for i, (_, w) in enumerate(launches):
            t0 = w[:, 0].min()
            nt = NP - 1                                       # the last field is the launch index
            rel = (w[:, :nt] - t0) * 0.01                     # 100 MHz ticks -> us
            m_row, x_row = np.zeros(nt), np.zeros(nt)
            for k in range(nt):
                col = rel[:, k][w[:, k] > 0]
                m_row[k], x_row[k] = (np.median(col), col.max()) if len(col) else (np.nan, np.nan)
            med.append(m_row)
            mx.append(x_row)
            end = max(w[:, 10].max(), w[:, 7].max())
            ends.append((end - t0) * 0.01)
            sd = w[:, 4].reshape(-1, 4)
            spread.append(np.median(sd.max(axis=1) - sd.min(axis=1)) * 0.01)
            live = w[:, 0] > 0
            for key, col in (("entry", rel[:, 0][live]), ("stream_done", rel[:, 4][live]),
                             ("stream", (rel[:, 4] - rel[:, 3])[live & (w[:, 3] > 0)])):
                if len(col):
                    pct[key].append(np.percentile(col, [10, 50, 90, 100]))
            if i + 1 < len(launches):
                gaps.append((launches[i + 1][1][:, 0].min() - end) * 0.01)
        med = np.nanmedian(np.stack(med), axis=0)
        mx = np.nanmedian(np.stack(mx), axis=0)
        out[mode] = {"us_per_step": round(ms * 1e3, 3), "launches": len(launches),
                     "wavefronts": int((launches[-1][1][:, 0] > 0).sum()),
                     "phases_us": {PHASES[k]: {"median": round(float(med[k]), 2), "max": round(float(mx[k]), 2)}
                                   for k in range(len(med))},
                     "end_us": round(float(np.median(ends)), 2),
                     "gap_us": round(float(np.median(gaps)), 2) if gaps else None,
                     "wave_spread_us": round(float(np.median(spread)), 2),
                     "entry_pct_us": [round(float(x), 2) for x in np.median(np.stack(pct["entry"]), axis=0)],
                     "stream_done_pct_us": [round(float(x), 2) for x in np.median(np.stack(pct["stream_done"]), axis=0)],
                     "stream_us_pct": [round(float(x), 2) for x in np.median(np.stack(pct["stream"]), axis=0)]}
        del states
        torch.cuda.empty_cache()
        print(f"# phase-trace {mode} {out[mode]}", file=sys.stderr, flush=True)
    return out


def traffic_record():
    """HBM bytes per decode launch measured by the FETCH_SIZE / WRITE_SIZE
    passes over pmc_workload (profiles/decode_config1_traffic.json), or None."""
    path = os.path.join(ROOT, "profiles", "decode_config1_traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-bf16", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="skip the config 3 / config 4 sections")
    ap.add_argument("--pmc", action="store_true", help="run the counter-pass workload only")
    ap.add_argument("--pmc-decode-shapes", action="store_true",
                    help="run the decode counter workload (12 config-2 and 2 config-3 shapes) only")
    ap.add_argument("--phase-trace", action="store_true",
                    help="print the config-1 decode phase timeline from the trace build (libhyq_trace.so)")
    ap.add_argument("--phase-trace-shape", metavar="B,HQ,HKV,N",
                    help="with --phase-trace: the decode shape (default 1,32,8,8192)")
    ap.add_argument("--prefill-only", action="store_true", help="run the config-4 prefill section only")
    ap.add_argument("--pmc-summary", nargs="+", metavar="CSV",
                    help="summarise the FETCH_SIZE, WRITE_SIZE (and optional SQ) passes over "
                         "--pmc-decode-shapes: FETCH_CSV WRITE_CSV [SQ_CSV] (no GPU)")
    ap.add_argument("--prefill-trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="per-kernel table of a kernel trace of --prefill-only (no GPU)")
    ap.add_argument("--boundary-only", action="store_true",
                    help="run the config-3 boundary section (select, freeze, flush) only")
    ap.add_argument("--legacy-only", action="store_true",
                    help="time the legacy-format decode (direct against dequantise-first) only")
    ap.add_argument("--kernel-trace-summary", metavar="KERNEL_TRACE_CSV",
                    help="median duration per kernel and grid of a kernel trace (no GPU)")
    args = ap.parse_args()
    if args.pmc_summary:
        print(json.dumps(pmc_decode_summary(*args.pmc_summary), indent=1))
        return
    if args.prefill_trace_summary:
        print(json.dumps(prefill_trace_summary(args.prefill_trace_summary), indent=1))
        return
    if args.kernel_trace_summary:
        for r in kernel_trace_summary(args.kernel_trace_summary):
            print(json.dumps(r))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(--gpus must be 1)", file=sys.stderr)
        sys.exit(2)
    if args.phase_trace:
        os.environ["HYQ_LIBRARY"] = os.path.join(ROOT, "hyquant_amd", "libhyq_trace.so")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    import hyquant_amd  # noqa: F401  (fails loudly if libhyq.so is missing)
    if args.phase_trace:
        shp = tuple(int(x) for x in args.phase_trace_shape.split(",")) if args.phase_trace_shape else (1, 32, 8, 8192)
        print(json.dumps({"phase_trace": phase_trace(dev, args.steps, shp)}), flush=True)
        return
    if args.pmc_decode_shapes:
        pmc_decode_shapes_workload(dev)
        return
    if args.pmc:
        pmc_workload(dev)
        return
    if args.prefill_only:
        print(json.dumps({"config4_prefill": bench_prefill(dev)}), flush=True)
        return
    if args.boundary_only:
        print(json.dumps({"config3_boundary": bench_boundary(dev)}), flush=True)
        return
    if args.legacy_only:
        print(json.dumps({"legacy_decode": bench_legacy(dev)}), flush=True)
        return

    B, HQ, HKV, N = 1, 32, 8, 8192
    ms, nbytes, R, eager = bench_hybrid(B, HQ, HKV, N, dev, args.warmup, args.steps)
    us = ms * 1e3
    gbs = nbytes / (ms * 1e-3) / 1e9
    Nq, T, S, W = seg_sizes(N)
    res = {
        "metric": METRIC,
        "value": round(us, 3),
        "unit": "us/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Gaussian K/V with N(0,2) per-channel K offsets, int4 K4V4 prefix "
                "quantised on the GPU by hyq_quant_pack)",
        "config": {"workload": "config1: fused hybrid decode, B=1, 32q/8kv, d128, prefix 8192",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "prefix": N,
                   "n_quant": Nq, "n_topk": T, "n_staging": S, "n_window": W,
                   "cache_copies_rotated": R,
                   "timing": f"median of {REPLAYS} HIP-graph replays of K steps, the graphs rotating over the "
                             f"{R} copies (>= 1 GiB between two uses of a copy), HIP events on the kernel's stream",
                   "eager_us_per_step": round(eager * 1e3, 3)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode_kernel (one launch per step)",
                     "algorithmic_bytes_per_launch": nbytes},
    }
    res["accuracy"] = {"decode_config1": {k: (float("%.3e" % x) if isinstance(x, float) else x)
                                          for k, x in decode_error(dev).items()}}
    tr = traffic_record()
    if tr:
        res["roofline"]["traffic"] = tr.get("traffic_bytes_per_launch")
        res["roofline"]["traffic_source"] = "profiles/decode_config1_traffic.json (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)"
    if not args.no_bf16:
        ms16, b16, _, _ = bench_bf16(B, HQ, HKV, N, dev, args.warmup, args.steps)
        res["bf16_comparator"] = {"us_per_step": round(ms16 * 1e3, 3),
                                  "gbs": round(b16 / (ms16 * 1e-3) / 1e9, 1),
                                  "frac_peak": round(b16 / (ms16 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                  "speedup_hybrid_vs_bf16": round(ms16 / ms, 3),
                                  "meets_3x": bool(ms16 / ms >= 3.0)}
    if not args.no_sweep:
        traffic = sweep_traffic_record()
        sweep = []
        for b in (1, 16):
            for n in (1024, 2048, 4096, 8192, 16384, 32768):
                m, nb, _, _ = bench_hybrid(b, HQ, HKV, n, dev, 10, 100)
                row = {"batch": b, "prefix": n, "us_per_step": round(m * 1e3, 3),
                       "gbs": round(nb / (m * 1e-3) / 1e9, 1),
                       "frac_peak": round(nb / (m * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
                if (b, n) in traffic:
                    # HBM bytes per launch from the FETCH_SIZE + WRITE_SIZE
                    # passes (profiles/decode_sweep_traffic.json) over this
                    # row's step time
                    row["counter_traffic_bytes"] = traffic[(b, n)]
                    row["counter_gbs"] = round(traffic[(b, n)] / (m * 1e-3) / 1e9, 1)
                if not args.no_bf16:
                    m16, nb16, _, _ = bench_bf16(b, HQ, HKV, n, dev, 5, 50)
                    row["bf16_us_per_step"] = round(m16 * 1e3, 3)
                    row["bf16_frac_peak"] = round(nb16 / (m16 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)
                    row["speedup_vs_bf16"] = round(m16 / m, 3)
                    row["meets_3x"] = bool(m16 / m >= 3.0)
                sweep.append(row)
                print(f"# sweep {row}", file=sys.stderr, flush=True)
        res["sweep"] = sweep
    if not args.no_extra:
        res["cache_modes"] = bench_modes(dev)
        res["config3_wide_gqa"] = bench_wide_gqa(dev)
        res["config3_boundary"] = bench_boundary(dev)
        res["config4_prefill"] = bench_prefill(dev)
    if not args.no_cpu:
        res["cpu_baseline"] = cpu_baseline()
        res["cpu_baseline_config0"] = cpu_baseline(N=1024, S=37)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
