"""GPU parity of the fused four-segment hybrid decode (hyq_decode_hybrid) and
the bf16 comparator (hyq_decode_bf16) against the float64 oracle.

Tolerance (north-star): max-abs error <= 2e-3 on the bf16 outputs; the
relative error (max-abs / max |ref|) is printed beside it, together with the
error of the reference's own bf16 eager math on the same state."""

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O
from tests.gpu_util import state_to_device, to_dev_bf16

pytestmark = pytest.mark.gpu

ATOL = 2e-3


def _run(st, q, kv_repeat, k_bits=4, v_bits=4, **kw):
    import hyquant_amd as hq
    dev = torch.device("cuda")
    t = state_to_device(st, dev)
    out = hq.fused_d_stage_decode(to_dev_bf16(q, dev), t["k_packed"], t["v_packed"], t["k_scale"], t["v_scale"],
                                  t["k_topk"], t["v_topk"], t["k_staging"], t["v_staging"],
                                  t["k_window"], t["v_window"], k_bits, v_bits, kv_repeat=kv_repeat, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def _check(name, out, ref, eager=None, ref_abs=None):
    """Default: max-abs <= 2e-3 (the benchmark distribution, outputs ~0.1).
    With ref_abs = sum_t p_t|v_t|/l (synthetic peaked cases whose outputs reach
    |o| ~ 4, where bf16 rounding of the output alone exceeds 2e-3): elementwise
    |out - ref| <= 2e-3 + 2^-9 ref_abs + 2^-8 |ref|, i.e. the reference
    kernel's own bf16 rounding of P' = p*s_v (<= 2^-9 ref_abs, F8) plus the
    bf16 rounding of the output (half an ulp, <= 2^-8 |ref|)."""
    diff = np.abs(out - ref)
    err = float(np.max(diff))
    rel = err / float(np.max(np.abs(ref)))
    msg = f"{name}: max-abs {err:.3e} rel {rel:.3e} (max|ref| {float(np.max(np.abs(ref))):.3f})"
    if eager is not None:
        msg += f" | bf16-eager max-abs {float(np.max(np.abs(eager - ref))):.3e}"
    print(msg, flush=True)
    assert np.all(np.isfinite(out))
    if ref_abs is None:
        assert err <= ATOL, msg
    else:
        bound = ATOL + 2.0 ** -9 * ref_abs + 2.0 ** -8 * np.abs(ref)
        bad = np.argwhere(diff > bound)
        for i, j in bad[:6]:
            print(f"  violation at head {i} ch {j}: out {out[i, j]:.6f} ref {ref[i, j]:.6f} "
                  f"ref_abs {ref_abs[i, j]:.6f} bound {bound[i, j]:.3e}", flush=True)
        assert bad.size == 0, msg


@pytest.mark.parametrize("cfg", [
    dict(B=1, HQ=32, HKV=8, N=1024, S=37),     # config 0
    dict(B=1, HQ=32, HKV=8, N=8192, S=64),     # config 1
    dict(B=2, HQ=64, HKV=8, N=2048, S=64),     # Qwen3-32B GQA 8
    dict(B=2, HQ=32, HKV=2, N=2048, S=64),     # GLM-4-9B GQA 16
])
def test_decode_config_parity(cfg):
    print(f"decode cfg {cfg}", flush=True)
    inp = O.make_decode_inputs(W=128, seed=0, **cfg)
    st = O.build_decode_state(inp)
    G = cfg["HQ"] // cfg["HKV"]
    out = _run(st, inp.q_dec, G)
    ref = O.decode_fp64_state(inp.q_dec, st, G)
    eager = O.decode_bf16_eager(inp.q_dec, st, G, cfg["B"]) if cfg["N"] <= 2048 else None
    _check(f"cfg {cfg}", out, ref, eager)


def test_decode_32k_prefix():
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=32768, W=128, S=64, seed=3)
    st = O.build_decode_state(inp)
    out = _run(st, inp.q_dec, 4)
    _check("N=32768", out, O.decode_fp64_state(inp.q_dec, st, 4))


@pytest.mark.parametrize("G", [1, 3, 4, 8, 16])
@pytest.mark.parametrize("lens", [(0, 37, 0, 5), (300, 0, 0, 128), (641, 19, 77, 128), (1000, 33, 127, 3)])
def test_decode_shapes_and_ragged_segments(G, lens):
    nq, T, S, W = lens
    rng = np.random.default_rng(hash((G,) + lens) % (1 << 31))
    BHK, D = 3, 128
    print(f"decode G={G} nq={nq} T={T} S={S} W={W}", flush=True)
    b = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32) * 1.5)
    kp, ks = O.quantize_per_token(b(nq), 4)
    vp, vs = O.quantize_per_token(b(nq), 4)
    st = O.DecodeState(kp, vp, ks, vs, b(T), b(T), b(W), b(W), np.zeros((BHK, 128, D), np.float32),
                       np.zeros((BHK, 128, D), np.float32))
    st.k_ring[:, :S] = b(S)
    st.v_ring[:, :S] = b(S)
    st.ring_ptr = S
    q = O.bf16_round(rng.standard_normal((BHK * G, D)).astype(np.float32) * 2)
    out = _run(st, q, G)
    _check(f"G={G} {lens}", out, O.decode_fp64_state(q, st, G), ref_abs=O.decode_fp64_state(q, st, G, abs_v=True))


def test_decode_split_invariance_and_determinism():
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=4096, W=128, S=64, seed=5)
    st = O.build_decode_state(inp)
    ref = O.decode_fp64_state(inp.q_dec, st, 4)
    outs = []
    for split in (32, 128, 512, 4096, 0):
        o = _run(st, inp.q_dec, 4, split_tokens=split)
        _check(f"split={split}", o, ref)
        outs.append(o)
    again = _run(st, inp.q_dec, 4, split_tokens=0)
    assert np.array_equal(again, outs[-1])


def test_decode_strided_staging_view_and_sm_scale():
    """The cache passes the active slice of its 128-slot ring (a strided view)."""
    import hyquant_amd as hq
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=1024, W=128, S=37, seed=2)
    st = O.build_decode_state(inp)
    dev = torch.device("cuda")
    t = state_to_device(st, dev)
    ring_k = to_dev_bf16(st.k_ring, dev)
    ring_v = to_dev_bf16(st.v_ring, dev)
    q = to_dev_bf16(inp.q_dec, dev)
    out = hq.fused_d_stage_decode(q, t["k_packed"], t["v_packed"], t["k_scale"], t["v_scale"],
                                  t["k_topk"], t["v_topk"], ring_k[:, :37], ring_v[:, :37],
                                  t["k_window"], t["v_window"], 4, 4, kv_repeat=4, sm_scale=0.05)
    ref = O.decode_fp64_state(inp.q_dec, st, 4, sm_scale=0.05)
    _check("strided staging, sm_scale=0.05", out.float().cpu().numpy(), ref)


@pytest.mark.parametrize("fp16", [False, True])
def test_decode_host_paths_bit_identical(fp16):
    """The three host paths of fused_d_stage_decode (the C++ extension, the
    Python fast path, the checked path) fill the same parameters: their
    outputs are bit-identical, with the default and an explicit sm_scale and
    a strided staging view."""
    import hyquant_amd as hq
    from hyquant_amd import decode_d_stage as dd
    fx = dd._load_fast_ext()
    if not fx:
        pytest.skip("hyquant_amd/_hyq_fast.so not built")
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=2048, W=128, S=37, seed=9)
    st = O.build_decode_state(inp)
    dev = torch.device("cuda")
    t = state_to_device(st, dev)
    dt = torch.float16 if fp16 else torch.bfloat16
    cv = (lambda x: x.to(dt)) if fp16 else (lambda x: x)
    ring_k, ring_v = cv(to_dev_bf16(st.k_ring, dev)), cv(to_dev_bf16(st.v_ring, dev))
    q = cv(to_dev_bf16(inp.q_dec, dev))
    segs = [cv(t["k_topk"]), cv(t["v_topk"]), ring_k[:, :37], ring_v[:, :37], cv(t["k_window"]), cv(t["v_window"])]
    for sm in (None, 0.05):
        args = [q, t["k_packed"], t["v_packed"], t["k_scale"], t["v_scale"], *segs, 4, 4, 4, sm, 0]
        ref = hq.fused_d_stage_decode(*args[:13], kv_repeat=4, sm_scale=sm)        # allocates the workspace
        py = dd._fast_decode(*args)
        chk = dd._decode(*args, None, None)
        stream = torch.cuda.current_stream(dev).cuda_stream
        w = dd._ws_raw[(dev.index if dev.index is not None else 0, stream)]
        status, ext = fx.decode(*args[:14], float("nan") if sm is None else sm, 0, stream, w[0], w[1])
        torch.cuda.synchronize()
        assert status == 0
        assert ext.dtype == dt and ext.shape == q.shape
        for name, o in (("python fast path", py), ("checked path", chk), ("extension", ext)):
            assert torch.equal(o.view(torch.int16), ref.view(torch.int16)), (name, sm)


@pytest.mark.parametrize("n,G", [(1000, 4), (8192, 4), (333, 16)])
def test_bf16_comparator(n, G):
    import hyquant_amd as hq
    rng = np.random.default_rng(n)
    BHK, D = 8, 128
    k = O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    v = O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32))
    q = O.bf16_round(rng.standard_normal((BHK * G, D)).astype(np.float32))
    out = hq.decode_bf16_full(to_dev_bf16(q, "cuda"), to_dev_bf16(k, "cuda"), to_dev_bf16(v, "cuda"), kv_repeat=G)
    e = np.zeros((BHK, 0, D), np.float32)
    kp, ks = np.zeros((BHK, 0, 64), np.int8), np.zeros((BHK, 0), np.float16)
    ref = O.decode_fp64(q, kp, kp, ks, ks, k, v, e, e, e, e, kv_repeat=G)
    ref_abs = O.decode_fp64(q, kp, kp, ks, ks, k, v, e, e, e, e, kv_repeat=G, abs_v=True)
    _check(f"bf16 full n={n} G={G}", out.float().cpu().numpy(), ref, ref_abs=ref_abs)


def test_decode_workspace_reuse_interleaved():
    """Calls of different shapes and states issued back to back on one stream
    share the cached workspace: each launch's arrival counters must start at
    zero and end at zero, and no launch may read another's partials."""
    import hyquant_amd as hq
    dev = torch.device("cuda")
    cfgs = {
        "A": dict(B=1, HQ=32, HKV=8, N=8192, S=64, seed=7),
        "B": dict(B=2, HQ=64, HKV=8, N=2048, S=64, seed=8),     # G = 8
        "C": dict(B=8, HQ=32, HKV=8, N=4096, S=64, seed=9),     # 64 KV heads: few long pieces
    }
    data = {}
    for name, cfg in cfgs.items():
        inp = O.make_decode_inputs(W=128, **cfg)
        st = O.build_decode_state(inp)
        data[name] = (inp, st, state_to_device(st, dev), to_dev_bf16(inp.q_dec, dev), cfg["HQ"] // cfg["HKV"])

    def call(name, **kw):
        _, _, t, q, G = data[name]
        return hq.fused_d_stage_decode(q, t["k_packed"], t["v_packed"], t["k_scale"], t["v_scale"],
                                       t["k_topk"], t["v_topk"], t["k_staging"], t["v_staging"],
                                       t["k_window"], t["v_window"], 4, 4, kv_repeat=G, **kw)

    order = ["A", "B", "C", "A", "C", "B"]
    outs = [call(n) for n in order]
    # pieces of 128 int4 tokens' bytes give A 78 pieces per head: two merge batches
    outs.append(call("A", split_tokens=128))
    order.append("A")
    torch.cuda.synchronize()
    refs = {n: O.decode_fp64_state(data[n][0].q_dec, data[n][1], data[n][4]) for n in cfgs}
    for i, (n, o) in enumerate(zip(order, outs)):
        _check(f"interleaved #{i} state {n}", o.float().cpu().numpy(), refs[n])
    assert torch.equal(outs[0], outs[3]) and torch.equal(outs[1], outs[5]) and torch.equal(outs[2], outs[4])



def test_decode_graph_replay_interleaved():
    """The same interleaved calls captured in one HIP graph: every replay
    (with eager decode calls on the same workspace between replays) must give
    outputs bit-identical to the eager calls, so the arrival counters are
    back at zero after every launch and no launch reads another's partials."""
    import hyquant_amd as hq
    dev = torch.device("cuda")
    cfgs = {
        "A": dict(B=1, HQ=32, HKV=8, N=8192, S=64, seed=17),
        "B": dict(B=2, HQ=64, HKV=8, N=2048, S=64, seed=18),    # G = 8: column merge
        "C": dict(B=8, HQ=32, HKV=8, N=4096, S=64, seed=19),    # 64 KV heads
        "D": dict(B=1, HQ=32, HKV=2, N=4096, S=37, seed=20),    # G = 16
    }
    data = {}
    for name, cfg in cfgs.items():
        inp = O.make_decode_inputs(W=128, **cfg)
        st = O.build_decode_state(inp)
        data[name] = (state_to_device(st, dev), to_dev_bf16(inp.q_dec, dev), cfg["HQ"] // cfg["HKV"])

    def call(name, **kw):
        t, q, G = data[name]
        return hq.fused_d_stage_decode(q, t["k_packed"], t["v_packed"], t["k_scale"], t["v_scale"],
                                       t["k_topk"], t["v_topk"], t["k_staging"], t["v_staging"],
                                       t["k_window"], t["v_window"], 4, 4, kv_repeat=G, **kw)

    order = [("A", {}), ("B", {}), ("C", {}), ("D", {}), ("A", {"split_tokens": 128}), ("C", {}), ("B", {})]
    eager = [call(n, **kw) for n, kw in order]        # also sizes the cached workspace before capture
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for n, kw in order:                            # warm-up on the capture stream (its own workspace)
            call(n, **kw)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        outs = [call(n, **kw) for n, kw in order]
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        for i, ((n, _), o) in enumerate(zip(order, outs)):
            assert torch.equal(o, eager[i]), f"replay {rep}, call {i} ({n}) differs from the eager call"
        # eager calls between replays (on the capture stream's workspace as well)
        with torch.cuda.stream(s):
            mid = call("D")
        torch.cuda.synchronize()
        assert torch.equal(mid, eager[3])


BIT_PAIRS = [(4, 4), (4, 2), (2, 4), (8, 8), (2, 2), (4, 8), (8, 4), (2, 8), (8, 2)]


@pytest.mark.parametrize("kb,vb", BIT_PAIRS)
def test_decode_bit_widths_on_config_inputs(kb, vb):
    """The reference's fused kernel takes K_BITS / V_BITS in {2, 4, 8}
    (src/ops/decode_d_stage.py:610-690): every pair, frozen from the same
    prefill, against the fp64 oracle of the same codes."""
    print(f"decode K{kb}V{vb}", flush=True)
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=2048, W=128, S=40, seed=11)
    st = O.freeze(inp.keys, inp.values, inp.query_tail, inp.W, inp.rho, 4, k_bits=kb, v_bits=vb)
    O.append_staging(st, inp.k_new, inp.v_new)
    assert st.k_packed.shape[-1] == 16 * kb and st.v_packed.shape[-1] == 16 * vb
    out = _run(st, inp.q_dec, 4, k_bits=kb, v_bits=vb)
    _check(f"K{kb}V{vb}", out, O.decode_fp64_state(inp.q_dec, st, 4))


@pytest.mark.parametrize("kb,vb", [(8, 8), (2, 2), (4, 2), (2, 8)])
@pytest.mark.parametrize("G", [1, 16])
def test_decode_bit_widths_ragged(kb, vb, G):
    """Random packed bytes, so every code of each width occurs (the quantiser
    never emits the most negative one), random fp16 scales, a ragged prefix."""
    rng = np.random.default_rng(kb * 100 + vb * 10 + G)
    BHK, D, nq, T, S, W = 3, 128, 641, 19, 77, 128
    print(f"decode ragged K{kb}V{vb} G={G}", flush=True)
    b = lambda n: O.bf16_round(rng.standard_normal((BHK, n, D)).astype(np.float32) * 1.5)
    kp = rng.integers(-128, 128, size=(BHK, nq, 16 * kb), dtype=np.int8)
    vp = rng.integers(-128, 128, size=(BHK, nq, 16 * vb), dtype=np.int8)
    # scale magnitudes keep |k| and |v| near those of the bf16 segments
    ks = (rng.uniform(0.5, 2.0, size=(BHK, nq)) / (2 ** (kb - 1))).astype(np.float16)
    vs = (rng.uniform(0.5, 2.0, size=(BHK, nq)) / (2 ** (vb - 1))).astype(np.float16)
    codes = O.unpack_codes(kp, kb)
    assert codes.min() == -(2 ** (kb - 1)) and codes.max() == 2 ** (kb - 1) - 1
    st = O.DecodeState(kp, vp, ks, vs, b(T), b(T), b(W), b(W), np.zeros((BHK, 128, D), np.float32),
                       np.zeros((BHK, 128, D), np.float32), k_bits=kb, v_bits=vb)
    st.k_ring[:, :S] = b(S)
    st.v_ring[:, :S] = b(S)
    st.ring_ptr = S
    q = O.bf16_round(rng.standard_normal((BHK * G, D)).astype(np.float32) * 2)
    out = _run(st, q, G, k_bits=kb, v_bits=vb)
    _check(f"ragged K{kb}V{vb} G={G}", out, O.decode_fp64_state(q, st, G),
           ref_abs=O.decode_fp64_state(q, st, G, abs_v=True))


@pytest.mark.parametrize("kb,vb", [(4, 4), (4, 2)])
def test_decode_batched_ragged_lengths(kb, vb):
    """fused_d_stage_decode_batched (src/ops/decode_d_stage.py:1008-1129):
    sequences of different lengths stacked along BH and padded; the padding
    holds large garbage that must never be attended."""
    import hyquant_amd as hq
    rng = np.random.default_rng(40 + kb + vb)
    D, HKV, G = 128, 2, 4
    lens = [(300, 20), (641, 150), (0, 77), (1000, 5)]      # (prefix, bf16) per sequence
    mq, mb = max(l[0] for l in lens), max(l[1] for l in lens)
    BHK = HKV * len(lens)
    kp = rng.integers(-128, 128, size=(BHK, mq, 16 * kb), dtype=np.int8)
    vp = rng.integers(-128, 128, size=(BHK, mq, 16 * vb), dtype=np.int8)
    ks = (rng.uniform(0.5, 2.0, size=(BHK, mq)) / 2 ** (kb - 1)).astype(np.float16)
    vs = (rng.uniform(0.5, 2.0, size=(BHK, mq)) / 2 ** (vb - 1)).astype(np.float16)
    kbf = O.bf16_round(rng.standard_normal((BHK, mb, D)).astype(np.float32))
    vbf = O.bf16_round(rng.standard_normal((BHK, mb, D)).astype(np.float32))
    lq = np.zeros(BHK, np.int32)
    lb = np.zeros(BHK, np.int32)
    for s, (nq, nb) in enumerate(lens):
        h = slice(s * HKV, (s + 1) * HKV)
        lq[h], lb[h] = nq, nb
        ks[h, nq:] = 60000.0                                 # padding: huge scales and values
        kbf[h, nb:] = 1e4
        vbf[h, nb:] = 1e4
    q = O.bf16_round(rng.standard_normal((BHK * G, D)).astype(np.float32) * 2)
    dev = torch.device("cuda")
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    out = hq.fused_d_stage_decode_batched(to_dev_bf16(q, dev), t(kp), t(vp), t(ks), t(vs),
                                          to_dev_bf16(kbf, dev), to_dev_bf16(vbf, dev), t(lq), t(lb),
                                          kb, vb, kv_repeat=G)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    e = np.zeros((HKV, 0, D), np.float32)
    for s, (nq, nb) in enumerate(lens):
        h = slice(s * HKV, (s + 1) * HKV)
        qs = q[s * HKV * G:(s + 1) * HKV * G]
        args = (qs, kp[h, :nq], vp[h, :nq], ks[h, :nq], vs[h, :nq], kbf[h, :nb], vbf[h, :nb], e, e, e, e)
        ref = O.decode_fp64(*args, k_bits=kb, v_bits=vb, kv_repeat=G)
        ref_abs = O.decode_fp64(*args, k_bits=kb, v_bits=vb, kv_repeat=G, abs_v=True)
        _check(f"batched seq {s} lens {nq}/{nb}", out[s * HKV * G:(s + 1) * HKV * G], ref, ref_abs=ref_abs)


def _bf16_neighbours_ok(out16: np.ndarray, outb: np.ndarray) -> np.ndarray:
    """out16 = fp16(r) and outb = bf16(r) of one float32 r: bf16(out16) equals
    outb unless out16 sits exactly halfway between two bf16 values (then the
    rounding of r decides), where outb must be one of those two.  Below 2^-14
    fp16 is subnormal and coarser than bf16: there |outb - out16| <= 2^-24."""
    x = out16.astype(np.float32)
    rb = O.bf16_round(x)
    lo = O.bf16_round(np.nextafter(x, np.float32(-np.inf)).astype(np.float32))
    hi = O.bf16_round(np.nextafter(x, np.float32(np.inf)).astype(np.float32))
    tiny = (np.abs(x) < 2.0 ** -14) & (np.abs(outb - x) <= 2.0 ** -24)
    return (rb == outb) | ((lo != hi) & ((outb == lo) | (outb == hi))) | tiny


@pytest.mark.parametrize("N,split", [(300, 0), (4096, 0), (4096, 256)])
def test_decode_fp16_model(N, split):
    """An fp16 model: fp16 q and fp16 top-k / staging / window segments.  The
    reference rounds them to bf16 before its products
    (src/ops/decode_d_stage.py:537-541, 240-263) and returns q.dtype (:866):
    the fp16 result is within 2e-3 of the fp64 oracle on the bf16-rounded
    state, and it is the same float32 result as a bf16 call on the
    bf16-rounded inputs, rounded to fp16 instead of bf16 (checked exactly)."""
    import hyquant_amd as hq
    inp = O.make_decode_inputs(B=1, HQ=32, HKV=8, N=N, W=128, S=37, seed=5)
    st = O.build_decode_state(inp)
    G = 4
    rng = np.random.default_rng(N + split)
    # fp16 values with mantissa bits bf16 does not hold
    f16 = lambda a: (a * (1 + rng.uniform(-2 ** -8, 2 ** -8, a.shape))).astype(np.float16)
    names = ("k_topk", "v_topk", "k_staging", "v_staging", "k_window", "v_window")
    seg16 = {n: f16(np.asarray(getattr(st, n), np.float32)) for n in names}
    q16 = (inp.q_dec * rng.uniform(0.9, 1.1, inp.q_dec.shape)).astype(np.float16)
    assert not np.array_equal(O.bf16_round(q16.astype(np.float32)), q16.astype(np.float32))
    # the oracle state: the same values rounded to bf16
    rb = lambda a: O.bf16_round(a.astype(np.float32))
    st.k_topk, st.v_topk = rb(seg16["k_topk"]), rb(seg16["v_topk"])
    st.k_window, st.v_window = rb(seg16["k_window"]), rb(seg16["v_window"])
    st.k_ring[:, :st.ring_ptr] = rb(seg16["k_staging"])
    st.v_ring[:, :st.ring_ptr] = rb(seg16["v_staging"])
    qb = rb(q16)
    dev = torch.device("cuda")
    t = state_to_device(st, dev)
    d16 = {n: torch.from_numpy(np.ascontiguousarray(seg16[n])).to(dev) for n in names}
    print(f"decode fp16 model N={N} split={split}", flush=True)
    out16 = hq.fused_d_stage_decode(torch.from_numpy(q16).to(dev), t["k_packed"], t["v_packed"], t["k_scale"],
                                    t["v_scale"], *[d16[n] for n in names], 4, 4, kv_repeat=G,
                                    split_tokens=split)
    outb = hq.fused_d_stage_decode(to_dev_bf16(qb, dev), t["k_packed"], t["v_packed"], t["k_scale"],
                                   t["v_scale"], *[t[n] for n in names], 4, 4, kv_repeat=G, split_tokens=split)
    torch.cuda.synchronize()
    assert out16.dtype == torch.float16 and outb.dtype == torch.bfloat16
    o16 = out16.float().cpu().numpy()
    ob = outb.float().cpu().numpy()
    _check(f"fp16 model N={N}", o16, O.decode_fp64_state(qb, st, G))
    ok = _bf16_neighbours_ok(o16, ob)
    assert ok.all(), f"{int((~ok).sum())} outputs are not the fp16 rounding of the bf16 call's float32 result"
