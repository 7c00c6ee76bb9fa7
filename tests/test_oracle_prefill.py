"""Pins for the oracle's hybrid prefill (src/ops/sage_unified.py:398-622) and
per-block int8 quantisation (src/ops/vendor/sageattention/triton/
quant_per_block.py:21-46): known answers of the fp32 add-then-truncate rounding,
an exact-rational rederivation, the window-start table, a per-element brute
force of the key partition, and the reduction to exact causal attention."""

import math
from fractions import Fraction

import numpy as np
import pytest

from oracle import hyq_oracle as O
from tests._exact import to_bf16, to_fp16, to_fp32


def _rand_bf16(rng, shape, scale=1.0):
    return O.bf16_round((rng.standard_normal(shape) * scale).astype(np.float32))


def _codes_exact(block, sm):
    """quant_per_block_int8_kernel by exact rationals: every fp32 operation
    rounded once (x*sm, amax/127, x/scale, +-0.5), then truncation."""
    c = Fraction(float(np.float32(sm)))
    xs = [to_fp32(Fraction(float(x)) * c) for x in block.ravel()]
    amax = max(abs(x) for x in xs)
    scale = to_fp32(amax / 127)
    if scale == 0:
        return np.zeros(block.shape, np.int8), 0.0
    out = []
    for x in xs:
        r = to_fp32(x / scale)
        r = to_fp32(r + (Fraction(1, 2) if r >= 0 else Fraction(-1, 2)))
        out.append(int(r))          # int() truncates toward zero
    return np.array(out, np.int8).reshape(block.shape), float(scale)


def test_per_block_int8_known_answers():
    # amax 127 -> scale 1: half-way values round away from zero
    x = np.array([[127.0, 2.5, -2.5, 0.5, -0.5, 0.0, -0.0, 1.4999999, -127.0]], np.float32)
    codes, sc = O.per_block_int8(x, 1.0, 128)
    assert sc.tolist() == [1.0]
    assert codes.tolist() == [[127, 3, -3, 1, -1, 0, 0, 1, -127]]
    # fp32 quirk of add-then-truncate: r = 0.5 - 2^-25 gives r + 0.5 = 1.0 in fp32
    r = np.float32(0.5) - np.float32(2.0 ** -25)
    x = np.array([[127.0, r]], np.float32)
    assert O.per_block_int8(x, 1.0, 128)[0].tolist() == [[127, 1]]
    # a block of zeros: scale 0, codes 0 (0/0 is not propagated)
    codes, sc = O.per_block_int8(np.zeros((3, 4), np.float32), 0.3, 128)
    assert sc.tolist() == [0.0] and not codes.any()


@pytest.mark.parametrize("blk,sm", [(128, 0.08838834764831845 * O.LOG2E), (64, 1.0), (5, 0.37)])
def test_per_block_int8_matches_rational_rederivation(blk, sm):
    rng = np.random.default_rng(blk)
    x = _rand_bf16(rng, (2, 13, 16), 3.0)
    x[1, 3] = 0.0
    codes, scales = O.per_block_int8(x, sm, blk)
    for h in range(2):
        for i in range((13 + blk - 1) // blk):
            exp_c, exp_s = _codes_exact(x[h, i * blk:(i + 1) * blk], sm)
            assert np.array_equal(codes[h, i * blk:(i + 1) * blk], exp_c)
            assert float(scales[h, i]) == exp_s


def test_window_start_table():
    # floor64(max(0, 128 b - (W - 1))), sage_unified.py:482-485
    assert [O.window_start(b, 128) for b in range(5)] == [0, 0, 128, 256, 384]
    assert [O.window_start(b, 256) for b in range(5)] == [0, 0, 0, 128, 256]
    assert [O.window_start(b, 100) for b in range(4)] == [0, 0, 128, 256]
    assert [O.window_start(b, 1) for b in range(3)] == [0, 128, 256]
    assert [O.window_start(b, 64) for b in range(3)] == [0, 64, 192]


def test_operands_against_rationals():
    rng = np.random.default_rng(1)
    q = _rand_bf16(rng, (1, 1, 3, 8))
    k = _rand_bf16(rng, (1, 1, 5, 8), 2.0)
    v = _rand_bf16(rng, (1, 1, 5, 8))
    op = O.prefill_operands(q, k, v, sm_scale=8 ** -0.5)
    c = Fraction(float(np.float32(8 ** -0.5 * O.LOG2E)))
    for i in range(3):
        for d in range(8):
            exp = to_fp16(to_bf16(to_fp32(Fraction(float(q[0, 0, i, d])) * c)))
            assert Fraction(float(op["q16"][0, 0, i, d])) == exp
    for d in range(8):
        km = to_bf16(sum(Fraction(float(k[0, 0, j, d])) for j in range(5)) / 5)
        assert Fraction(float(op["km"][0, 0, 0, d])) == km
        for j in range(5):
            exp = to_fp16(to_bf16(Fraction(float(k[0, 0, j, d])) - km))
            assert Fraction(float(op["k16"][0, 0, j, d])) == exp


def test_operands_fp16_model_against_rationals_and_torch():
    """The fp16 branch (sage_unified.py:569, :575-576): q16 = fp16(fp32(q) * c)
    with one rounding, km = fp16(mean), k16 = fp16(fp32(k - km)); rederived
    with exact rationals, and q16 / k16 (given km) equal to torch's own fp16
    arithmetic on the same tensors."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(11)
    q = (rng.standard_normal((1, 1, 3, 8)) * 3).astype(np.float16).astype(np.float32)
    k = (rng.standard_normal((1, 1, 5, 8)) * 2 + 0.5).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((1, 1, 5, 8)).astype(np.float16).astype(np.float32)
    assert not np.array_equal(O.bf16_round(q), q)         # fp16 values bf16 cannot hold
    op = O.prefill_operands(q, k, v, sm_scale=8 ** -0.5, fp16=True)
    c = Fraction(float(np.float32(8 ** -0.5 * O.LOG2E)))
    for i in range(3):
        for d in range(8):
            exp = to_fp16(to_fp32(Fraction(float(q[0, 0, i, d])) * c))
            assert Fraction(float(op["q16"][0, 0, i, d])) == exp
    for d in range(8):
        km = to_fp16(sum(Fraction(float(k[0, 0, j, d])) for j in range(5)) / 5)
        assert Fraction(float(op["km"][0, 0, 0, d])) == km
        for j in range(5):
            exp = to_fp16(to_fp32(Fraction(float(k[0, 0, j, d])) - km))
            assert Fraction(float(op["k16"][0, 0, j, d])) == exp
    # torch's fp16 elementwise ops on the same values
    qt = torch.from_numpy(q).to(torch.float16)
    sm_l2e = 8 ** -0.5 * O.LOG2E
    assert np.array_equal((qt * sm_l2e).float().numpy(), op["q16"])
    kt = torch.from_numpy(k).to(torch.float16)
    kmt = torch.from_numpy(op["km"]).to(torch.float16)
    assert np.array_equal((kt - kmt).float().numpy(), op["k16"])
    assert np.array_equal(O.to_fp16(v), v)
    # the bf16 branch differs on these inputs (it rounds q * c to bf16 first)
    assert not np.array_equal(O.prefill_operands(q, k, v, sm_scale=8 ** -0.5)["q16"], op["q16"])


def test_lists_partition_and_duplicates():
    N, W = 700, 100
    vidx = np.array([5, 3, 590, 599, 3, 10_000, -4])           # duplicate, out of range both ways
    vert, rest, nv, nr = O.prefill_lists(vidx, N, W)
    assert vert.tolist() == [0, 3, 3, 5, 590, 599, 599]
    assert len(rest) == 600 - 5 and not set(rest) & set(vert)
    assert set(rest) | set(vert) == set(range(600))
    wla = [O.window_start(b, W) for b in range(6)]
    assert nr.tolist() == [sum(r < w for r in rest) for w in wla]
    assert nv.tolist() == [sum(x < w for x in vert) for w in wla]


def _brute_prefill(q, k, v, vidx, W, qk="int8"):
    """Per-element restatement: for query i and key j <= i decide the category
    directly (window: wla(i // 128) <= j; vertical: j in the index set, once per
    occurrence; rest otherwise), score it, and take one softmax per row."""
    B, HQ, N, D = q.shape
    G = HQ // k.shape[1]
    op = O.prefill_operands(q, k, v)
    P = max(0, N - W)
    out = np.zeros(q.shape)
    for b in range(B):
        for h in range(HQ):
            hk = h // G
            vlist = sorted(min(max(int(x), 0), P - 1) for x in vidx[b, h]) if P else []
            vset = set(vlist)
            rest = [j for j in range(P) if j not in vset]
            rank = {j: r for r, j in enumerate(rest)}
            quant = O.per_block_fp8 if qk == "fp8" else O.per_block_int8
            k8, ksc = quant(op["k16"][b, hk, rest], 1.0, 64) if rest else (None, None)
            q8, qsc = O.per_block_fp8(q, op["c"], 128) if qk == "fp8" else (op["q8"], op["q_scale"])
            for i in range(N):
                wla = max(0, 128 * (i // 128) - (W - 1)) // 64 * 64
                s, vals = [], []
                for j in range(i + 1):
                    if j >= wla:
                        mult = 1
                    elif j in vset:
                        mult = vlist.count(j)
                    else:
                        r = rank[j]
                        dot = sum(float(x) * float(y) for x, y in zip(q8[b, h, i], k8[r]))
                        s.append(dot * float(qsc[b, h, i // 128]) * float(ksc[r // 64]))
                        vals.append(op["v16"][b, hk, j])
                        continue
                    sc = float(np.dot(op["q16"][b, h, i].astype(np.float64), op["k16"][b, hk, j].astype(np.float64)))
                    s += [sc] * mult
                    vals += [op["v16"][b, hk, j]] * mult
                s = np.array(s)
                p = np.exp2(s - s.max())
                out[b, h, i] = p @ np.array(vals, np.float64) / p.sum()
    return out


@pytest.mark.parametrize("N,W,T", [(300, 64, 12), (520, 128, 30), (200, 1, 7)])
def test_hybrid_prefill_matches_per_element_brute_force(N, W, T):
    rng = np.random.default_rng(N + W)
    q = _rand_bf16(rng, (1, 2, N, 16))
    k = _rand_bf16(rng, (1, 1, N, 16), 1.5)
    v = _rand_bf16(rng, (1, 1, N, 16))
    vidx = np.stack([rng.permutation(N - W)[:T] for _ in range(2)])[None]
    vidx[0, 1, 1] = vidx[0, 1, 0]                                  # one repeated index
    got = O.hybrid_prefill_fp64(q, k, v, vidx, W, sm_scale=16 ** -0.5)
    exp = _brute_prefill(q, k, v, vidx, W)
    assert np.abs(got - exp).max() < 1e-12


def test_fp8qk_prefill_matches_per_element_brute_force():
    """The FP8-QK variant (sage_unified_fp8.py:158-311): the same partition
    with the rest keys scored from e4m3 Q and K, element by element."""
    rng = np.random.default_rng(31)
    N, W, T = 300, 64, 12
    q = _rand_bf16(rng, (1, 2, N, 16))
    k = _rand_bf16(rng, (1, 1, N, 16), 1.5)
    v = _rand_bf16(rng, (1, 1, N, 16))
    vidx = np.stack([rng.permutation(N - W)[:T] for _ in range(2)])[None]
    got = O.hybrid_prefill_fp64(q, k, v, vidx, W, sm_scale=16 ** -0.5, qk_mode="fp8")
    exp = _brute_prefill(q, k, v, vidx, W, qk="fp8")
    assert np.abs(got - exp).max() < 1e-12


def test_per_block_fp8_known_answers():
    # amax 448 -> scale 1: the codes are the e4m3 roundings of the values themselves
    x = np.array([[448.0, 17.0, -17.0, 0.3, 1e-4, 0.0, -448.0, 240.0]], np.float32)
    codes, sc = O.per_block_fp8(x[None], 1.0, 2)
    assert sc.tolist() == [[1.0]]
    assert codes[0].tolist() == [[448.0, 16.0, -16.0, 0.3125, 0.0, 0.0, -448.0, 240.0]]
    # an all-zero block gets scale 1 (not 0) and zero codes
    codes, sc = O.per_block_fp8(np.zeros((1, 3, 4), np.float32), 2.0, 8)
    assert sc.tolist() == [[1.0]] and not codes.any()


def test_per_block_fp8_matches_rational_rederivation():
    """Each fp32 step rounded once by exact rationals (x * sm, amax / 448,
    x / scale), then the nearest e4m3 grid value (ties to even mantissa)."""
    grid = _e4m3_values()
    rng = np.random.default_rng(7)
    x = O.bf16_round((rng.standard_normal((64, 16)) * 3).astype(np.float32))
    sm = 0.0883883
    codes, sc = O.per_block_fp8(x, sm, 64)
    c = Fraction(float(np.float32(sm)))
    xs = [to_fp32(Fraction(float(t)) * c) for t in x.ravel()]
    scale = to_fp32(max(abs(t) for t in xs) / 448)
    assert float(scale) == float(sc[0])
    for t, got in zip(xs, codes.ravel()):
        r = float(to_fp32(t / scale))
        r = min(max(r, -448.0), 448.0)
        a = abs(r)
        i = int(np.searchsorted(grid, a))
        cands = [grid[j] for j in (i - 1, i) if 0 <= j < len(grid)]
        best = min(cands, key=lambda g: (abs(g - a), _mant_odd(g)))
        assert got == math.copysign(best, r) or (best == 0 and got == 0)


def _mant_odd(g):
    """1 when the e4m3 value g has an odd mantissa (loses a round-to-even tie)."""
    if g == 0:
        return 0
    e = max(math.floor(math.log2(g)), -6)
    return int(round(g / 2.0 ** (e - 3))) & 1


@pytest.mark.parametrize("W", [64, 300])
def test_hybrid_prefill_reduces_to_exact_attention(W):
    """W >= N, or int8 rest scoring switched off, leaves one softmax over every
    key j <= i exactly once: textbook causal attention on (q16, k16, v16)."""
    rng = np.random.default_rng(W)
    q = _rand_bf16(rng, (1, 4, 290, 32))
    k = _rand_bf16(rng, (1, 2, 290, 32), 1.5)
    v = _rand_bf16(rng, (1, 2, 290, 32))
    vidx = np.stack([rng.permutation(max(1, 290 - W))[:9] for _ in range(4)])[None]
    op = O.prefill_operands(q, k, v)
    exact = O.exact_causal_attention(op["q16"], op["k16"], op["v16"], sm_scale=math.log(2))
    got = O.hybrid_prefill_fp64(q, k, v, vidx, W, int8_rest=(W >= 290))
    assert np.abs(got - exact).max() < 1e-12
    # smoothing only shifts each row's logits by a constant (up to rounding)
    raw = O.exact_causal_attention(q, k, v)
    assert np.abs(exact - raw).max() < 2e-2


def test_hybrid_prefill_int8_error_is_small():
    q, k, v = O.make_prefill_inputs(B=1, HQ=4, HKV=1, N=640, W=128, seed=3)
    from oracle.hyq_oracle import compute_vertical_indices
    vidx = compute_vertical_indices(q, k, 128, 0.05, kv_repeat=4)
    got = O.hybrid_prefill_fp64(q, k, v, vidx, 128)
    ref = O.exact_causal_attention(q, k, v)
    mse = float(((got - ref) ** 2).mean())
    assert mse < 1e-4, mse


# ---------------------------------------------------------------------------
# sage_unified_attention (window-only modes)
# ---------------------------------------------------------------------------

def test_unified_w0_partition_reduces_to_exact_attention():
    """W = 0 with int8 scoring off: one softmax over every key j <= i exactly
    once, i.e. textbook causal attention on (q16, k16, v16)."""
    rng = np.random.default_rng(11)
    q = _rand_bf16(rng, (1, 4, 330, 32))
    k = _rand_bf16(rng, (1, 2, 330, 32), 1.5)
    v = _rand_bf16(rng, (1, 2, 330, 32))
    op = O.prefill_operands(q, k, v)
    exact = O.exact_causal_attention(op["q16"], op["k16"], op["v16"], sm_scale=math.log(2))
    got = O.unified_prefill_fp64(q, k, v, 0, int8=False)
    assert np.abs(got - exact).max() < 1e-12


def test_unified_w0_matches_per_element_brute_force():
    """W = 0 with int8 scoring, element by element: query i attends keys
    0..i with s = q8[i] . k8[j] * q_scale[i // 128] * k_scale[j // 64], K
    quantised per 64 positions of the whole (smoothed) sequence."""
    rng = np.random.default_rng(12)
    N, D = 300, 16
    q = _rand_bf16(rng, (1, 2, N, D))
    k = _rand_bf16(rng, (1, 1, N, D), 1.5)
    v = _rand_bf16(rng, (1, 1, N, D))
    op = O.prefill_operands(q, k, v, sm_scale=D ** -0.5)
    k8, ksc = O.per_block_int8(op["k16"][0, 0], 1.0, 64)
    got = O.unified_prefill_fp64(q, k, v, 0, sm_scale=D ** -0.5)
    exp = np.zeros_like(got)
    for h in range(2):
        for i in range(N):
            s = [float(np.dot(op["q8"][0, h, i].astype(np.int64), k8[j].astype(np.int64)))
                 * float(op["q_scale"][0, h, i // 128]) * float(ksc[j // 64]) for j in range(i + 1)]
            s = np.array(s)
            p = np.exp2(s - s.max())
            exp[0, h, i] = p @ op["v16"][0, 0, :i + 1].astype(np.float64) / p.sum()
    assert np.abs(got - exp).max() < 1e-12


def test_unified_int8_error_is_small():
    q, k, v = O.make_prefill_inputs(B=1, HQ=4, HKV=1, N=520, W=128, seed=4)
    ref = O.exact_causal_attention(q, k, v)
    for W in (0, 128):
        got = O.unified_prefill_fp64(q, k, v, W)
        mse = float(((got - ref) ** 2).mean())
        assert mse < 1e-4, (W, mse)


# ---------------------------------------------------------------------------
# OCP e4m3 rounding and the fp8-PV mode
# ---------------------------------------------------------------------------

def _e4m3_values():
    """Every finite non-negative e4m3fn value, from its bit patterns."""
    vals = []
    for e in range(16):
        for m in range(8):
            if e == 15 and m == 7:
                continue                       # NaN encoding
            vals.append(m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7))
    return np.array(sorted(set(vals)))


def test_e4m3_round_grid_ties_and_torch():
    torch = pytest.importorskip("torch")
    vals = _e4m3_values()
    assert vals[-1] == 448.0 and len(vals) == 127
    assert np.array_equal(O.e4m3_round(vals), vals)
    assert np.array_equal(O.e4m3_round(-vals), -vals)
    # midpoints go to the neighbour with the even mantissa
    mids = (vals[:-1] + vals[1:]) / 2
    got = O.e4m3_round(mids)
    ref = torch.from_numpy(mids).to(torch.float32).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(got, ref)
    # random values in range against torch's conversion
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(20000) * np.exp2(rng.uniform(-12, 8, 20000))).astype(np.float32)
    x = x[np.abs(x) < 448]
    ref = torch.from_numpy(x).to(torch.float8_e4m3fn).to(torch.float64).numpy()
    assert np.array_equal(O.e4m3_round(x), ref)
    # hand known answers: ties to even, subnormal spacing, saturation
    assert list(O.e4m3_round([1.0625, 1.1875, 2 ** -10, 3 * 2 ** -10, 464.0, 1000.0, -1000.0])) == \
        [1.0, 1.25, 0.0, 2 ** -8, 448.0, 448.0, -448.0]


def test_fp8_prefill_channel_scale_invariance():
    """Scaling a V channel by a power of two scales only that output channel by
    the same factor (the per-channel scale absorbs it exactly)."""
    q, k, v = O.make_prefill_inputs(B=1, HQ=2, HKV=1, N=300, W=64, seed=11)
    vidx = O.compute_vertical_indices(q, k, 64, 0.05, kv_repeat=2)
    base = O.hybrid_prefill_fp64(q, k, v, vidx, 64, pv_mode="fp8")
    f = np.exp2(np.arange(128) % 7 - 3).astype(np.float32)
    scaled = O.hybrid_prefill_fp64(q, k, v * f, vidx, 64, pv_mode="fp8")
    assert np.array_equal(scaled, base * f)


def test_fp8_prefill_uniform_scores_closed_form():
    """q = 0: every attended key scores 0, so p' = 2^8.807 for all of them; the
    output of row i is (448 sum_rest V8 + fp16(p') sum_other V16') vs / (n p')."""
    N, W = 200, 64
    q, k, v = O.make_prefill_inputs(B=1, HQ=1, HKV=1, N=N, W=W, seed=12)
    q = np.zeros_like(q)
    vidx = np.array([[[3, 17, 50, 99]]], np.int64)
    got = O.hybrid_prefill_fp64(q, k, v, vidx, W, pv_mode="fp8")[0, 0]
    vs, v8, v16 = O.fp8_v_operands(v)
    vs, v8, v16 = vs[0, 0, 0].astype(np.float64), v8[0, 0], v16[0, 0].astype(np.float64)
    pp = 2.0 ** 8.807
    p16 = float(np.float16(pp))
    vert = set(int(x) for x in vidx[0, 0])
    for i in (0, 63, 64, 127, 128, 150, 199):
        wla = O.window_start(i // 128, W)
        num = np.zeros(128)
        n = 0
        for j in range(i + 1):
            if j >= wla:                                  # window key
                num += p16 * v16[j]
            elif j in vert and j < N - W:                 # vertical key below wla
                num += p16 * v16[j]
            else:                                         # rest key
                num += 448.0 * v8[j]
            n += 1
        np.testing.assert_allclose(got[i], num / (n * pp) * vs, rtol=1e-12, atol=1e-15)


def test_fp8_prefill_error_against_exact_attention():
    q, k, v = O.make_prefill_inputs(B=1, HQ=2, HKV=1, N=512, W=128, seed=13)
    vidx = O.compute_vertical_indices(q, k, 128, 0.05, kv_repeat=2)
    exact = O.exact_causal_attention(q, k, v)
    f16 = O.hybrid_prefill_fp64(q, k, v, vidx, 128)
    f8 = O.hybrid_prefill_fp64(q, k, v, vidx, 128, pv_mode="fp8")
    mse16 = float(np.mean((f16 - exact) ** 2))
    mse8 = float(np.mean((f8 - exact) ** 2))
    print(f"MSE vs exact: fp16 PV {mse16:.3e}, fp8 PV {mse8:.3e}")
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, 128, abs_v=True)
    # e4m3 keeps 3 mantissa bits: P8 and V8 each within 2^-4 relative
    assert np.all(np.abs(f8 - f16) <= 2.0 ** -3 * ref_abs + 1e-6)
    assert mse8 < 1e-3


def test_prefill_blocks_option_equals_full_computation():
    """Restricting the restatement to some query blocks gives those rows
    exactly as the full computation does (and zeros elsewhere), for the
    hybrid, fp8 and window-only forms."""
    rng = np.random.default_rng(61)
    q = O.bf16_round(rng.standard_normal((1, 2, 700, 128)).astype(np.float32))
    k = O.bf16_round(rng.standard_normal((1, 1, 700, 128)).astype(np.float32) * 1.5)
    v = O.bf16_round(rng.standard_normal((1, 1, 700, 128)).astype(np.float32))
    vidx = rng.permutation(600)[:40].reshape(1, 1, 40).repeat(2, axis=1)
    blocks = [0, 3, 5]
    rows = np.concatenate([np.arange(b * 128, min(700, (b + 1) * 128)) for b in blocks])
    other = np.setdiff1d(np.arange(700), rows)
    for kw in ({}, {"pv_mode": "fp8"}, {"qk_mode": "fp8"}):
        full = O.hybrid_prefill_fp64(q, k, v, vidx, 100, **kw)
        part = O.hybrid_prefill_fp64(q, k, v, vidx, 100, blocks=blocks, **kw)
        assert np.array_equal(part[:, :, rows], full[:, :, rows]) and not part[:, :, other].any()
    full = O.unified_prefill_fp64(q, k, v, 100)
    part = O.unified_prefill_fp64(q, k, v, 100, blocks=blocks)
    assert np.array_equal(part[:, :, rows], full[:, :, rows])
    full = O.unified_prefill_fp64(q, k, v, 0)
    part = O.unified_prefill_fp64(q, k, v, 0, blocks=blocks)
    assert np.array_equal(part[:, :, rows], full[:, :, rows])


def test_round_span_brackets_every_perturbed_rounding():
    """_round_span(x) is zero exactly where every x' within a relative
    FP8_AMBIGUITY of x rounds like x (e4m3 and fp16), and otherwise equals the
    step between the two possible roundings: checked by brute force over
    random perturbations, and on a known e4m3 midpoint (1.0625 between 1 and
    1.125) and a value far from any midpoint (1.03)."""
    rng = np.random.default_rng(62)
    x = np.exp2(rng.uniform(-12, 8.8, 200000))
    f16 = lambda t: O.to_fp16(np.asarray(t, np.float32)).astype(np.float64)
    for rnd in (O.e4m3_round, f16):
        span = O._round_span(x, rnd, O.FP8_AMBIGUITY)
        base = rnd(x)
        for _ in range(4):
            d = rng.uniform(-1, 1, x.shape) * O.FP8_AMBIGUITY
            moved = rnd(x * (1 + d))
            assert np.all((moved == base) | (span > 0))
            assert np.all(np.abs(moved - base) <= span + 0.0)
    assert O._round_span(np.array([1.0625]), O.e4m3_round, 2.0 ** -14)[0] == 0.125
    assert O._round_span(np.array([1.03]), O.e4m3_round, 2.0 ** -14)[0] == 0.0


def test_fp8_tight_bound_rejects_planted_rounding_mistakes():
    """The bound of the GPU test test_prefill_fp8_pv_tight_where_running_max_is_exact
    has teeth: on its input family the honest restatement (rounded to bf16)
    satisfies it everywhere, while a restatement whose e4m3 rounding truncates,
    or scales every rest-key P' by 1%, violates it on most elements."""
    from tests.gpu_util import bf16_bracket, first_tile_max_inputs
    rng = np.random.default_rng(51)
    q, k, v, vidx = first_tile_max_inputs(rng, 1, 4, 1, 1000, 100, 45)
    ref, slack, exact = O.hybrid_prefill_fp64(q, k, v, vidx, 100, pv_mode="fp8", fp8_detail=True)
    ref_abs = O.hybrid_prefill_fp64(q, k, v, vidx, 100, pv_mode="fp8", abs_v=True)
    eps = slack + 2.0 ** -13 * ref_abs + 2.0 ** -15 * np.abs(ref) + 1e-6
    assert exact.mean() > 0.99
    ex = exact[..., None]
    assert not (bf16_bracket(O.bf16_round_f64(ref), ref, eps) & ex).any()
    honest = O.e4m3_round

    def truncating(x):
        x = np.asarray(x, np.float64)
        a = np.minimum(np.abs(x), O.FP8_MAX)
        with np.errstate(divide="ignore"):
            e = np.maximum(np.floor(np.log2(np.where(a > 0, a, 1.0))), -6.0)
        r = np.floor(a / np.exp2(e - 3.0)) * np.exp2(e - 3.0)
        return np.where(x < 0, -r, r)

    try:
        for planted in (truncating, lambda x: honest(np.asarray(x) * 1.01)):
            O.e4m3_round = planted
            wrong = O.bf16_round_f64(O.hybrid_prefill_fp64(q, k, v, vidx, 100, pv_mode="fp8"))
            O.e4m3_round = honest
            assert (bf16_bracket(wrong, ref, eps) & ex).mean() > 0.3
    finally:
        O.e4m3_round = honest
