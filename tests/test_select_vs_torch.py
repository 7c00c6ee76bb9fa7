"""The selector's definition against torch's own arithmetic (CPU only).

The oracle (and the GPU selector) defines a score as bf16(exact dot(qm, k))
with qm = bf16(exact mean of the query tail), and breaks score ties by the
lower index.  The reference (src/patch/_common.py:164-190) computes the mean
and the dot with torch in bf16 (float32 accumulation, one rounding to bf16 at
the end of each op) and takes torch.topk.  This test restates that with
torch on the CPU for both selector calls (the prefill-time call on the query
heads, GQA-native einsum; the freeze-time call on the KV-group mean queries,
src/ops/d_stage_kv_cache.py:130-138) and compares the index sets with the
oracle's on the config-1 inputs (B=1, 32q/8kv, 8192 tokens, W=128) and on two
batch entries of the config-3 inputs (32q/8kv, 16384 tokens, W=256).

Every index where the two sets differ must be explained by one of:
  * a tie: the position's torch score equals the torch score at the cut (the
    two rules break ties differently);
  * a rounding boundary: the position's torch score differs from the
    oracle's, and either the torch mean of its row differs from the oracle
    mean in a channel whose exact mean lies within the float32 accumulation
    bound of a bf16 rounding boundary, or the exact dot of the torch mean
    with the key lies within the float32 bound (2 * 128 * 2^-24 * sum|qm k|)
    of a bf16 rounding boundary.
The counts are printed (pytest -s); the boundary cases are bounded.  On
these inputs every differing index is a tie at the cut (2-3% of the selected
indices: bf16 scores have 8 significant bits, so many keys share the cut
score), the torch and oracle means agree, and the bf16 scores themselves
agree at every position but a handful.
"""

import math

import numpy as np
import pytest
import torch

from oracle import hyq_oracle as O

U32 = 2.0 ** -24


def _near_boundary(x: np.ndarray, eps: np.ndarray) -> np.ndarray:
    """x (float64) lies within eps of a bf16 rounding boundary: a midpoint
    between the bf16 value x rounds to and one of its neighbours (at a power
    of two the spacing below is half the spacing above)."""
    x = np.asarray(x, np.float64)
    r = O.bf16_round_f64(x).astype(np.float64)
    ax = np.maximum(np.abs(r), 2.0 ** -133)
    e = np.floor(np.log2(ax))
    above = 2.0 ** (e - 8)                          # half the spacing away from zero
    below = np.where(ax == 2.0 ** e, above / 2, above)
    up = np.where(r >= 0, r + above, r + below)
    down = np.where(r >= 0, r - below, r - above)
    return (np.abs(x - up) <= eps) | (np.abs(x - down) <= eps)


def _mean_rows_near(tail: np.ndarray, qm_t: np.ndarray, qm_o: np.ndarray) -> np.ndarray:
    """Per row: every channel where the torch mean differs from the oracle's
    has its exact mean within the float32 accumulation bound of a bf16
    rounding boundary (all rows whose means agree are False).  tail [rows,
    n, D] float values, qm [rows, D]."""
    n = tail.shape[1]
    ex = tail.astype(np.float64).mean(axis=1)
    eps = (2 * n + 2) * U32 * np.abs(tail).astype(np.float64).mean(axis=1)
    differ = qm_t != qm_o
    near = _near_boundary(ex, eps)
    return differ.any(axis=1) & np.all(near | ~differ, axis=1)


def _torch_select(qt: torch.Tensor, k: torch.Tensor, window: int, rho: float, kv_repeat: int):
    """src/patch/_common.py:161-190 on torch-CPU bf16 tensors; also returns
    the torch mean and scores."""
    B, H, QL, D = qt.shape
    P = max(0, k.shape[2] - window)
    tail = min(window, QL)
    q_mean = qt[:, :, -tail:, :].mean(dim=2, keepdim=True)
    kp = k[:, :, :P, :]
    if kv_repeat <= 1 or k.shape[1] == H:
        scores = torch.matmul(q_mean, kp.transpose(-1, -2).contiguous()).squeeze(2)
    else:
        HKV = k.shape[1]
        q_g = q_mean.view(B, HKV, kv_repeat, D)
        scores = torch.matmul(q_g, kp.transpose(-1, -2).contiguous()).reshape(B, H, P)
    top_k = min(max(1, int(math.ceil(P * rho))), P)
    _, idx = torch.topk(scores, k=top_k, dim=-1, largest=True, sorted=True)
    return idx.numpy(), q_mean.squeeze(2).float().numpy(), scores.float().numpy()


def _classify(name, idx_t, idx_o, qm_t, mean_near, scores_t, kp_rows):
    """Counts of (tied, rounding-boundary) differing indices; asserts that
    nothing else differs.  mean_near[row]: the row's torch and oracle means
    differ only in channels at a rounding boundary; kp_rows(row) -> the
    row's float64 prefix keys."""
    n_rows, n_diff, n_tie, n_round = idx_t.shape[0], 0, 0, 0
    for r in range(n_rows):
        st, so = set(idx_t[r].tolist()), set(idx_o[r].tolist())
        if st == so:
            continue
        diff = sorted(st ^ so)
        n_diff += len(diff)
        cut = scores_t[r, idx_t[r, -1]]                        # torch score at the cut
        k64 = kp_rows(r)[diff]
        q64 = qm_t[r].astype(np.float64)
        dot_near = _near_boundary(k64 @ q64, 2 * 128 * U32 * (np.abs(k64) @ np.abs(q64)))
        for j, p in enumerate(diff):
            if scores_t[r, p] == cut:
                n_tie += 1
            elif dot_near[j] or mean_near[r]:
                n_round += 1
            else:
                raise AssertionError(f"{name} row {r}: index {p} differs (torch score {scores_t[r, p]}, "
                                     f"cut {cut}) and is neither a tie nor at a bf16 rounding boundary")
    print(f"{name}: {n_rows} rows, {n_diff} differing indices ({n_tie} ties at the cut, "
          f"{n_round} at a bf16 rounding boundary), {int(mean_near.sum())} rows whose mean differs",
          flush=True)
    return n_diff, n_tie, n_round


@pytest.mark.parametrize("cfg", [
    dict(name="config1", B=1, N=8192, W=128, seed=0, rows=None),
    dict(name="config3 (2 of 32 batch entries)", B=2, N=16384, W=256, seed=3, rows=None),
])
def test_selector_definition_against_torch(cfg):
    HQ, HKV, D, rho = 32, 8, 128, 0.05
    G = HQ // HKV
    inp = O.make_decode_inputs(B=cfg["B"], HQ=HQ, HKV=HKV, N=cfg["N"], W=cfg["W"], S=1, seed=cfg["seed"])
    B, N, W = cfg["B"], cfg["N"], cfg["W"]
    qt = torch.from_numpy(inp.query_tail).to(torch.bfloat16)          # [B, HQ, W, D]
    k = torch.from_numpy(inp.keys).to(torch.bfloat16)                 # [B, HKV, N, D]
    keys64 = inp.keys.astype(np.float64)

    # prefill-time call: query heads, GQA-native
    idx_t, qm_t, sc_t = _torch_select(qt, k, W, rho, G)
    idx_o = O.compute_vertical_indices(inp.query_tail, inp.keys, W, rho, kv_repeat=G)
    qm_o = O.mean_bf16(inp.query_tail[:, :, -W:, :], 2)
    tail = inp.query_tail.reshape(B * HQ, W, D)
    near = _mean_rows_near(tail, qm_t.reshape(B * HQ, D), qm_o.reshape(B * HQ, D))
    P = N - W
    n1 = _classify(f"{cfg['name']} prefill-time", idx_t.reshape(B * HQ, -1), idx_o.reshape(B * HQ, -1),
                   qm_t.reshape(B * HQ, D), near, sc_t.reshape(B * HQ, P),
                   lambda r: keys64[r // HQ, (r % HQ) // G, :P])

    # freeze-time call: KV-group mean queries over the window-free prefix
    q_kv = qt.reshape(B, HKV, G, W, D).mean(dim=2)
    q_kv_o = O.group_mean_query(inp.query_tail, HKV)
    # the group means (4 bf16 values, an exact float32 sum, a division by 4)
    # are the oracle's exactly
    assert np.array_equal(q_kv.float().numpy(), q_kv_o.astype(np.float32))
    kpre = k[:, :, :P, :]
    idx_t2, qm_t2, sc_t2 = _torch_select(q_kv, kpre, W, rho, 1)
    idx_o2 = O.compute_vertical_indices(q_kv_o, inp.keys[:, :, :P, :], W, rho)
    qm_o2 = O.mean_bf16(q_kv_o[:, :, -W:, :], 2)
    near2 = _mean_rows_near(q_kv_o.reshape(B * HKV, W, D), qm_t2.reshape(B * HKV, D), qm_o2.reshape(B * HKV, D))
    P2 = P - W
    n2 = _classify(f"{cfg['name']} freeze-time", idx_t2.reshape(B * HKV, -1), idx_o2.reshape(B * HKV, -1),
                   qm_t2.reshape(B * HKV, D), near2, sc_t2.reshape(B * HKV, P2),
                   lambda r: keys64[r // HKV, r % HKV, :P2])
    # the scores themselves: torch's float32-accumulated bf16 products
    # against the oracle's exactly rounded ones, over every position
    so = O.vertical_scores(inp.query_tail, inp.keys, W, kv_repeat=G).reshape(B * HQ, P)
    so2 = O.vertical_scores(q_kv_o, inp.keys[:, :, :P, :], W).reshape(B * HKV, P2)
    n_sc = 0
    for st, so_, qm, krow in ((sc_t.reshape(B * HQ, P), so, qm_t.reshape(B * HQ, D),
                               lambda r: keys64[r // HQ, (r % HQ) // G, :P]),
                              (sc_t2.reshape(B * HKV, P2), so2, qm_t2.reshape(B * HKV, D),
                               lambda r: keys64[r // HKV, r % HKV, :P2])):
        for r, p in zip(*np.nonzero(st != so_)):
            k64, q64 = krow(r)[p], qm[r].astype(np.float64)
            assert _near_boundary(k64 @ q64, 2 * 128 * U32 * (np.abs(k64) @ np.abs(q64))), (r, p)
            n_sc += 1
    print(f"{cfg['name']}: {n_sc} of {B * HQ * P + B * HKV * P2} bf16 scores differ from the oracle's, "
          f"each within the float32 accumulation bound of a bf16 rounding boundary", flush=True)
    # every differing index is a tie at the cut or a rounding-boundary case
    # (asserted in _classify); the boundary cases stay rare
    T, T2 = idx_t.shape[-1], idx_t2.shape[-1]
    assert n1[2] <= 0.005 * B * HQ * T and n2[2] <= 0.005 * B * HKV * T2
