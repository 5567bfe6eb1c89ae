"""Pins for the oracle's router lookahead (or_ahead; k_moe_ahead_scores/_post,
patches/0010-team-and-streaming.patch:382-474), CPU only:

  * integer-valued weights, inputs and ratios make every score exact in any
    summation order, so the ranking is fixed by the mathematics: the k best
    experts best first, the lower id first on a tie (the reference's warp
    argmax rule, 0010:420-430), then only those whose table entry is the dummy,
    in rank order (0010:437-439);
  * on random inputs the scores equal the router's canonical logits of the f32
    products x * r (the lookahead is the router of the target layer applied to
    a rescaled input), and the kept ids match an fp64 ranking wherever the
    fp64 order is not within fp32 noise;
  * r = g_T / g_L makes W_T . (x_L * r) the target router on rmsnorm(residual) * g_T
    (what the reference's probe measured, STREAMING-IMPLEMENTATION.md).
"""
import numpy as np
import pytest

from oracle import oracle as O

rng = np.random.default_rng(5)
E, H = 128, 2048


def brute(scores, table, dummy, k):
    order = sorted(range(len(scores)), key=lambda e: (-scores[e], e))[:k]
    return [e for e in order if table[e] == dummy]


@pytest.mark.parametrize("k", [8, 4, 1])
def test_integer_inputs_exact_with_ties(k):
    for trial in range(20):
        W = rng.integers(-3, 4, (E, H)).astype(np.float32)
        x = rng.integers(-2, 3, H).astype(np.float32)
        r = rng.integers(1, 3, H).astype(np.float32)
        W[7] = W[3]                       # ties: 3 and 7 score the same, so do 90 and 20
        W[90] = W[20]
        S = 56
        table = np.where(rng.random(E) < 0.6, rng.integers(0, S, E), S).astype(np.int32)
        exact = (W.astype(np.int64) @ (x.astype(np.int64) * r.astype(np.int64))).astype(np.float64)
        ids, scores = O.ahead(W, x, r, table, S, k)
        assert np.array_equal(scores.astype(np.float64), exact)
        assert list(ids) == brute(exact, table, S, k)


def test_tie_prefers_lower_id_and_filter_keeps_rank_order():
    W = np.zeros((E, H), np.float32)
    x = np.ones(H, np.float32)
    r = np.ones(H, np.float32)
    for e, v in ((9, 5.0), (4, 5.0), (100, 7.0), (50, 6.0), (51, 6.0), (2, 1.0)):
        W[e, 0] = v
    table = np.full(E, 56, np.int32)
    table[100] = 3                       # resident: dropped from the candidates, not re-ranked
    ids, _ = O.ahead(W, x, r, table, 56, 5)
    assert list(ids) == [50, 51, 4, 9]   # ranks: 100, 50, 51, 4, 9
    ids, _ = O.ahead(W, x, r, table, 56, 1)
    assert list(ids) == []               # the best one is resident


def test_nan_ranks_last():
    W = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    W[11, 5] = np.nan
    x = rng.normal(size=H).astype(np.float32)
    ids, scores = O.ahead(W, x, np.ones(H, np.float32), np.full(E, 56, np.int32), 56, 8)
    assert np.isnan(scores[11]) and 11 not in ids and len(ids) == 8


def test_scores_are_the_router_logits_of_the_rescaled_input():
    W = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    x = rng.normal(size=H).astype(np.float32)
    r = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    xr = (x * r).astype(np.float32)
    _, scores = O.ahead(W, x, r, np.full(E, 56, np.int32), 56, 8)
    _, _, _, probs = O.route(W, xr, 8)
    # the router's probabilities are a softmax of exactly these logits
    lg = scores.astype(np.float64)
    p = np.exp(lg - lg.max())
    p /= p.sum()
    assert np.allclose(p, probs, rtol=1e-5, atol=1e-9)
    ids_r, _, _, _ = O.route(W, xr, 8)
    ids_a, _ = O.ahead(W, x, r, np.full(E, 56, np.int32), 56, 8)
    assert list(ids_a) == list(ids_r)       # same top-8, same order (softmax is monotone)


def test_random_inputs_match_fp64_ranking():
    agree = 0
    for trial in range(30):
        W = rng.normal(0, 0.02, (E, H)).astype(np.float32)
        x = rng.normal(size=H).astype(np.float32)
        r = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
        table = np.where(rng.random(E) < 0.5, 3, 56).astype(np.int32)
        s64 = W.astype(np.float64) @ (x * r).astype(np.float32).astype(np.float64)
        order = np.argsort(-s64, kind="stable")
        gaps = np.abs(np.diff(s64[order][:9]))
        if gaps.min() < 1e-5:
            continue                         # fp32 noise could legitimately swap a pair
        ids, _ = O.ahead(W, x, r, table, 56, 8)
        assert list(ids) == brute(s64, table, 56, 8)
        agree += 1
    assert agree >= 20


def test_ratio_gives_target_router_on_the_residual():
    # x_L = rmsnorm(res) * g_L;  x_L * (g_T / g_L) == rmsnorm(res) * g_T up to rounding
    res = rng.normal(size=H).astype(np.float32)
    gL = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    gT = (1 + 0.1 * rng.normal(size=H)).astype(np.float32)
    n = (res / np.sqrt(np.mean(res.astype(np.float64) ** 2))).astype(np.float32)
    xL = (n * gL).astype(np.float32)
    W = rng.normal(0, 0.02, (E, H)).astype(np.float32)
    _, s_ahead = O.ahead(W, xL, (gT / gL).astype(np.float32), np.full(E, 56, np.int32), 56, 8)
    s_true = W.astype(np.float64) @ (n.astype(np.float64) * gT)
    assert np.max(np.abs(s_ahead - s_true)) < 1e-4
