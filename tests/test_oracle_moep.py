"""The oracle's MOEP predictor / evictor (oracle/moep.c, a restatement of the
reference's cpp/moe-predictor.cpp) pinned before it checks the cache hooks:

  * against the committed fixtures the reference's own moe_predictor wrote
    (tests/golden/make_moep_golden.py): scores bit for bit, top-8 ids, the
    recall of every update of a 64-step SGD sequence, and after it the scores
    of the model the reference saved;
  * where the reference tree is present, against its moe_predictor built from
    source (oracle/_ref) on its shipped 48-layer models: scores, top-k and an
    online-learning sequence;
  * closed forms: a model whose rows are all zero scores the z-scored bias
    plus the prior on the prev ids; ties rank the lower id first.
"""
import os
import struct

import numpy as np
import pytest

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODELS = "/root/reference/models"


def golden():
    z = np.load(os.path.join(GOLD, "moep_small_expected.npz"))
    cases = []
    for i in range(int(z["n_cases"])):
        lists = {n: z[f"{n}_{i}"] for n in ("prev", "cur", "below", "self_prev")}
        cases.append((int(z[f"il_{i}"]), lists, z[f"truth_{i}"]))
    return z, cases


def test_oracle_matches_golden_scores_topk_and_updates(tmp_path):
    z, cases = golden()
    m = O.Moep(os.path.join(GOLD, "moep_small.bin"))
    assert m.n_expert == 16 and [m.has_layer(l) for l in range(5)] == [True, True, False, True, True]
    for i, (il, l, _) in enumerate(cases):
        s = m.score(il, **l)
        assert np.array_equal(s.view(np.uint32), z["scores"][i].view(np.uint32)), i
        assert list(m.top_k(s, 8)) == list(z["top"][i]), i
    for i, (il, l, t) in enumerate(cases):
        assert np.float32(m.update(il, t, 0.05, **l)) == z["recall"][i], i
    # the model after the updates scores like the one the reference saved
    after = tmp_path / "after.bin"
    after.write_bytes(z["after"].tobytes())
    saved = O.Moep(after)
    rng = np.random.default_rng(4)
    for il in (0, 1, 3, 4):
        for _ in range(20):
            l = {n: rng.integers(0, 16, int(rng.integers(0, 9))).astype(np.int32)
                 for n in ("prev", "cur", "below", "self_prev")}
            assert np.array_equal(m.score(il, **l).view(np.uint32), saved.score(il, **l).view(np.uint32))


def write_flat_model(path, E=8, bias=None, prior=0.5):
    """One layer, prev and cur blocks, every weight row zero."""
    with open(path, "wb") as f:
        f.write(b"MOEP")
        f.write(struct.pack("<11I", 3, 0, 0, E, 1, 8, 2 * E, 1, 2, 0, 0))
        f.write(struct.pack("<3I", 1, 0, E))
        f.write(struct.pack("<3I", 2, E, E))
        f.write(np.asarray([0], np.int32).tobytes())
        f.write(np.asarray([prior], np.float32).tobytes())
        f.write(np.asarray(bias, np.float32).tobytes())
        f.write(np.zeros((2 * E, E), np.float32).tobytes())


def test_closed_form_zero_rows_and_ties(tmp_path):
    E = 8
    bias = np.array([3, 1, 4, 1, 5, 9, 2, 6], np.float32)
    p = tmp_path / "flat.bin"
    write_flat_model(str(p), E, bias, prior=0.5)
    m = O.Moep(p)
    s = m.score(0, prev=[1, 7], cur=[2, 3])
    mu = np.float32(bias.sum(dtype=np.float32) / np.float32(E))
    want = (bias - mu) / (np.sqrt(np.sum((bias - mu) ** 2, dtype=np.float32) / np.float32(E)) + np.float32(1e-9))
    want[[1, 7]] += np.float32(0.5)
    assert np.allclose(s, want, rtol=0, atol=1e-6)
    # equal bias for ids 1 and 3 (both 1): with no prior they tie, the lower id first
    write_flat_model(str(p), E, bias, prior=0.0)
    m = O.Moep(p)
    s = m.score(0)
    assert list(m.top_k(s, 8)) == [5, 7, 4, 2, 0, 6, 1, 3]
    # a NaN ranks last
    s2 = s.copy()
    s2[5] = np.nan
    assert list(m.top_k(s2, 8))[-1] == 5


need_ref = pytest.mark.skipif(O.ref_predictor_lib() is None or not os.path.isdir(MODELS),
                              reason="the reference tree and oracle/_ref are not on this host")


def rand_lists(rng, E):
    return {n: rng.choice(E, int(rng.integers(0, 9)), replace=False).astype(np.int32)
            for n in ("prev", "cur", "below", "self_prev")}


@need_ref
@pytest.mark.parametrize("name", ["predictor-real", "evictor-real"])
def test_oracle_matches_reference_build_on_shipped_models(name):
    path = os.path.join(MODELS, name + ".bin")
    m, r = O.Moep(path), O.RefPredictor(path)
    E = m.n_expert
    rng = np.random.default_rng(12)
    layers = [l for l in range(48) if m.has_layer(l)]
    assert layers == [l for l in range(48) if r.has_layer(l)]
    for c in range(200):
        il = int(rng.choice(layers))
        l = rand_lists(rng, E)
        a, b = m.score(il, **l), r.score(il, E, **l)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), c
        assert list(m.top_k(a, 8)) == list(r.top_k(b, 8))
    for c in range(200):
        il = int(rng.choice(layers))
        l = rand_lists(rng, E)
        t = rng.choice(E, 8, replace=False).astype(np.int32)
        assert np.float32(m.update(il, t, 0.01, **l)) == np.float32(r.update(il, t, 0.01, **l)), c
    for c in range(50):
        il = int(rng.choice(layers))
        l = rand_lists(rng, E)
        assert np.array_equal(m.score(il, **l).view(np.uint32), r.score(il, E, **l).view(np.uint32))


# ---- the cache hooks, pinned where they reduce to what the reference's traces fix ----
def replay_x3t(i, evict=None, pred=None):
    import collections

    import x3t
    slots, experts, frames, routes = x3t.load(i)
    layers = sorted(slots)
    c = O.Cache([slots[l] for l in layers], n_experts=experts[0], **x3t.X3T_KNOBS)
    if evict is not None:
        c.set_evictor(evict)
    if pred is not None:
        c.set_predictor(*pred)
    by = collections.defaultdict(list)
    for s, il, n_ids, n_tok, pairs in routes:
        by[s].append((il, n_tok, [e for e, _ in pairs]))
    got = {0: {l: list(c.frame(l)) for l in layers}}
    for s in range(max(frames)):
        for il, n_tok, ids in by.get(s, []):
            c.observe(il, np.array(ids, np.int32), n_tok)
        c.step()
        got[s + 1] = {l: list(c.frame(l)) for l in layers}
    return [(s, l) for s in frames for l in layers if frames[s][l] != got[s][l]], c


def write_zero_model(path, E=128, n_layers=48, blocks=(1, 2, 3, 4)):
    with open(path, "wb") as f:
        f.write(b"MOEP")
        f.write(struct.pack("<11I", 3, 0, 0, E, n_layers, 8, len(blocks) * E, n_layers, len(blocks), 0, 0))
        for i, kind in enumerate(blocks):
            f.write(struct.pack("<3I", kind, i * E, E))
        f.write(np.arange(n_layers, dtype=np.int32).tobytes())
        f.write(np.zeros(n_layers, np.float32).tobytes())
        f.write(np.zeros((n_layers, E), np.float32).tobytes())
        f.write(np.zeros((n_layers, len(blocks) * E, E), np.float32).tobytes())


@pytest.mark.parametrize("i", [0, 3])
def test_flat_evictor_reduces_to_lru_on_x3t(i, tmp_path):
    """An evictor that scores every expert alike picks by recency alone: the
    reference's own recorded placements (LRU, window admission) reproduce."""
    p = tmp_path / "zero.bin"
    write_zero_model(str(p))
    bad, _ = replay_x3t(i, evict=O.Moep(p))
    assert bad == [], bad[:5]


def test_evictor_that_prefers_hot_experts_changes_the_placement(tmp_path):
    """A planted mistake: an evictor whose bias ranks expert ids in order
    (a different victim than LRU whenever scores differ) breaks the X3T frames,
    so the reduction above is not vacuous."""
    p = tmp_path / "ramp.bin"
    write_zero_model(str(p))
    raw = bytearray(p.read_bytes())
    E, NL = 128, 48
    off = 4 + 44 + 4 * 12 + 4 * NL + 4 * NL             # header, block table, layer list, priors
    bias = np.tile(np.arange(E, dtype=np.float32), NL)
    raw[off:off + bias.nbytes] = bias.tobytes()
    p.write_bytes(bytes(raw))
    bad, _ = replay_x3t(0, evict=O.Moep(p))
    assert bad != []


def test_flat_predictor_issues_the_lowest_ids_and_keeps_the_demand_reserve(tmp_path):
    """A predictor scoring every expert alike names the lowest absent ids
    (ties rank the lower id first): the speculative uploads of a step are at
    most predict_top per layer, and the demand path's max_inserts slots stay
    free (early issue cannot starve)."""
    p = tmp_path / "zero.bin"
    write_zero_model(str(p), n_layers=4, blocks=(1, 2))
    m = O.Moep(p)
    slots = [8, 8, 8, 8]
    c = O.Cache(slots, admit="off", early_issue=True)
    c.set_predictor(m, 3, 0.0)
    rng = np.random.default_rng(1)
    prev_spec = 0
    for t in range(30):
        for l in range(4):
            c.observe(l, rng.choice(128, 8, replace=False).astype(np.int32))
        c.step()
        st = c.predictor_stats()
        assert st["n_spec"] - prev_spec <= 3 * 3             # layers 1..3, predict_top each
        prev_spec = st["n_spec"]
        for l in range(4):
            fr = c.frame(l)
            assert np.sum(fr >= 0) <= slots[l] - 2          # max_inserts spare slots at the boundary
    assert prev_spec > 0
