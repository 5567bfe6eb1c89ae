"""The product's slot-table state machine (libmoeprefetch.so, device=-1 host
mode: no GPU, every upload completes at once) against the reference's engine
traces and against the oracle on synthetic routing streams (CPU only)."""
import collections
import os

import numpy as np
import pytest

import x3t
from moep_models import write_moep
from moe_prefetch import MoeCache
from moe_prefetch.workload import zipf_targets
from oracle import oracle as O


def product_cache(slots, **kw):
    return MoeCache(len(slots), n_experts=kw.pop("n_experts", 128), slot_profile=list(slots),
                    device=-1, **kw)


@pytest.mark.parametrize("i", [0, 1, 2, 3])
def test_product_reproduces_x3t(i, tmp_path):
    slots, experts, frames, routes = x3t.load(i)
    layers = sorted(slots)
    c = product_cache([slots[l] for l in layers], max_inserts=2, admit="window", admit_window=8,
                      batch_tables=True)
    rp, mp = str(tmp_path / "routes.txt"), str(tmp_path / "map.txt")
    c.trace_open(rp, mp)
    by = collections.defaultdict(list)
    for s, il, n_ids, n_tok, pairs in routes:
        by[s].append((il, n_tok, [e for e, _ in pairs]))
    for s in range(max(frames)):
        for il, n_tok, ids in by.get(s, []):
            c.observe(il, np.array(ids, np.int32), n_tok)
        c.step()
    c.close()
    # byte-identical trace files
    assert open(rp).read() == x3t.read_text(os.path.join(x3t.GOLDEN, f"{i}.routes-record.txt.gz"))
    assert open(mp).read() == x3t.read_text(os.path.join(x3t.GOLDEN, f"{i}.map.txt.gz"))


KNOBS = [
    dict(admit="off"),
    dict(admit="window", admit_window=8),
    dict(admit="window", admit_window=3, max_inserts=1),
    dict(admit="heat", admit_half=16, admit_floor=1.0),
    dict(admit="heat", admit_half=64, admit_floor=0.0, max_inserts=3),
    dict(admit="off", early_issue=True),
    dict(admit="window", early_issue=True),
    dict(admit="heat", early_issue=True, admit_half=8),
    dict(admit="window", deterministic=True),
    dict(admit="window", cache_prior=0.01, batch_tables=True),
]


@pytest.mark.parametrize("knobs", KNOBS, ids=lambda k: ",".join(f"{a}={b}" for a, b in k.items()))
def test_product_matches_oracle(knobs):
    L, T = 6, 160
    slots = [12, 20, 8, 16, 12, 32]
    tg = [zipf_targets(99, l, T, s=1.0, reuse=0.5) for l in range(L)]
    ok = dict(knobs)
    ok["admit"] = knobs.get("admit", "off")
    oc = O.Cache(slots, **{k: v for k, v in ok.items()})
    pc = product_cache(slots, **knobs)
    for t in range(T):
        for l in range(L):
            oc.observe(l, tg[l][t])
            pc.observe(l, tg[l][t])
        oc.step()
        pc.step()
        for l in range(L):
            assert np.array_equal(oc.frame(l), pc.frame(l)), (t, l)
            ot, op = oc.table(l)
            pt, pp = pc.table(l)
            assert np.array_equal(ot, pt) and np.array_equal(op, pp)
    os_, ps = oc.stats(), pc.stats()
    for k in ("n_steps", "clock", "n_hit", "n_miss", "n_uploads", "n_scheduled", "n_published",
              "n_admit_ok", "n_admit_denied", "n_table_flushes"):
        assert os_[k] == ps[k], k
    assert ps["n_hit"] + ps["n_miss"] == L * T * 8


def test_batched_tokens_observe_token_major():
    # n_tok > 1: ids are visited token-major, one pending list, dedup across tokens
    slots = [16]
    oc = O.Cache(slots, admit="off")
    pc = product_cache(slots, admit="off")
    rng = np.random.default_rng(5)
    for t in range(40):
        ids = rng.integers(0, 128, size=(4, 8)).astype(np.int32)
        oc.observe(0, ids.reshape(-1), 4)
        pc.observe(0, ids.reshape(-1), 4)
        oc.step()
        pc.step()
        assert np.array_equal(oc.frame(0), pc.frame(0))


def test_invariants_hold():
    L, T = 4, 300
    slots = [8, 8, 16, 24]
    pc = product_cache(slots, admit="window")
    tg = [zipf_targets(7, l, T) for l in range(L)]
    for t in range(T):
        for l in range(L):
            pc.observe(l, tg[l][t])
        pc.step()
        for l in range(L):
            fr = pc.frame(l)
            res = fr[fr >= 0]
            assert len(set(res.tolist())) == len(res)           # no expert in two slots
            tbl, _ = pc.table(l)
            for s, e in enumerate(fr):
                if e >= 0:
                    assert tbl[e] == s
            assert np.sum(tbl < slots[l]) == len(res)            # dummy for every absent expert
    st = pc.stats()
    assert st["n_scheduled"] <= 2 * L * T                         # <= max_inserts per layer per step


def test_from_env_reads_reference_variables():
    env = {"LLAMA_MOE_ADMIT": "window", "LLAMA_MOE_ADMIT_WINDOW": "5", "LLAMA_MOE_BATCH_TABLES": "1",
           "LLAMA_MOE_CACHE_PRIOR": "0.01", "LLAMA_MOE_SLOT_PROFILE": "0:88,2:40",
           "LLAMA_MOE_DETERMINISTIC": "1"}
    c = MoeCache.from_env(4, 56, env=env, device=-1)
    assert c.slots == [88, 56, 40, 56]
    assert c.requires_sync()
    _, prior = c.table(0)
    assert prior.shape == (128,) and not prior.any()


def test_from_env_survives_models_that_do_not_load(tmp_path, capfd):
    # an evictor path that does not exist and a predictor with a PCA block:
    # each is reported loudly and serving goes on without it (patches/0006:521-556)
    pca = str(tmp_path / "pca.bin")
    write_moep(pca, 128, 4, [0, 1, 2], blocks=(1, 2), seed=3, pca=(8, 16))
    env = {"LLAMA_MOE_EVICTOR": str(tmp_path / "missing.bin"), "LLAMA_MOE_PREDICTOR": pca,
           "LLAMA_MOE_PREDICT_TOP": "3", "LLAMA_MOE_ADMIT": "window"}
    c = MoeCache.from_env(4, 56, env=env, device=-1)
    err = capfd.readouterr().err
    assert "EVICTOR NOT LOADED" in err and "PREDICTOR NOT LOADED" in err
    assert c.predictor_stats() == {"n_updates": 0, "recall_sum": 0.0, "n_spec": 0}
    for t in range(4):                      # the cache serves as if neither variable were set
        for l in range(4):
            c.observe(l, [t, t + 1, 7, 9, 11, 13, 15, 17])
        c.step()
    assert c.stats()["n_steps"] == 4
    c.close()


def test_bad_knob_is_loud():
    with pytest.raises(ValueError):
        MoeCache(2, admit="sometimes", device=-1)


def test_decode_path_arguments():
    # split 0..3 and graph 0 (direct launches), 1 (a graph where it is faster)
    # or 2 (always a graph); anything else is MOE_ERR_ARG and changes nothing
    from moe_prefetch import _lib
    c = product_cache([8, 8])
    for split, graph in ((0, 0), (0, 1), (0, 2), (3, 2), (1, 1), (2, 0)):
        c.set_decode_path(split=split, graph=graph)
    for split, graph in ((0, 3), (0, -1), (4, 1), (-1, 0)):
        with pytest.raises(_lib.MoeError, match="must be"):
            c.set_decode_path(split=split, graph=graph)
    # the fused launch's wait bound: (0, 60] seconds
    for sec in (1e-7, 0.5, 60.0):
        c.set_wait_bound(sec)
    for sec in (0.0, -1.0, 61.0, float("nan")):
        with pytest.raises(_lib.MoeError, match="must be in"):
            c.set_wait_bound(sec)
    c.close()


# ---- MOEP predictor / evictor hooks (patches/0006:295-427, 765-922; 0007:149-168, 330-355, 655-724) ----
HOOKS = [
    dict(pred=True),
    dict(pred=True, online_lr=0.05),
    dict(pred=True, online_lr=0.02, probation=True),
    dict(evict=True),
    dict(evict=True, early_issue=True),
    dict(pred=True, evict=True, online_lr=0.03, probation=True),
    dict(pred=True, evict=True, admit="heat", admit_half=16, admit_floor=0.5),
    dict(pred=True, evict=True, admit="window", predict_top=5),
]


def hooked_pair(tmp_path, slots, hooks, L, E=128):
    from moe_prefetch.moep import MoePredictor
    pp, ep = str(tmp_path / "pred.bin"), str(tmp_path / "evict.bin")
    write_moep(pp, E, L, list(range(L - 1)), blocks=(1, 2), seed=5)
    write_moep(ep, E, L, list(range(L)), blocks=(1, 2, 3, 4), seed=6, prior=0.0)
    knobs = {k: v for k, v in hooks.items() if k not in ("pred", "evict", "online_lr", "probation", "predict_top")}
    knobs.setdefault("admit", "off")
    oc = O.Cache(slots, **knobs)
    pc = product_cache(slots, **knobs)
    models = []
    if hooks.get("pred"):
        om, pm = O.Moep(pp), MoePredictor(pp)
        oc.set_predictor(om, hooks.get("predict_top", 3), hooks.get("online_lr", 0.0))
        pc.set_predictor(pm, hooks.get("predict_top", 3), hooks.get("online_lr", 0.0))
        models += [om, pm]
    if hooks.get("evict"):
        om, pm = O.Moep(ep), MoePredictor(ep)
        oc.set_evictor(om)
        pc.set_evictor(pm)
        models += [om, pm]
    if hooks.get("probation"):
        oc.set_spec_probation(True)
        pc.set_spec_probation(True)
    return oc, pc, models


@pytest.mark.parametrize("hooks", HOOKS, ids=lambda k: ",".join(f"{a}={b}" for a, b in k.items()))
def test_predictor_and_evictor_match_oracle(hooks, tmp_path):
    L, T = 6, 200
    slots = [12, 20, 8, 16, 12, 32]
    tg = [zipf_targets(31, l, T, s=1.0, reuse=0.5) for l in range(L)]
    oc, pc, _models = hooked_pair(tmp_path, slots, hooks, L)
    for t in range(T):
        for l in range(L):
            oc.observe(l, tg[l][t])
            pc.observe(l, tg[l][t])
        oc.step()
        pc.step()
        for l in range(L):
            assert np.array_equal(oc.frame(l), pc.frame(l)), (t, l)
            assert np.array_equal(oc.table(l)[0], pc.table(l)[0])
    os_, ps = oc.stats(), pc.stats()
    for k in ("n_steps", "clock", "n_hit", "n_miss", "n_uploads", "n_scheduled", "n_published",
              "n_admit_ok", "n_admit_denied"):
        assert os_[k] == ps[k], k
    op, pp = oc.predictor_stats(), pc.predictor_stats()
    assert op == pp, (op, pp)
    if hooks.get("pred"):
        assert pp["n_spec"] > 0                                   # speculative uploads were issued
        if hooks.get("online_lr"):
            # the model lists layers 0..L-2: each token, the predictions made at
            # layers 0..L-2 for the next layer resolve where the model holds the
            # target (layers 1..L-2), when that layer is observed
            assert pp["n_updates"] == (L - 2) * T
    if hooks.get("evict"):
        # the evictor changes the placement against plain LRU on the same stream
        plain = product_cache(slots, **{k: v for k, v in hooks.items()
                                        if k in ("admit", "admit_half", "admit_floor", "early_issue")} or {"admit": "off"})
        for t in range(T):
            for l in range(L):
                plain.observe(l, tg[l][t])
            plain.step()
        assert any(not np.array_equal(plain.frame(l), pc.frame(l)) for l in range(L))


def test_hooks_refuse_models_the_cache_cannot_score(tmp_path):
    from moe_prefetch.moep import MoePredictor
    p = str(tmp_path / "e64.bin")
    write_moep(p, 64, 4, [0, 1, 2])
    c = product_cache([8, 8, 8, 8])
    m = MoePredictor(p)
    with pytest.raises(Exception, match="64 experts"):
        c.set_predictor(m, 3)
    with pytest.raises(Exception, match="64 experts"):
        c.set_evictor(m)
    c.set_predictor(None, 0)          # clearing is always allowed
    c.set_evictor(None)


@pytest.mark.skipif(not os.path.isdir("/root/reference/models"), reason="the reference's shipped models are not here")
@pytest.mark.parametrize("i", [0, 1])
def test_x3t_routes_with_shipped_models_match_oracle(i):
    """The reference's recorded route ids (48 layers, byte-priced slots) through
    the product and the oracle with its shipped evictor and online predictor."""
    from moe_prefetch.moep import MoePredictor
    slots, experts, frames, routes = x3t.load(i)
    layers = sorted(slots)
    sl = [slots[l] for l in layers]
    knobs = dict(max_inserts=2, admit="window", admit_window=8, batch_tables=True)
    oc = O.Cache(sl, **knobs)
    pc = product_cache(sl, **knobs)
    ep, pp = "/root/reference/models/evictor-real.bin", "/root/reference/models/predictor-real.bin"
    keep = [O.Moep(ep), MoePredictor(ep), O.Moep(pp), MoePredictor(pp)]
    oc.set_evictor(keep[0])
    pc.set_evictor(keep[1])
    oc.set_predictor(keep[2], 3, 0.01)
    pc.set_predictor(keep[3], 3, 0.01)
    by = collections.defaultdict(list)
    for s, il, n_ids, n_tok, pairs in routes:
        by[s].append((il, n_tok, [e for e, _ in pairs]))
    for s in range(max(frames)):
        for il, n_tok, ids in by.get(s, []):
            oc.observe(il, np.array(ids, np.int32), n_tok)
            pc.observe(il, np.array(ids, np.int32), n_tok)
        oc.step()
        pc.step()
        for l in range(len(layers)):
            assert np.array_equal(oc.frame(l), pc.frame(l)), (s, l)
    assert oc.predictor_stats() == pc.predictor_stats()
    assert pc.predictor_stats()["n_updates"] > 1000


def test_sidecar_batch_share_arguments():
    # the batched decode's host share: 0/0 falls back to the single-token
    # share, anything else needs 0 <= num <= den, den >= 1
    c = product_cache([8, 8])
    c.set_sidecar_batch((2, 3))
    c.set_sidecar_batch(None)
    c.set_sidecar_batch((0, 1))
    for bad in ((3, 2), (1, 0), (-1, 2)):
        with pytest.raises(Exception):
            c.set_sidecar_batch(bad)
