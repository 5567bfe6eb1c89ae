"""Heat file (LLAMA_MOE_HEAT_FILE), freeze (LLAMA_MOE_CACHE_FREEZE) and
placement-map replay (LLAMA_MOE_MAP_REPLAY): the product's state machine
(host mode, no GPU) and the oracle against each other, against brute-force
restatements of the file formats and warm-start order, and -- for replay --
against the reference's own engine recordings: replaying an X3T placement map
with its routed ids reproduces the recorded route trace byte for byte."""
import collections
import os

import numpy as np
import pytest

import x3t
from moe_prefetch import MoeCache
from moe_prefetch.workload import zipf_targets
from oracle import oracle as O


def product_cache(slots, **kw):
    return MoeCache(len(slots), n_experts=kw.pop("n_experts", 128), slot_profile=list(slots), device=-1, **kw)


def stream(L, T, seed=5, s=1.0, reuse=0.5):
    return [zipf_targets(seed, l, T, s=s, reuse=reuse) for l in range(L)]


def run_both(caches, tg, T, L):
    for t in range(T):
        for l in range(L):
            for c in caches:
                c.observe(l, tg[l][t])
        for c in caches:
            c.step()


# ---- heat file ---------------------------------------------------------------------
def heat_text(counts, L, E):
    lines = [f"moe-heat 1 {L} {E}"]
    for l in range(L):
        for e in range(E):
            if counts[l][e]:
                lines.append(f"{l} {e} {counts[l][e]}")
    return "\n".join(lines) + "\n"


def test_heat_file_saved_every_512_steps(tmp_path):
    L, E, T = 3, 128, 1030
    slots = [16, 24, 8]
    tg = stream(L, T)
    pp, op = str(tmp_path / "p.heat"), str(tmp_path / "o.heat")
    pc = product_cache(slots, admit="window")
    oc = O.Cache(slots, admit="window")
    assert pc.heat_file(pp) == (0, 0) and oc.heat_file(op) == (0, 0)     # no file yet: cold start
    counts = [[0] * E for _ in range(L)]
    for t in range(T):
        for l in range(L):
            pc.observe(l, tg[l][t])
            oc.observe(l, tg[l][t])
            for e in tg[l][t]:
                counts[l][e] += 1
        pc.step()
        oc.step()
        if t + 1 == 512:
            want512 = heat_text(counts, L, E)
            assert open(pp).read() == want512 and open(op).read() == want512
        if t + 1 == 1024:
            want1024 = heat_text(counts, L, E)
    # the last save was at step 1024; steps 1025..1030 wrote nothing
    assert open(pp).read() == want1024 == open(op).read()
    assert not os.path.exists(pp + ".tmp")
    pc.close()
    oc.close()


def warm_expect(counts, S, reserve):
    """Brute force: halved counts, count descending then id ascending, only
    experts with a non-zero halved count, at most S - reserve of them."""
    half = [c // 2 for c in counts]
    order = sorted(range(len(counts)), key=lambda e: (-half[e], e))
    placed = [e for e in order if half[e] > 0][:max(0, S - reserve)]
    frame = [-1] * S
    for s, e in enumerate(placed):
        frame[s] = e
    return frame


@pytest.mark.parametrize("knobs", [dict(admit="window"), dict(admit="off", early_issue=True, max_inserts=3),
                                   dict(admit="heat", admit_half=16)], ids=["window", "early", "heat"])
def test_heat_warm_start(tmp_path, knobs):
    L, E = 3, 128
    slots = [16, 40, 8]
    rng = np.random.default_rng(11)
    counts = [[0] * E for _ in range(L)]
    for l in range(L):
        for e in rng.choice(E, 60, replace=False):
            counts[l][e] = int(rng.integers(1, 9))       # 1 halves to 0: never placed
        counts[l][3] = counts[l][5] = 6                  # a tie: the lower id first
    path = str(tmp_path / "warm.heat")
    open(path, "w").write(heat_text(counts, L, E))
    reserve = knobs.get("max_inserts", 2) if knobs.get("early_issue") else 0
    pc = product_cache(slots, **knobs)
    oc = O.Cache(slots, **knobs)
    n_rec = sum(1 for l in range(L) for e in range(E) if counts[l][e])
    rp, ro = pc.heat_file(path), oc.heat_file(path)
    assert rp == ro and rp[0] == n_rec
    for l in range(L):
        want = warm_expect(counts[l], slots[l], reserve)
        assert list(pc.frame(l)) == want and list(oc.frame(l)) == want, l
    assert rp[1] == sum(sum(1 for v in warm_expect(counts[l], slots[l], reserve) if v >= 0) for l in range(L))
    # then the same decode on both: frames, tables and counters stay equal
    tg = stream(L, 200, seed=3)
    for t in range(200):
        for l in range(L):
            pc.observe(l, tg[l][t])
            oc.observe(l, tg[l][t])
        pc.step()
        oc.step()
        for l in range(L):
            assert np.array_equal(pc.frame(l), oc.frame(l)), (t, l)
    ps, os_ = pc.stats(), oc.stats()
    for k in ("clock", "n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied"):
        assert ps[k] == os_[k], k
    pc.close()
    oc.close()


def test_heat_warm_set_evicted_coldest_first(tmp_path):
    # one full layer, admission off, a stream of experts never placed: each
    # step's two uploads evict the least recently used -- the coldest of the
    # warm set first (slot S-1, then S-2, ...), since the hottest was given
    # the most recent use
    E, S = 128, 12
    counts = [[0] * E]
    for i, e in enumerate(range(40, 40 + S)):
        counts[0][e] = 2 * (S - i) + 2                   # expert 40 hottest ... 40+S-1 coldest
    path = str(tmp_path / "one.heat")
    open(path, "w").write(heat_text(counts, 1, E))
    for c in (product_cache([S], admit="off"), O.Cache([S], admit="off")):
        c.heat_file(path)
        warm = list(c.frame(0))
        assert warm == list(range(40, 40 + S))
        evicted = []
        new = iter(range(60, 128))
        for t in range(4):
            ids = np.array([next(new) for _ in range(8)], np.int32)
            before = set(c.frame(0))
            c.observe(0, ids)
            c.step()
            evicted += sorted((before - set(c.frame(0))) - {-1}, reverse=True)
        # 2 uploads a step, publication a step later: the victims are the warm
        # set's coldest, in order
        assert evicted == list(range(40 + S - 1, 40 + S - 1 - len(evicted), -1)), evicted
        assert len(evicted) >= 4
        c.close()


def test_heat_file_refused_for_other_dimensions(tmp_path):
    path = str(tmp_path / "other.heat")
    open(path, "w").write("moe-heat 1 5 128\n0 3 10\n")
    pc = product_cache([8, 8], admit="off")
    oc = O.Cache([8, 8], admit="off")
    assert pc.heat_file(path) == (0, 0) and oc.heat_file(path) == (0, 0)
    assert (pc.frame(0) == -1).all() and (oc.frame(0) == -1).all()
    pc.close()
    oc.close()


def test_freeze_never_uploads():
    L, T = 2, 60
    tg = stream(L, T)
    for early in (False, True):
        pc = product_cache([8, 8], admit="off", early_issue=early)
        oc = O.Cache([8, 8], admit="off", early_issue=early)
        pc.freeze()
        oc.freeze()
        run_both([pc, oc], tg, T, L)
        for c in (pc, oc):
            st = c.stats()
            assert st["n_scheduled"] == 0 and st["n_published"] == 0 and st["n_hit"] == 0
            assert (c.frame(0) == -1).all()
            c.close()


# ---- placement-map replay ------------------------------------------------------------
@pytest.mark.parametrize("i", [0, 1, 2, 3])
def test_replay_x3t_reproduces_route_trace(i, tmp_path):
    # replaying the reference's recorded placements with its routed ids gives
    # back its route trace: every id:slot pair is the replayed placement
    slots, experts, frames, routes = x3t.load(i)
    layers = sorted(slots)
    mp = str(tmp_path / "map.txt")
    open(mp, "w").write(x3t.read_text(os.path.join(x3t.GOLDEN, f"{i}.map.txt.gz")))
    by = collections.defaultdict(list)
    for s, il, n_ids, n_tok, pairs in routes:
        by[s].append((il, n_tok, [e for e, _ in pairs]))
    outs = []
    for kind in ("product", "oracle"):
        c = product_cache([slots[l] for l in layers], admit="window", batch_tables=True) if kind == "product" \
            else O.Cache([slots[l] for l in layers], admit="window", batch_tables=True)
        c.map_replay(mp)
        rp = str(tmp_path / f"{kind}.routes")
        c.trace_open(rp, None)
        for s in range(max(frames)):
            for il, n_tok, ids in by.get(s, []):
                c.observe(il, np.array(ids, np.int32), n_tok)
            c.step()
            if s + 1 in frames:
                for l in layers:
                    assert list(c.frame(l)) == frames[s + 1][l], (kind, s, l)
        assert c.stats()["n_scheduled"] == 0
        c.close()
        outs.append(open(rp).read())
    want = x3t.read_text(os.path.join(x3t.GOLDEN, f"{i}.routes-record.txt.gz"))
    assert outs[0] == want and outs[1] == want


def test_replay_own_recording_with_other_routing(tmp_path):
    # record a run, replay it under different routing: the placement follows
    # the recording step by step, and a hit is exactly membership in it
    L, T = 3, 80
    slots = [12, 20, 8]
    rec = str(tmp_path / "rec.map")
    pc = product_cache(slots, admit="window", batch_tables=True)
    pc.trace_open(None, rec)
    tga = stream(L, T, seed=1)
    for t in range(T):
        for l in range(L):
            pc.observe(l, tga[l][t])
        pc.step()
    pc.close()
    _, _, frames = x3t.parse_map(open(rec).read())
    tgb = stream(L, T, seed=2, s=0.8)
    want_hits = sum(int(np.isin(tgb[l][t], frames[t][l]).sum()) for t in range(T) for l in range(L))
    for c in (product_cache(slots, admit="window", batch_tables=True),
              O.Cache(slots, admit="window", batch_tables=True)):
        c.map_replay(rec)
        for t in range(T):
            for l in range(L):
                assert list(c.frame(l)) == frames[t][l], (t, l)
                c.observe(l, tgb[l][t])
            c.step()
        st = c.stats()
        assert st["n_hit"] == want_hits and st["n_scheduled"] == 0
        c.close()


def test_replay_rejects_bad_maps(tmp_path):
    p = str(tmp_path / "bad.map")
    open(p, "w").write("moe-map 1 2\nlayer 0 8 128\nlayer 1 9 128\nstep 0\n")
    with pytest.raises(Exception):
        product_cache([8, 8], admit="off").map_replay(p)           # slot counts differ
    open(p, "w").write("moe-map 1 1\nlayer 0 4 128\nstep 0\nmap 0 1 2 3 -1\n")
    c = product_cache([4], admit="off")
    c.map_replay(p)
    assert list(c.frame(0)) == [1, 2, 3, -1]
    c.observe(0, np.arange(8, dtype=np.int32))
    with pytest.raises(Exception):
        c.step()                                                   # no frame for step 1
    c.close()
