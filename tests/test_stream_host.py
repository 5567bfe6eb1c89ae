"""Just-in-time streaming in the slot state machine (patches/0010-team-and-streaming.patch:
take 1466-1530, account 1183-1210, adopt 1722-1760, map frame one step late
1096-1129, pool target / upload skip / observe skip 1135-1175), driven step by
step on the product's host-only cache and on the oracle with the same script:
every frame, table, counter, map record and route trace must agree.  Then the
reference's own exactness test for streaming (J5 in
docs/STREAMING-IMPLEMENTATION.md) restated on the host: replaying the map
recorded with streaming, without streaming, gives back the streamed run's route
trace -- every routed expert read from the same slot -- and adoption is
checked against its rules directly."""
import numpy as np
import pytest

from moe_prefetch import MoeCache
from moe_prefetch.workload import zipf_targets
from oracle import oracle as O

E, K = 128, 8
EB = 2654208                    # bytes of one Q4_K expert at H 2048, I 768
CHUNK = 512 * 1024


class Product:
    """The product cache behind the oracle's method names."""

    def __init__(self, slots, **kw):
        self.c = MoeCache(len(slots), n_experts=E, slot_profile=list(slots), device=-1, **kw)

    def stream_enable(self, per_layer=4, reserve=2, gbps=45.7, chunk_bytes=CHUNK):
        self.c.set_streaming(True, per_layer=per_layer, reserve=reserve, top_k=8, gbps=gbps,
                             chunk_kib=chunk_bytes >> 10)

    def __getattr__(self, name):
        return getattr(self.c, name)

    def stream_stats(self):
        s = self.c.stream_stats()
        return {k: s[k] for k in O.STREAM_STATS}


def script(c, slots, T, seed, trace=None, hold_p=0.0, gbps=45.7, chunks=(0, 14), wrong=0.3):
    """Drive one cache through T tokens: per layer the table read (posted),
    the GPU's slots (resident, or a streamed job that landed before the read),
    a lookahead record for the next two layers (the true next routing mixed
    with wrong guesses), and some chunks handed to a copy engine whose last
    chunk lands at once.  Returns the per-token GPU slots."""
    rng = np.random.default_rng(seed)
    L = len(slots)
    tg = [zipf_targets(seed, l, T + 1, s=1.0, reuse=0.5) for l in range(L)]
    landed = set()
    out = []
    for t in range(T):
        gsl = []
        for l in range(L):
            now = (t * L + l) * 100000
            c.stream_posted(l)
            frame = c.frame(l)
            fr = {int(e): s for s, e in enumerate(frame) if e >= 0}
            g = []
            for e in tg[l][t]:
                e = int(e)
                if e in fr:
                    g.append(fr[e])
                    continue
                slot = slots[l]
                for (jl, je, js) in landed:
                    if jl == l and je == e:
                        slot = js
                g.append(slot)
            gsl.append(np.array(g, np.int32))
            targets = np.array([l + 1 if l + 1 < L else -1, l + 2 if l + 2 < L else -1], np.int32)
            ids = np.full((2, 8), -1, np.int32)
            n = np.zeros(2, np.int32)
            for i, T_ in enumerate(targets):
                if T_ < 0:
                    continue
                cand = [int(e) for e in tg[T_][t]]
                for j in range(len(cand)):
                    if rng.random() < wrong:
                        cand[j] = int(rng.integers(0, E))
                cand = list(dict.fromkeys(cand))[:8]
                fr_t = set(int(e) for e in c.frame(T_) if e >= 0)
                cand = [e for e in cand if e not in fr_t]
                n[i] = len(cand)
                ids[i, :len(cand)] = cand
            c.stream_take(l, targets, n, ids, now, now, EB)
            hold = int(rng.integers(l, L)) if rng.random() < hold_p else -1
            for _ in range(int(rng.integers(*chunks))):
                ch = c.stream_next(now + int(rng.integers(0, 40000)), hold)
                if ch is None:
                    break
                if ch[3]:
                    c.stream_land(ch[0])
                    landed.add(c.stream_job(ch[0]))
        for l in range(L):
            c.observe_gpu(l, tg[l][t], gsl[l])
        c.step()
        landed.clear()
        out.append(gsl)
    return out


KNOBS = [dict(admit="window", max_inserts=2), dict(admit="off", max_inserts=2), dict(admit="heat", admit_half=16)]


@pytest.mark.parametrize("knobs", KNOBS, ids=["window", "off", "heat"])
@pytest.mark.parametrize("stream", [dict(per_layer=4, reserve=2), dict(per_layer=2, reserve=0),
                                    dict(per_layer=8, reserve=4), dict(per_layer=4, reserve=2, chunk_bytes=2592 << 10)],
                         ids=["default", "tight", "wide", "whole-expert"])
def test_stream_product_equals_oracle(tmp_path, knobs, stream):
    slots = [16, 24, 12, 20]
    T = 60
    runs = []
    for kind in ("product", "oracle"):
        kw = dict(batch_tables=True, early_issue=True, **knobs)
        c = Product(slots, **kw) if kind == "product" else O.Cache(slots, **kw)
        c.stream_enable(**stream)
        rp, mp = str(tmp_path / f"{kind}.routes"), str(tmp_path / f"{kind}.map")
        c.trace_open(rp, mp)
        script(c, slots, T, seed=7, hold_p=0.3)
        frames = [list(c.frame(l)) for l in range(len(slots))]
        tables = [c.table(l)[0].tolist() for l in range(len(slots))]
        st, ss = c.stats(), c.stream_stats()
        c.close()
        runs.append((frames, tables, st, ss, open(rp).read(), open(mp).read()))
    p, o = runs
    assert p[0] == o[0] and p[1] == o[1]
    for k in ("clock", "n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied"):
        assert p[2][k] == o[2][k], k
    assert p[3] == o[3]
    assert p[3]["offered"] > 0 and p[3]["in_time"] > 0 and p[3]["landed"] > 0
    assert p[4] == o[4]
    assert p[5] == o[5]


def test_replay_of_streamed_map_gives_the_same_route_trace(tmp_path):
    # J5 on the host: the map recorded with streaming puts each token's in-time
    # experts into the frame before it, in the slots the GPU used; replayed
    # without streaming, every routed expert is read from the same slot
    slots = [16, 24, 12, 20]
    T = 80
    rec_r, rec_m = str(tmp_path / "s.routes"), str(tmp_path / "s.map")
    c = Product(slots, admit="window", batch_tables=True, early_issue=True)
    c.stream_enable()
    c.trace_open(rec_r, rec_m)
    script(c, slots, T, seed=3)
    ss = c.stream_stats()
    c.close()
    assert ss["in_time"] > 10           # otherwise the test says nothing (the reference's J5 rule)
    rep_r = str(tmp_path / "r.routes")
    for kind in ("product", "oracle"):
        r = Product(slots, admit="window", batch_tables=True) if kind == "product" else \
            O.Cache(slots, admit="window", batch_tables=True)
        r.map_replay(rec_m)
        r.trace_open(rep_r, None)
        tg = [zipf_targets(3, l, T + 1, s=1.0, reuse=0.5) for l in range(len(slots))]
        for t in range(T):
            for l in range(len(slots)):
                r.observe(l, tg[l][t])
            r.step()
        r.close()
        assert open(rep_r).read() == open(rec_r).read(), kind


def test_adoption_rules():
    # one layer, early issue, admission off: a landed expert the layer routed
    # joins with a recent use; a landed one it did not route joins as the
    # oldest (the first to go); a job whose copy never landed gives its slot back
    for mk in (lambda s, **k: Product(s, **k), lambda s, **k: O.Cache(s, **k)):
        S = 12
        c = mk([S, S, S], admit="off", batch_tables=True, early_issue=True, max_inserts=2)
        c.stream_enable(per_layer=4, reserve=2)
        for e in range(3):                                   # three residents through the demand path
            c.observe(1, np.array([e], np.int32))
            c.step()
        c.observe(1, np.array([0, 1, 2], np.int32))          # hits: their recency is above 1
        c.step()
        c.stream_posted(0)
        ids = np.full((2, 8), -1, np.int32)
        ids[0, :3] = [50, 51, 52]
        assert c.stream_take(0, np.array([1, -1], np.int32), np.array([3, 0], np.int32), ids, 0, 0, EB) == 3
        jobs = [c.stream_job(j) for j in range(3)]
        assert [j[1] for j in jobs] == [50, 51, 52] and all(j[0] == 1 for j in jobs)
        # the copy engine finishes 50 and 51 (EDF: equal deadlines go in offer order); 52 never lands
        landed = set()
        while len(landed) < 2:
            ch = c.stream_next(0, -1)
            assert ch is not None
            if ch[3]:
                c.stream_land(ch[0])
                landed.add(ch[0])
        assert landed == {0, 1}
        c.stream_posted(1)
        slot50 = jobs[0][2]
        # layer 1 routes 50 (in time: the GPU read its streamed slot) and 52 (missed)
        c.observe_gpu(1, np.array([50, 52], np.int32), np.array([slot50, S], np.int32))
        c.step()
        f = list(c.frame(1))
        assert f[slot50] == 50 and f[jobs[1][2]] == 51 and 52 not in f and f[jobs[2][2]] == -1
        ss = c.stream_stats()
        # 52 had a job and was routed, but the GPU read the dummy: late
        assert (ss["offered"], ss["landed"], ss["in_time"], ss["late"], ss["unused"]) == (3, 2, 1, 1, 1)
        # 51 (landed, never routed) is the least recently used resident: the
        # layer's next eviction takes it before 0, 1, 2 and 50
        resident = {0, 1, 2, 50, 51}
        new = iter(range(70, 128))
        first = None
        for _ in range(20):
            c.observe(1, np.array([next(new), next(new)], np.int32))
            c.step()
            gone = resident - set(int(v) for v in c.frame(1))
            if gone:
                first = gone
                break
        assert first == {51}
        c.close()


def test_streamed_expert_is_not_uploaded_again_and_not_counted_twice():
    # while an expert streams in, the demand path neither uploads it nor counts
    # its miss; the GPU's view decides (here: late, so one miss)
    for mk in (lambda s, **k: Product(s, **k), lambda s, **k: O.Cache(s, **k)):
        c = mk([8, 8], admit="off", batch_tables=True, early_issue=True)
        c.stream_enable(per_layer=4, reserve=2)
        ids = np.full((2, 8), -1, np.int32)
        ids[0, 0] = 9
        c.stream_posted(0)
        assert c.stream_take(0, np.array([1, -1], np.int32), np.array([1, 0], np.int32), ids, 0, 0, EB) == 1
        c.stream_posted(1)
        c.observe_gpu(1, np.array([9], np.int32), np.array([8], np.int32))     # the GPU missed it
        st = c.stats()
        assert st["n_miss"] == 1 and st["n_scheduled"] == 0                    # no upload of 9
        assert c.stream_stats()["late"] == 1
        c.step()
        assert 9 not in list(c.frame(1))                                        # never landed
        c.close()


def test_stream_needs_early_issue_and_no_replay():
    with pytest.raises(Exception):
        Product([8], admit="off").stream_enable()
    with pytest.raises(Exception):
        O.Cache([8], admit="off").stream_enable()
    c = Product([8], admit="off", early_issue=True, deterministic=True)
    with pytest.raises(Exception):
        c.stream_enable()
