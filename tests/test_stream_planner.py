"""The just-in-time copy planner (moe_planner, patches/0010-team-and-streaming.patch:777-909):
the product's (exported through the C ABI) and the oracle's, each held to the
reference's own planner cases (cpp/test-moe-planner.cpp, restated below with
its constants), to brute-force checks of earliest-deadline-first order, and to
each other on random operation sequences."""
import numpy as np
import pytest

from moe_prefetch import stream as S
from oracle import oracle as O

EXPERT = 2831155          # ~2.7 MiB, the three slices of one Qwen3-30B expert (test-moe-planner.cpp:10)
FAST = 1e9                # bytes per ns: nothing is ever late
PCIE = 45.7               # 45.7 GB/s
CHUNK = 512 * 1024


def planners():
    return [("product", S.Planner), ("oracle", O.Planner)]


@pytest.fixture(params=["product", "oracle"])
def mk(request):
    return S.Planner if request.param == "product" else O.Planner


def test_dedupe_and_refresh(mk):
    p = mk(CHUNK)
    assert p.offer(5, 10, EXPERT, 1000) == 0
    assert p.offer(5, 10, EXPERT, 800) == -1          # the d = 1 refresh of a d = 2 job
    assert p.get(0)["deadline_ns"] == 800
    assert p.offer(5, 10, EXPERT, 900) == -1          # a later deadline never loosens it
    assert p.get(0)["deadline_ns"] == 800
    assert p.offer(6, 10, EXPERT, 900) == 1           # same expert, other layer: a different job
    assert p.size() == 2


def test_edf_order(mk):
    p = mk(CHUNK)
    a = p.offer(7, 1, EXPERT, 500000)
    b = p.offer(6, 2, EXPERT, 300000)
    c = p.next(0, FAST)
    assert c and c[0] == b
    while not c[3]:                                   # b runs to completion before a gets a chunk
        c = p.next(0, FAST)
        assert c and c[0] == b
    c = p.next(0, FAST)
    assert c and c[0] == a


def test_chunks(mk):
    p = mk(CHUNK)
    p.offer(3, 4, EXPERT, 1000000)
    off, n = 0, 0
    while True:
        c = p.next(0, FAST)
        if c is None:
            break
        job, offset, length, last = c
        assert job == 0 and offset == off and 0 < length <= CHUNK
        off += length
        n += 1
        assert last == (off == EXPERT)
    assert off == EXPERT and n == 6
    assert p.get(0)["sent"] == EXPERT and not p.get(0)["dropped"]


def test_drop_late(mk):
    p = mk(CHUNK)
    p.offer(3, 4, EXPERT, 10000)                      # needs ~62 us at 45.7 GB/s, has 10 us
    assert p.next(0, PCIE) is None
    j = p.get(0)
    assert j["dropped"] and j["drop"] == S.DROP_LATE
    assert p.counters()["drop_late"] == 1
    p.offer(3, 5, EXPERT, 70000)                      # a job that fits is still sent
    c = p.next(0, PCIE)
    assert c and c[0] == 1
    q = mk(CHUNK)
    q.offer(3, 5, EXPERT, 70000)
    assert q.next(20000, PCIE) is None                # the same job behind 20 us of queued copies


def test_posted(mk):
    p = mk(CHUNK)
    p.offer(9, 1, EXPERT, 1000000)
    p.offer(10, 2, EXPERT, 2000000)
    c = p.next(0, FAST)
    assert c and c[0] == 0
    p.posted(9)                                       # layer 9 has read its table: too late for job 0
    assert p.get(0)["dropped"] and p.get(0)["drop"] == S.DROP_POSTED
    assert not p.get(1)["dropped"]
    c = p.next(0, FAST)
    assert c and c[0] == 1
    assert p.offer(9, 3, EXPERT, 3000000) == -1       # nothing new for a layer that already posted
    p.posted(10)
    assert p.counters()["drop_posted"] == 2


def test_hold(mk):
    p = mk(CHUNK)
    near = p.offer(5, 1, EXPERT, 100000)
    far = p.offer(8, 2, EXPERT, 50000)
    c = p.next(0, FAST, 6)
    assert c and c[0] == near                         # the far target waits while a miss computes
    c = p.next(0, FAST, -1)
    assert c and c[0] == far                          # no hold: earliest deadline
    q = mk(CHUNK)
    q.offer(8, 2, EXPERT, 50000)
    assert q.next(0, FAST, 6) is None and not q.get(0)["dropped"]   # held, not dropped


def test_preempt_at_chunk_boundary(mk):
    p = mk(CHUNK)
    a = p.offer(20, 1, EXPERT, 1000000)
    c = p.next(0, FAST)
    assert c and c[0] == a and not c[3]
    b = p.offer(15, 2, EXPERT, 200000)
    c = p.next(0, FAST)
    assert c and c[0] == b and c[1] == 0


def test_reset(mk):
    p = mk(CHUNK)
    p.offer(1, 1, EXPERT, 1)
    p.posted(4)
    p.reset()
    assert p.size() == 0
    assert p.offer(1, 1, EXPERT, 1000) == 0
    assert p.offer(4, 1, EXPERT, 1000) == 1           # reset also forgets which layers posted


# ---- brute force ---------------------------------------------------------------------
def test_next_is_earliest_deadline_of_what_can_still_land(mk):
    """Every chunk handed out belongs to the earliest-deadline job that is
    neither finished, dropped nor held; a job is dropped exactly when its
    remaining bytes cannot land by its deadline from free_at."""
    rng = np.random.default_rng(3)
    for trial in range(30):
        p = mk(CHUNK)
        model = []                                    # [target, expert, bytes, sent, deadline, dropped]
        for step in range(60):
            op = rng.integers(0, 4)
            if op == 0:
                t, e = int(rng.integers(0, 6)), int(rng.integers(0, 5))
                nb = int(rng.integers(1, 4 * CHUNK))
                dl = int(rng.integers(0, 400000))
                p.offer(t, e, nb, dl)
                continue
            free_at = int(rng.integers(0, 100000))
            bpn = float(rng.choice([FAST, PCIE, 20.0]))
            hold = int(rng.integers(-1, 6))
            before = [p.get(i) for i in range(p.size())]
            c = p.next(free_at, bpn, hold)
            # expected: drops, then the pick
            pick, want_drop = -1, []
            for i, j in enumerate(before):
                if j["dropped"] or j["sent"] >= j["bytes"]:
                    continue
                if free_at + int((j["bytes"] - j["sent"]) / bpn) > j["deadline_ns"]:
                    want_drop.append(i)
                    continue
                if hold >= 0 and j["target"] > hold:
                    continue
                if pick < 0 or j["deadline_ns"] < before[pick]["deadline_ns"]:
                    pick = i
            for i in want_drop:
                assert p.get(i)["dropped"] and p.get(i)["drop"] == S.DROP_LATE
            if pick < 0:
                assert c is None
            else:
                assert c is not None and c[0] == pick
                j = before[pick]
                assert c[1] == j["sent"] and c[2] == min(CHUNK, j["bytes"] - j["sent"])
                assert c[3] == (c[2] == j["bytes"] - j["sent"])


def test_product_and_oracle_agree_on_random_sequences():
    rng = np.random.default_rng(11)
    for trial in range(40):
        ps, po = S.Planner(CHUNK), O.Planner(CHUNK)
        for step in range(120):
            op = int(rng.integers(0, 10))
            if op < 4:
                args = (int(rng.integers(0, 8)), int(rng.integers(0, 6)), int(rng.integers(1, 5 * CHUNK)),
                        int(rng.integers(0, 500000)))
                assert ps.offer(*args) == po.offer(*args), (trial, step, args)
            elif op < 5:
                t = int(rng.integers(0, 8))
                ps.posted(t)
                po.posted(t)
            elif op < 6 and rng.random() < 0.2:
                ps.reset()
                po.reset()
            else:
                args = (int(rng.integers(0, 200000)), float(rng.choice([FAST, PCIE, 10.0])),
                        int(rng.integers(-1, 8)))
                assert ps.next(*args) == po.next(*args), (trial, step, args)
            assert ps.size() == po.size()
        for i in range(ps.size()):
            assert ps.get(i) == po.get(i)
        assert ps.counters() == po.counters()
