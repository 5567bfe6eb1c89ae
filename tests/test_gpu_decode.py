"""GPU parity of the whole decode step (MoeCache.decode_token: router, slot
lookup, experts from HBM slots or the pinned store, combine, routed ids back,
observe, step, uploads on the side stream, table flush) against the oracle run
on the same inputs: every routed id and every placement frame bit-exact, every
traced route line identical, layer outputs bit for bit (every decode path:
one launch, or resident and absent experts as two launches whose second adds
the rows in k order).  With the
cache prior the routing depends on the published tables, so ids agreeing
token after token also checks publication timing end to end."""
import os

import numpy as np
import pytest
import torch

from gpu_rig import L, Rig, stream
from moe_prefetch import ExpertCache, _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu
Q4, Q6 = _lib.TYPE_Q4K, _lib.TYPE_Q6K


def check_run(rig, tmp_path, out_every=1, tol=1e-3, oc=None, record_map=True, tokens=None):
    """Decode `tokens` (default: all of the rig's) and compare with the oracle
    token by token.  Leaves the product's and the oracle's counters and the
    number of evictions seen in the frames (a slot whose expert was replaced)
    on the rig as stats, ostats and n_evicted."""
    rp, mp = str(tmp_path / "gpu.routes"), str(tmp_path / "gpu.map") if record_map else None
    orp, omp = str(tmp_path / "ora.routes"), str(tmp_path / "ora.map") if record_map else None
    rig.cache.trace_open(rp, mp)
    oc = rig.oracle_cache() if oc is None else oc
    oc.trace_open(orp, omp)
    tokens = list(range(rig.T)) if tokens is None else list(tokens)
    keep = set(tokens[::out_every]) | {tokens[-1]}
    ids_all, outs, frames = rig.run(tokens=tokens, keep_out=keep)
    worst = 0.0
    prev = [oc.frame(l) for l in range(rig.nl)]
    rig.n_evicted = 0
    for t in tokens:
        for l in range(rig.nl):
            tbl, prior = oc.table(l)
            use_prior = prior if rig.knobs.get("cache_prior", 0.0) > 0 else None
            bias = None if rig.bh is None else rig.bh[t, l]
            rids, rw, _, _ = O.route(rig.Wh[l], rig.xh[t, l], 8, bias=bias, prior=use_prior, table=tbl,
                                     prior_on_logits=rig.prior_on_logits())
            assert np.array_equal(ids_all[t][l], rids), (t, l, ids_all[t][l], rids)
            if t in keep:
                want = rig.oracle_layer(t, l, rids, rw)
                r = float(np.linalg.norm(outs[t][l].astype(np.float64) - want) / np.linalg.norm(want))
                worst = max(worst, r)
                assert r < tol, (t, l, r)
                assert np.array_equal(outs[t][l], want), (t, l, r)    # every decode path: bit for bit
            oc.observe(l, rids)
        oc.step()
        for l in range(rig.nl):
            f = oc.frame(l)
            assert np.array_equal(frames[t][l], f), (t, l)
            rig.n_evicted += int(np.sum((prev[l] >= 0) & (f != prev[l])))
            prev[l] = f
    rig.stats, rig.ostats = rig.cache.stats(), oc.stats()
    rig.pstats, rig.opstats = rig.cache.predictor_stats(), oc.predictor_stats()
    rig.cache.close()
    oc.close()
    assert open(rp).read() == open(orp).read()
    if record_map:
        assert open(mp).read() == open(omp).read()
    return worst


@pytest.mark.parametrize("split,graph", [(1, 2), (0, 2), (2, 2), (3, 2), (1, 0), (0, 0), (2, 0), (3, 0), (0, 1)],
                         ids=["fork-graph", "fused-graph", "serial-graph", "unfused-graph", "fork-eager",
                              "fused-eager", "serial-eager", "unfused-eager", "fused-direct"])
def test_decode_4_layers_window_admission(tmp_path, split, graph):
    # every decode path (the fused front with one expert launch; router,
    # selection and experts as four launches; resident/absent experts split
    # over two streams or one after the other; captured graph replayed per
    # token (graph 2: kept for 4 layers) or eager launches; graph 1 launches
    # a token this short directly) must give the oracle's ids, frames and
    # outputs; the graph is replayed 40 times with eager copies, host work and
    # synchronisation between replays
    rig = Rig([16, 24, 12, 40], [Q4, Q6, Q4, Q6], T=40, admit="window", batch_tables=True)
    rig.cache.set_decode_path(split=split, graph=graph)
    if split and not graph:
        rig.cache.set_timing(True)          # per-kernel events around every launch
    try:
        worst = check_run(rig, tmp_path)
        print("worst rel-L2", worst)
    finally:
        rig.close()


@pytest.mark.parametrize("graph", [0, 2], ids=["direct", "graph"])
def test_fused_wait_bound_reports_and_recovers(graph):
    """The fused launch's bounded waits, forced from the host: with the bound
    at 0.1 us the workgroups that wait give up and exit (every kernel ends
    normally), and the token fails with MOE_ERR_HIP naming the wait -- launched
    directly (the published late word, or no done word and the bounded spin's
    fallback to the copy back and synchronisation) and as a graph.  The failed
    token observed and stepped nothing; with the bound restored the next tokens
    decode as the oracle's (ids and outputs bit for bit)."""
    rig = Rig([16, 24], [Q4, Q6], T=4, admit="window", batch_tables=True)
    rig.cache.set_decode_path(split=0, graph=graph)
    oc = rig.oracle_cache()
    out = torch.empty((rig.nl, rig.x.shape[-1]), dtype=torch.float32, device=rig.dev)
    bias = lambda t: None if rig.bias is None else rig.bias[t]
    try:
        rig.cache.set_wait_bound(1e-7)
        with pytest.raises(_lib.MoeError, match="gave up waiting"):
            rig.cache.decode_token(rig.x[0], out, bias=bias(0), stream=stream())
        rig.cache.set_wait_bound(0.5)
        for t in (1, 2, 3):
            ids = rig.cache.decode_token(rig.x[t], out, bias=bias(t), stream=stream())
            torch.cuda.synchronize()
            got = out.cpu().numpy()
            for l in range(rig.nl):
                tbl, _ = oc.table(l)
                b = None if rig.bh is None else rig.bh[t, l]
                rids, rw, _, _ = O.route(rig.Wh[l], rig.xh[t, l], 8, bias=b, table=tbl)
                assert np.array_equal(ids[l], rids), (t, l, ids[l], rids)
                assert np.array_equal(got[l], rig.oracle_layer(t, l, rids, rw)), (t, l)
                oc.observe(l, rids)
            oc.step()
    finally:
        oc.close()
        rig.close()


def test_layer_op_wait_bound_reports_and_recovers():
    """The per-layer op with the fused launch's waits forced to give up (the
    bound at 0.1 us, set from the host; every kernel exits normally): the step
    after the token's layers reports MOE_ERR_HIP naming the wait.  With the bound
    restored the next tokens decode layer by layer with ids and outputs equal
    to the oracle's (no cache prior, so the routing does not depend on what
    the failed token observed)."""
    rig = Rig([16, 24], [Q4, Q6], T=3, admit="window", batch_tables=True)
    c = rig.cache
    c.set_decode_path(split=0, graph=0)
    ids_dev = torch.empty((rig.nl, 8), dtype=torch.int32, device=rig.dev)
    outs = torch.empty((rig.nl, rig.x.shape[-1]), dtype=torch.float32, device=rig.dev)

    def token(t):
        for l in range(rig.nl):
            c.decode_layer(l, rig.x[t, l], outs[l], bias=None if rig.bias is None else rig.bias[t, l],
                           ids=ids_dev[l], stream=stream())
        ids = ids_dev.cpu().numpy()
        for l in range(rig.nl):
            c.observe(l, ids[l])
        c.step()
        return ids

    try:
        c.set_wait_bound(1e-7)
        with pytest.raises(_lib.MoeError, match="gave up waiting"):
            token(0)
        c.set_wait_bound(0.5)
        for t in (1, 2):
            ids = token(t)
            torch.cuda.synchronize()
            got = outs.cpu().numpy()
            for l in range(rig.nl):
                b = None if rig.bh is None else rig.bh[t, l]
                rids, rw, _, _ = O.route(rig.Wh[l], rig.xh[t, l], 8, bias=b)
                assert np.array_equal(ids[l], rids), (t, l, ids[l], rids)
                assert np.array_equal(got[l], rig.oracle_layer(t, l, rids, rw)), (t, l)
    finally:
        rig.close()


@pytest.mark.parametrize("E,I,graph", [(64, 256, 2), (192, 512, 0)], ids=["e64_i256_graph", "e192_i512_eager"])
def test_decode_fused_chunk_counts(tmp_path, E, I, graph):
    # the fused layer routes in registers per 64-expert chunk (1 to 4 chunks:
    # one instantiation each); E = 64 and E = 192, with the cache prior on so
    # the routing reads the published tables every token
    rig = Rig([24, 40], [Q4, Q6], T=32, I=I, E=E, admit="window", batch_tables=True, cache_prior=0.01)
    rig.cache.set_decode_path(split=0, graph=graph)
    try:
        worst = check_run(rig, tmp_path)
        print("worst rel-L2", worst)
    finally:
        rig.close()


def test_decode_256_experts_shared_expert(tmp_path):
    # the wide variant: 256 routed experts (top-8) plus an always-on shared
    # expert, I = 512, cache prior 0.01, Zipf(1.0) popularity with reuse 0.5
    rig = Rig([40, 24], [Q4, Q6], T=40, I=512, E=256, shared=True, zipf_s=1.0, reuse=0.5, admit="window",
              batch_tables=True, cache_prior=0.01)
    try:
        worst = check_run(rig, tmp_path)
        print("worst rel-L2", worst)
    finally:
        rig.close()


@pytest.mark.parametrize("shape", ["e256_shared_i512", "e128_i768", "e128_unsteered_prior", "e256_shared_i512_cpu",
                                   "e128_i768_cpu_2of3", "e128_i768_cpu_1of2_b5", "e128_i768_cpu_0of1",
                                   "e128_i768_cpu_1of1_b80_timed"])
def test_decode_batch_matches_oracle(shape):
    # moe_decode_batch: batches of 16 tokens through every layer (route -- the
    # cache prior biases single-token selection only, so it is off here --,
    # dispatch, grouped experts from slots or the pinned store, the shared
    # expert), observed token-major and stepped: ids, frames and counters equal
    # to the oracle's, outputs bit for bit.  *_cpu: CPU-assisted serving, the
    # host computing the pairs of (a share of) the absent experts
    # (b5: batches of 5 tokens; 0of1: CPU-assisted serving on, the host's share empty;
    # b80: batches above 64 tokens run on the GPU alone with serving on, timed per kernel)
    share = {"e256_shared_i512_cpu": (1, 1), "e128_i768_cpu_2of3": (2, 3), "e128_i768_cpu_1of2_b5": (1, 2),
             "e128_i768_cpu_0of1": (0, 1), "e128_i768_cpu_1of1_b80_timed": (1, 1)}.get(shape)
    B = 5 if shape.endswith("_b5") else 80 if "_b80" in shape else 16
    timed = shape.endswith("_timed")
    shape = shape.split("_cpu")[0]
    nb = 2 if B > 16 else 4
    T = max(64, B * nb)
    if shape == "e256_shared_i512":
        rig = Rig([48, 32], [Q4, Q6], T=T, I=512, E=256, shared=True, zipf_s=1.0, reuse=0.5, admit="window",
                  batch_tables=True, cache_prior=0.01)
    elif shape == "e128_i768":
        rig = Rig([20, 28], [Q6, Q4], T=T, I=768, admit="window", batch_tables=True)
    else:   # W x alone: a 0.01 prior on probabilities near 1/128 would change the ids
        rig = Rig([24, 24], [Q4, Q6], T=T, steer=False, admit="window", batch_tables=True, cache_prior=0.01)
    oc = rig.oracle_cache()
    if share:
        rig.cache.set_sidecar(4, share)
    if timed:
        rig.cache.set_timing(True)
    try:
        out = torch.empty((rig.nl, B, 2048), dtype=torch.float32, device=rig.dev)
        for b in range(nb):
            toks = range(B * b, B * (b + 1))
            xb = rig.x[B * b:B * (b + 1)].transpose(0, 1).contiguous()
            bb = None if rig.bias is None else rig.bias[B * b:B * (b + 1)].transpose(0, 1).contiguous()
            ids = rig.cache.decode_batch(xb, out, bias=bb, stream=torch.cuda.current_stream().cuda_stream)
            got = out.cpu().numpy()
            for l in range(rig.nl):
                tbl, prior = oc.table(l)
                use_prior = prior if rig.knobs.get("cache_prior", 0.0) > 0 and B == 1 else None
                want_ids = []
                for j, t in enumerate(toks):
                    bias = None if rig.bh is None else rig.bh[t, l]
                    rids, rw, _, _ = O.route(rig.Wh[l], rig.xh[t, l], 8, bias=bias, prior=use_prior, table=tbl)
                    assert np.array_equal(ids[l, j], rids), (b, l, j)
                    want = rig.oracle_layer(t, l, rids, rw)
                    assert np.array_equal(got[l, j], want), (b, l, j, float(np.abs(got[l, j] - want).max()))
                    want_ids.append(rids)
                oc.observe(l, np.stack(want_ids), n_tok=B)
            oc.step()
            for l in range(rig.nl):
                assert np.array_equal(rig.cache.frame(l), oc.frame(l)), (b, l)
        st, ost = rig.cache.stats(), oc.stats()
        for k in ("n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied"):
            assert st[k] == ost[k], (k, st[k], ost[k])
        if share:
            # the host computed pairs (none at 0/1, nor in batches above 64 tokens)
            assert (st["n_cpu_served"] > 0) == (share[0] > 0 and B <= 64)
        if timed:
            kt = rig.cache.kernel_times()
            assert kt["grouped_launches"] == nb * rig.nl and kt["grouped_gateup_ms"] > 0 and kt["grouped_down_ms"] > 0
            assert kt["grouped_pairs"] == nb * B * 8 * rig.nl          # every pair on the GPU
            assert kt["grouped_gateup_hbm_bytes"] + kt["grouped_gateup_host_bytes"] > 0
    finally:
        oc.close()
        rig.close()


def test_decode_cache_prior_delta(tmp_path):
    # no steering: routing is W x alone, and the 0.01 prior on resident
    # experts' probabilities changes the selection
    rig = Rig([24, 24], [Q4, Q6], T=48, steer=False, admit="window", cache_prior=0.01)
    try:
        check_run(rig, tmp_path)
    finally:
        rig.close()


@pytest.mark.parametrize("graph", [2, 0], ids=["graph", "eager"])
def test_decode_cache_prior_on_logits_fused(tmp_path, graph):
    # the logits-space variant of the cache prior (delta added to resident
    # experts' logits before the top-k, gate weights from the unbiased
    # softmax) on the default fused launch, which routes the token inside
    # every gate/up wave; no steering, so the prior changes the selection
    rig = Rig([24, 24, 16], [Q4, Q6, Q4], T=48, steer=False, admit="window", batch_tables=True, cache_prior=0.01,
              prior_space="logits")
    rig.cache.set_decode_path(split=0, graph=graph)
    try:
        check_run(rig, tmp_path)
    finally:
        rig.close()


@pytest.mark.parametrize("knobs", [dict(admit="off"), dict(admit="heat", admit_half=8),
                                   dict(admit="off", early_issue=True), dict(admit="window", deterministic=True)],
                         ids=["off", "heat", "early", "sorted"])
def test_decode_knobs(tmp_path, knobs):
    rig = Rig([8, 16], [Q6, Q4], T=24, I=512, zipf_s=1.0, reuse=0.5, **knobs)
    try:
        check_run(rig, tmp_path, out_every=3)
    finally:
        rig.close()


@pytest.mark.parametrize("knobs", [dict(admit="window", batch_tables=True),
                                   dict(admit="off", early_issue=True, max_inserts=3)], ids=["window", "early"])
def test_staged_uploads_fill_slots(knobs):
    # uploads of experts the token read from the pinned store are copied from
    # the HBM staging area: afterwards every occupied slot holds its expert's
    # bytes, and ids, frames, outputs and counters equal a run with staging off
    T = 40
    runs = {}
    for staging in (True, False):
        rig = Rig([12, 20, 16], [Q4, Q6, Q4], T=T, **knobs)
        rig.cache.set_staging(staging)
        rig.cache.set_upload_stats(True)
        try:
            ids, outs, frames = rig.run()
            rig.cache.sync()
            st = rig.cache.stats()
            # every finished upload timed on its stream, by source (LLAMA_MOE_UPLOAD_STATS)
            assert st["n_upload_h2d"] + st["n_upload_d2d"] == st["n_copied"] > 0
            assert st["n_upload_d2d"] <= st["n_staged"] and (st["n_upload_d2d"] > 0) == staging
            assert st["upload_d2d_us"] > 0 if staging else st["upload_d2d_us"] == 0
            if st["n_upload_h2d"]:
                assert st["upload_h2d_us"] > 0
            for l in range(rig.nl):
                v = rig.cache.lookup(l)
                eb = rig.eb[l]
                back = np.empty(eb, np.uint8)
                for s, e in enumerate(rig.cache.frame(l)):
                    if e < 0:
                        continue
                    assert L().moe_memcpy(back.ctypes.data, v.slot_pool + s * v.slot_bytes, eb) == 0
                    assert np.array_equal(back, rig.stores[l].arr[e * eb:(e + 1) * eb]), (staging, l, s, e)
            runs[staging] = (ids, outs, frames, st)
        finally:
            rig.close()
    on, off = runs[True], runs[False]
    assert on[3]["n_scheduled"] > 0
    assert on[3]["n_staged"] == on[3]["n_scheduled"]      # every upload was of an expert the token read
    assert off[3]["n_staged"] == 0
    for t in range(T):
        assert np.array_equal(on[0][t], off[0][t]) and np.array_equal(on[1][t], off[1][t]), t
        for l in range(3):
            assert np.array_equal(on[2][t][l], off[2][t][l]), (t, l)
    for k in ("n_hit", "n_miss", "n_scheduled", "n_published", "bytes_uploaded"):
        assert on[3][k] == off[3][k], k


@pytest.mark.parametrize("case", ["all-graph", "two-thirds-graph", "all-eager", "e256-shared", "e64-prior",
                                  "e192-prior"])
def test_sidecar_decode_matches_oracle(tmp_path, case):
    # CPU-assisted serving: the fused launch posts each logit and Q8_K(x) to
    # mapped host memory, the host routes the token from them and computes the
    # absent experts assigned to it, the join kernel combines in k order --
    # ids, frames, traces and outputs bit for bit as the oracle's.  e64 / e192:
    # one and three 64-expert chunks in the host's routing, with the cache
    # prior on the probabilities
    if case == "e256-shared":
        rig = Rig([40, 24], [Q4, Q6], T=32, I=512, E=256, shared=True, zipf_s=1.0, reuse=0.5, admit="window",
                  batch_tables=True, cache_prior=0.01)
    elif case == "e64-prior":
        rig = Rig([16, 24], [Q4, Q6], T=32, I=256, E=64, admit="window", batch_tables=True, cache_prior=0.01)
    elif case == "e192-prior":
        rig = Rig([24, 40], [Q6, Q4], T=32, I=512, E=192, admit="window", batch_tables=True, cache_prior=0.01)
    else:
        rig = Rig([16, 24, 12, 40], [Q4, Q6, Q4, Q6], T=40, admit="window", batch_tables=True)
    share = (2, 3) if case == "two-thirds-graph" else (1, 1)
    rig.cache.set_decode_path(split=0, graph=case != "all-eager")
    rig.cache.set_sidecar(6, share)
    try:
        check_run(rig, tmp_path)
    finally:
        rig.close()


def test_sidecar_counts_cpu_served():
    rig = Rig([16, 24], [Q4, Q6], T=24, admit="window", batch_tables=True)
    try:
        rig.cache.set_sidecar(4)
        ids_on, outs_on, _ = rig.run()
        st = rig.cache.stats()
        assert st["n_cpu_served"] == st["n_miss"] > 0       # every absent expert went to the CPU
        assert st["n_staged"] == 0                          # none was read by the kernels
        with pytest.raises(_lib.MoeError):
            rig.cache.set_decode_path(split=1)              # the split paths need the sidecar off
        rig.cache.set_sidecar(0)
        rig.cache.set_decode_path(split=1)
    finally:
        rig.close()


def test_heat_warm_start_and_map_replay_on_gpu(tmp_path):
    # a heat file places the hottest experts' bytes in their slots before the
    # first token; the decode that follows matches an oracle warm-started from
    # the same file.  Its recorded placement map, replayed on a fresh cache,
    # puts the same experts in the same slots step by step (bytes copied from
    # the store), and the decode under replay matches the oracle's replay.
    E = 128
    rng = np.random.default_rng(21)
    heat = tmp_path / "warm.heat"
    lines = [f"moe-heat 1 2 {E}"]
    for l in range(2):
        for e in sorted(rng.choice(E, 50, replace=False)):
            lines.append(f"{l} {e} {int(rng.integers(1, 30))}")
    heat.write_text("\n".join(lines) + "\n")
    slots = [16, 24]
    rig = Rig(slots, [Q4, Q6], T=24, admit="window", batch_tables=True)
    try:
        n_rec, n_placed = rig.cache.heat_file(str(heat))
        assert n_rec == 100 and n_placed > 0
        for l in range(2):
            v, eb = rig.cache.lookup(l), rig.eb[l]
            back = np.empty(eb, np.uint8)
            for s, e in enumerate(rig.cache.frame(l)):
                if e >= 0:
                    assert L().moe_memcpy(back.ctypes.data, v.slot_pool + s * v.slot_bytes, eb) == 0
                    assert np.array_equal(back, rig.stores[l].arr[e * eb:(e + 1) * eb]), (l, s, e)
        oc = rig.oracle_cache()
        assert oc.heat_file(str(heat)) == (n_rec, n_placed)
        check_run(rig, tmp_path, oc=oc)
    finally:
        rig.close()
    rec = str(tmp_path / "gpu.map")
    rig2 = Rig(slots, [Q4, Q6], T=24, admit="window", batch_tables=True)
    try:
        rig2.cache.map_replay(rec)
        assert rig2.cache.requires_sync()          # replay overwrites slots: sync before the step
        oc2 = rig2.oracle_cache()
        oc2.map_replay(rec)
        check_run(rig2, tmp_path, oc=oc2, record_map=False)
    finally:
        rig2.close()


def test_decode_48_layers_full_shape(tmp_path):
    """The stacked Qwen3-30B-A3B shape at full size (48 layers, 56 slots, Q6_K
    down in odd layers, pinned store of all 128 experts per layer), for the
    first tokens of the decode: ids and frames bit-exact, outputs sampled."""
    rig = Rig([56] * 48, [Q6 if l % 2 else Q4 for l in range(48)], T=12, admit="window", batch_tables=True)
    try:
        check_run(rig, tmp_path, out_every=6)
    finally:
        rig.close()


def test_decode_48_layers_past_cache_fill(tmp_path):
    """The stacked shape through the cache fill and into eviction: with at
    most 2 uploads per layer per token a 56-slot layer cannot fill before
    token 28, and the first LRU victims come near token 40.  64 tokens: ids,
    frames, route and map traces bit-exact at every token, outputs sampled,
    and the run must have evicted and denied admission (P6:785-841,
    P7:398-429) with the oracle's counters."""
    rig = Rig([56] * 48, [Q6 if l % 2 else Q4 for l in range(48)], T=64, admit="window", batch_tables=True)
    try:
        check_run(rig, tmp_path, out_every=16)
    finally:
        rig.close()
    st, ost = rig.stats, rig.ostats
    for k in ("n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied", "n_table_flushes"):
        assert st[k] == ost[k], (k, st[k], ost[k])
    print("evicted", rig.n_evicted, "denied", st["n_admit_denied"], "hit", st["n_hit"] / (st["n_hit"] + st["n_miss"]))
    assert rig.n_evicted > 100 and st["n_admit_denied"] > 100
    assert st["n_evicted"] == rig.n_evicted          # the step's count equals the evictions the frames show


def test_sidecar_host_abort_then_next_token_exact(tmp_path):
    """The host gives up on a token (here: layer 1 has no router, so the
    decode fails after layer 0's kernels, its join included, were launched):
    the host writes SC_ABORT, layer 0's join ends its bounded wait, the call
    returns an error, and every kernel has exited.  The next tokens decode
    bit-exact against an oracle that never saw the failed token: the stale
    SC_ABORT must not end their joins early (P9:322-359; the reference forces
    the same case with a dead host, cpp/test-moe-sidecar.cpp:150)."""
    rig = Rig([16, 24], [Q4, Q6], T=10, admit="window", batch_tables=True, skip_router={1})
    rig.cache.set_decode_path(split=0, graph=False)
    rig.cache.set_sidecar(4)
    out = torch.empty((rig.nl, 2048), dtype=torch.float32, device=rig.dev)
    with pytest.raises(_lib.MoeError, match="router"):
        rig.cache.decode_token(rig.x[0], out, bias=rig.bias[0], stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rig.cache.stats()["n_steps"] == 0            # the failed token observed and stepped nothing
    rig.cache.set_router(1, rig.W[1])
    try:
        check_run(rig, tmp_path, tokens=range(1, rig.T))
    finally:
        rig.close()
    assert rig.stats["n_cpu_served"] > 0


def test_decode_with_predictor_and_evictor(tmp_path):
    """The MOEP hooks on the GPU decode (patches/0006:295-427, 765-922;
    0007:149-168, 330-355, 655-724): an online-learning predictor issuing
    speculative next-layer uploads on probation, and an evictor choosing the
    victims; ids, frames, traces and outputs equal the oracle's token by token,
    and so do the predictor's resolved predictions, recall and speculative
    uploads."""
    from moep_models import write_moep
    from moe_prefetch.moep import MoePredictor
    pp, ep = str(tmp_path / "pred.bin"), str(tmp_path / "evict.bin")
    write_moep(pp, 128, 4, [0, 1, 2], blocks=(1, 2), seed=5)
    write_moep(ep, 128, 4, [0, 1, 2, 3], blocks=(1, 2, 3, 4), seed=6, prior=0.0)
    rig = Rig([16, 24, 12, 40], [Q4, Q6, Q4, Q6], T=48, admit="window", batch_tables=True)
    models = [MoePredictor(pp), MoePredictor(ep), O.Moep(pp), O.Moep(ep)]
    try:
        rig.cache.set_predictor(models[0], 3, 0.02)
        rig.cache.set_evictor(models[1])
        rig.cache.set_spec_probation(True)
        oc = rig.oracle_cache()
        oc.set_predictor(models[2], 3, 0.02)
        oc.set_evictor(models[3])
        oc.set_spec_probation(True)
        check_run(rig, tmp_path, oc=oc)
        assert rig.pstats == rig.opstats, (rig.pstats, rig.opstats)
        # predictions for layers 1..3; one resolves where the model holds the
        # target layer (1 and 2), every token
        assert rig.pstats["n_spec"] > 0 and rig.pstats["n_updates"] == 2 * 48
        assert rig.n_evicted > 0
    finally:
        rig.close()


def test_expert_cache_dropin():
    from gpu_rig import L
    n_layers, n_experts, cap, nb = 2, 16, 4, 1 << 20
    c = ExpertCache(n_layers, n_experts, cap, device="cuda", bytes_per_expert=nb)
    rng = np.random.default_rng(0)
    c.staging[:] = rng.integers(0, 256, size=c.staging.shape, dtype=np.uint8)
    assert c.prefetch(0, [1, 2, 3]) == 3
    assert c.prefetch(0, [1, 2]) == 0                  # resident: LRU touch only
    c.sync()
    hit, late, miss = c.query(0, [1, 2, 9])
    assert hit == [1, 2] and late == [] and miss == [9]
    c.admit(0, [9, 10])                                # 4 slots: 3 used + 9; 10 evicts LRU (3)
    c.sync()
    hit, late, miss = c.query(0, [3, 9, 10])
    assert miss == [3] and sorted(hit) == [9, 10]
    s = c.summary()
    assert s["fetches"] == 5 and s["evictions"] == 1 and abs(s["gb_moved"] - 5 * nb / 1e9) < 1e-12
    assert s["expert_hit_rate"] == 4 / 6
    assert c.vram_bytes() == n_layers * cap * nb
    # the bytes really moved: slot of expert 10 holds staging[10]
    back = np.empty(nb, np.uint8)
    slot = c.maps[0][10]
    assert L().moe_memcpy(back.ctypes.data, c.slot_ptr(0, slot), nb) == 0
    assert np.array_equal(back, c.staging[10])
    c.close()


@pytest.mark.parametrize("case", ["fused", "fused-sidecar", "fused-sidecar-2of3-each-early", "fused-timing-each",
                                  "unfused-sidecar", "fused-prior-logits-sidecar"])
def test_decode_layer_by_layer(tmp_path, case):
    """The per-layer op (moe_decode_layer: the reference's cached-MoE graph op,
    patches/0009:659-705) driving a real decode: layer l + 1's input is
    x_l + out_l (fp32, the same bits on the host), so no layer's input exists
    before the layer below has run.  Per token: every layer through
    moe_decode_layer (the fused launch, or split 3's launches; with the
    sidecar the call returns once its layer is launched and the cache's
    server thread serves the host's share in call order), the ids
    observed -- after the token, or after each layer as the reference's
    callback does (`each`, with early issue: uploads start mid-token) -- and
    one step.  Ids, frames, route and map traces and outputs equal the
    oracle's bit for bit, 40 tokens x 4 layers."""
    knobs = dict(admit="window", batch_tables=True)
    if "early" in case:
        knobs = dict(admit="off", early_issue=True)
    if "prior-logits" in case:
        knobs.update(cache_prior=0.01, prior_space="logits")
    rig = Rig([16, 24, 12, 40], [Q4, Q6, Q4, Q6], T=40, steer="prior" not in case, **knobs)
    rig.cache.set_decode_path(split=3 if case.startswith("unfused") else 0, graph=False)
    if "sidecar" in case:
        rig.cache.set_sidecar(6, (2, 3) if "2of3" in case else (1, 1))
    if "timing" in case:
        rig.cache.set_timing(True)
    each = "each" in case
    rp, mp = str(tmp_path / "gpu.routes"), str(tmp_path / "gpu.map")
    orp, omp = str(tmp_path / "ora.routes"), str(tmp_path / "ora.map")
    rig.cache.trace_open(rp, mp)
    oc = rig.oracle_cache()
    oc.trace_open(orp, omp)
    nl, dev, st = rig.nl, rig.dev, torch.cuda.current_stream().cuda_stream
    ids_dev = torch.empty((nl, 8), dtype=torch.int32, device=dev)
    outs = torch.empty((nl, 2048), dtype=torch.float32, device=dev)
    try:
        for t in range(rig.T):
            x = rig.x[t, 0].clone()
            for l in range(nl):
                b = None if rig.bias is None else rig.bias[t, l]
                rig.cache.decode_layer(l, x, outs[l], bias=b, ids=ids_dev[l], stream=st)
                if each:
                    rig.cache.observe(l, ids_dev[l].cpu().numpy())
                x = x + outs[l]
            got_ids = ids_dev.cpu().numpy()
            got = outs.cpu().numpy()
            if not each:
                for l in range(nl):
                    rig.cache.observe(l, got_ids[l])
            rig.cache.step()
            xh = rig.xh[t, 0].copy()
            for l in range(nl):
                tbl, prior = oc.table(l)
                use_prior = prior if rig.knobs.get("cache_prior", 0.0) > 0 else None
                bias = None if rig.bh is None else rig.bh[t, l]
                rids, rw, _, _ = O.route(rig.Wh[l], xh, 8, bias=bias, prior=use_prior, table=tbl,
                                         prior_on_logits=rig.prior_on_logits())
                assert np.array_equal(got_ids[l], rids), (t, l, got_ids[l], rids)
                want = rig.oracle_layer(t, l, rids, rw, x=xh)
                assert np.array_equal(got[l], want), (t, l, float(np.abs(got[l] - want).max()))
                oc.observe(l, rids)
                xh = (xh + want).astype(np.float32)
            oc.step()
            for l in range(nl):
                assert np.array_equal(rig.cache.frame(l), oc.frame(l)), (t, l)
        st_, ost = rig.cache.stats(), oc.stats()
        for k in ("n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied"):
            assert st_[k] == ost[k], (k, st_[k], ost[k])
        assert st_["n_scheduled"] > 0
        if "sidecar" in case:
            assert st_["n_cpu_served"] > 0
        else:
            assert st_["n_staged"] > 0          # uploads copied from what the layer kernels staged
        if "timing" in case:
            kt = rig.cache.kernel_times()
            assert kt["n_layers"] == rig.T * nl and kt["layer_ms"] > 0 and kt["layer_hbm_bytes"] > 0
    finally:
        rig.cache.close()
        oc.close()
        rig.close()
    assert open(rp).read() == open(orp).read()
    assert open(mp).read() == open(omp).read()


@pytest.mark.parametrize("graph", [2, 0], ids=["graph", "eager"])
def test_decode_one_layer_all_resident_fused(tmp_path, graph):
    """The one-layer workload: a layer of 128 experts, all resident (placed
    by a heat file naming each of them, patches/0007:431-485), an N(0,0.02)
    router with no steering, 40 tokens through the default fused launch:
    every id, frame, trace line and output bit-exact, every routed expert a
    hit, no upload."""
    E = 128
    heat = tmp_path / "all.heat"
    # (counts are halved at load, patches/0007:461: every count here stays above 0)
    heat.write_text("\n".join([f"moe-heat 1 1 {E}"] + [f"0 {e} {2 * (E - e)}" for e in range(E)]) + "\n")
    rig = Rig([E], [Q4], T=40, steer=False, admit="window", batch_tables=True)
    rig.cache.set_decode_path(split=0, graph=graph)
    try:
        assert rig.cache.heat_file(str(heat)) == (E, E)
        assert sorted(rig.cache.frame(0).tolist()) == list(range(E))
        oc = rig.oracle_cache()
        assert oc.heat_file(str(heat)) == (E, E)
        check_run(rig, tmp_path, oc=oc)
    finally:
        rig.close()
    st = rig.stats
    assert st["n_miss"] == 0 and st["n_hit"] == 40 * 8 and st["n_scheduled"] == 0


def test_sidecar_channel_selftest(tmp_path):
    """The serving channel's self-test (patches/0009:436-472, 914-925) over the
    decode's own exchange words: 2000 bounded round trips pass; with the host
    withholding its answer from round 10 on, the kernel's own 50 ms bound ends
    its wait, the call reports the 40 failed exchanges and every kernel has
    exited; the decode with CPU-assisted serving that follows is bit-exact."""
    import ctypes
    rig = Rig([16, 24], [Q4, Q6], T=16, admit="window", batch_tables=True)
    try:
        bad = ctypes.c_int(-1)
        assert L().moe_cache_sidecar_selftest(rig.cache.h, 2000, -1, 2.0, ctypes.byref(bad)) == 0, \
            L().moe_last_error()
        assert bad.value == 0
        assert L().moe_cache_sidecar_selftest(rig.cache.h, 50, 10, 0.05, ctypes.byref(bad)) == _lib.MOE_ERR_HIP
        assert bad.value == 40 and b"40 of 50" in L().moe_last_error()
        torch.cuda.synchronize()
        rig.cache.set_sidecar(4)            # its own 10000-round test passes
        rig.cache.set_decode_path(split=0, graph=True)
        check_run(rig, tmp_path)
    finally:
        rig.close()
    assert rig.stats["n_cpu_served"] > 0


def test_decode_config3_full_shape(tmp_path):
    """Cache-aware routing at full size: the single-layer shape (N(0,0.02)
    router, no steering) stacked 48 deep over 56 slots, δ = 0.01 on the
    probabilities of resident experts (patches/0007:109-124); every id is
    routed against the published tables of its step, so ids, frames and
    traces agreeing token after token checks the prior end to end."""
    rig = Rig([56] * 48, [Q6 if l % 2 else Q4 for l in range(48)], T=16, steer=False, admit="window",
              batch_tables=True, cache_prior=0.01)
    try:
        check_run(rig, tmp_path, out_every=8)
    finally:
        rig.close()
    assert rig.stats["n_hit"] > 0


def test_decode_config5_full_shape(tmp_path):
    """The wide variant at full size: 40 layers x 256 routed experts (top-8)
    + 1 always-on shared expert, I = 512, 96 slots per layer, Q6_K down in odd
    layers, Zipf(1.0) popularity with reuse 0.5, δ = 0.01, window admission,
    with CPU-assisted serving as the bench runs it."""
    rig = Rig([96] * 40, [Q6 if l % 2 else Q4 for l in range(40)], T=16, I=512, E=256, shared=True, zipf_s=1.0,
              reuse=0.5, admit="window", batch_tables=True, cache_prior=0.01)
    rig.cache.set_sidecar(8)
    try:
        check_run(rig, tmp_path, out_every=8)
    finally:
        rig.close()
    assert rig.stats["n_cpu_served"] > 0
