"""GPU parity of router lookahead and just-in-time streaming
(patches/0010-team-and-streaming.patch), through the C ABI:

  moe_route_ahead   the lookahead candidates of one or two target layers equal
                    the oracle's (or_ahead) on random and tie-heavy integer
                    inputs, with tables mixing resident, absent and streamed
                    (STREAM_BIT) words
  streaming decode  on the residual-stream workload with the mover copying
                    experts in the middle of tokens: ids equal the oracle's
                    routing and every layer's output equals the oracle's bit
                    for bit, with and without CPU-assisted serving; after each
                    token the device tables equal the host mirrors (no word
                    keeps the streamed bit); the counters add up
  J5                the map recorded with streaming, replayed without it,
                    gives the same outputs, ids and route trace (every routed
                    expert read from the same slot), as the reference's own
                    streaming exactness test requires
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_rig import H, Rig, L, stream
from moe_prefetch import _lib
from moe_prefetch import stream as S
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
Q4, Q6 = _lib.TYPE_Q4K, _lib.TYPE_Q6K
STREAM_BIT = 0x40000000


def t_(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def route_desc(W, x, E, keep):
    K = 8
    ids = torch.empty((1, K), dtype=torch.int32, device=DEV)
    w = torch.empty((1, K), dtype=torch.float32, device=DEV)
    slots = torch.empty((1, K), dtype=torch.int32, device=DEV)
    q8 = torch.empty((1, (H // 256) * 292), dtype=torch.uint8, device=DEV)
    ws = torch.zeros(L().moe_route_workspace_bytes(E, 1), dtype=torch.uint8, device=DEV)
    keep += [ids, w, slots, q8, ws]
    return _lib.RouteDesc(W.data_ptr(), x.data_ptr(), None, None, None, E, 0, E, H, K, 1, ids.data_ptr(),
                          w.data_ptr(), slots.data_ptr(), None, q8.data_ptr(), ws.data_ptr())


@pytest.mark.parametrize("E,n_targets,top_k", [(128, 2, 8), (128, 1, 8), (256, 2, 8), (128, 2, 3)])
def test_route_ahead_equals_oracle(E, n_targets, top_k):
    rng = np.random.default_rng(E + 10 * n_targets + top_k)
    S_ = 56
    for trial in range(6):
        integer = trial % 2 == 1
        if integer:        # exact scores in any order, with ties
            Wl = rng.integers(-3, 4, (E, H)).astype(np.float32)
            Wt = [rng.integers(-3, 4, (E, H)).astype(np.float32) for _ in range(n_targets)]
            x = rng.integers(-2, 3, H).astype(np.float32)
            r = [rng.integers(1, 3, H).astype(np.float32) for _ in range(n_targets)]
            for w_ in Wt:
                w_[7] = w_[3]
        else:
            Wl = rng.normal(0, 0.02, (E, H)).astype(np.float32)
            Wt = [rng.normal(0, 0.02, (E, H)).astype(np.float32) for _ in range(n_targets)]
            x = rng.normal(size=H).astype(np.float32)
            r = [(1 + 0.1 * rng.normal(size=H)).astype(np.float32) for _ in range(n_targets)]
        tbls = []
        for t in range(n_targets):
            tb = np.where(rng.random(E) < 0.5, rng.integers(0, S_, E), S_).astype(np.int32)
            streamed = rng.random(E) < 0.1
            tb[streamed] = rng.integers(0, S_, int(streamed.sum())) | STREAM_BIT   # streamed in: not a candidate
            tbls.append(tb)
        keep = []
        Wd, xd = t_(Wl), t_(x)
        d = route_desc(Wd, xd, E, keep)
        Wtd = [t_(w_) for w_ in Wt]
        rd = [t_(r_) for r_ in r]
        tbd = [t_(tb) for tb in tbls]
        got = S.route_ahead(d, [w_.data_ptr() for w_ in Wtd], [r_.data_ptr() for r_ in rd],
                            [tb.data_ptr() for tb in tbd], [S_] * n_targets, top_k=top_k, stream=stream())
        for t in range(n_targets):
            want, _ = O.ahead(Wt[t], x, r[t], tbls[t], S_, top_k)
            assert list(got[t]) == list(want), (trial, t, got[t], want)


def dev_tables(rig):
    out = []
    for l in range(rig.nl):
        v = rig.cache.lookup(l)
        h = np.empty(rig.E, np.int32)
        _lib.check(L().moe_memcpy(h.ctypes.data, v.dev_table, rig.E * 4), "table readback")
        out.append(h)
    return out


def run_stream(rig, tmp_path, name, sidecar, record=True, check_tables=True):
    if sidecar:
        rig.cache.set_sidecar(4, share=(1, 1))
    rig.cache.set_streaming(True, per_layer=4, reserve=2, top_k=8)
    rp, mp = str(tmp_path / f"{name}.routes"), str(tmp_path / f"{name}.map") if record else None
    rig.cache.trace_open(rp, mp)
    out = torch.empty((rig.nl, H), dtype=torch.float32, device=DEV)
    ids_all, outs = [], []
    for t in range(rig.T):
        ids_all.append(rig.cache.decode_token(rig.x[t], out, stream=stream()).copy())
        outs.append(out.cpu().numpy().copy())
        if check_tables:
            for l, d in enumerate(dev_tables(rig)):
                assert not (d & STREAM_BIT).any(), (t, l)
                assert np.array_equal(d, rig.cache.table(l)[0]), (t, l)
    ss = rig.cache.stream_stats()
    return ids_all, outs, ss, rp, mp


def check_exact(rig, ids_all, outs):
    for t in range(rig.T):
        for l in range(rig.nl):
            rids, rw, _, _ = O.route(rig.Wh[l], rig.xh[t, l], 8)
            assert np.array_equal(ids_all[t][l], rids), (t, l)
            want = rig.oracle_layer(t, l, rids, rw)
            assert np.array_equal(outs[t][l], want), (t, l)


@pytest.mark.parametrize("sidecar", [False, True], ids=["gpu-only", "sidecar"])
def test_streaming_decode_exact_and_replayable(tmp_path, sidecar):
    slots = [24, 20, 24, 16, 24, 20, 24, 16]
    dts = [Q4, Q6] * 4
    print(f"[stream] residual workload, {len(slots)} layers, sidecar={sidecar}", flush=True)
    rig = Rig(slots, dts, T=48, residual=True, admit="window", batch_tables=True, early_issue=True)
    try:
        ids_all, outs, ss, rp, mp = run_stream(rig, tmp_path, "s", sidecar)
        rig.cache.close()
        print("stream counters", ss, flush=True)
        assert ss["failed"] == 0
        assert ss["records"] == rig.T * rig.nl
        assert ss["landed"] <= ss["offered"] and ss["in_time"] + ss["late"] <= ss["offered"]
        assert ss["unused"] <= ss["landed"]
        assert ss["offered"] > 0
        check_exact(rig, ids_all, outs)
    finally:
        rig.close()
    # J5: replay the recorded map without streaming
    rig2 = Rig(slots, dts, T=48, residual=True, admit="window", batch_tables=True)
    try:
        rig2.cache.map_replay(mp)
        rr = str(tmp_path / "r.routes")
        rig2.cache.trace_open(rr, None)
        out = torch.empty((rig2.nl, H), dtype=torch.float32, device=DEV)
        for t in range(rig2.T):
            ids = rig2.cache.decode_token(rig2.x[t], out, stream=stream())
            assert np.array_equal(ids, ids_all[t]), t
            assert np.array_equal(out.cpu().numpy(), outs[t]), t
        rig2.cache.close()
        assert open(rr).read() == open(rp).read()
    finally:
        rig2.close()


def test_streaming_graph_off_and_eager_timing(tmp_path):
    # the eager path (kernel timing on) streams the same way
    slots = [24, 16, 24, 16]
    rig = Rig(slots, [Q4, Q6, Q4, Q6], T=24, residual=True, admit="off", batch_tables=True, early_issue=True)
    try:
        rig.cache.set_timing(True)
        ids_all, outs, ss, _, _ = run_stream(rig, tmp_path, "e", False, record=False)
        assert ss["failed"] == 0 and ss["records"] == rig.T * rig.nl
        check_exact(rig, ids_all, outs)
        kt = rig.cache.kernel_times()
        assert kt["n_layers"] == rig.T * rig.nl
    finally:
        rig.close()


def test_streaming_off_again_and_errors():
    rig = Rig([16, 16], [Q4, Q6], T=4, residual=True, admit="off", batch_tables=True, early_issue=True)
    try:
        rig.cache.set_streaming(True)
        with pytest.raises(Exception):
            rig.cache.set_streaming(True)               # on already
        out = torch.empty((rig.nl, H), dtype=torch.float32, device=DEV)
        rig.cache.decode_token(rig.x[0], out, stream=stream())
        rig.cache.set_streaming(False)
        rig.cache.decode_token(rig.x[1], out, stream=stream())
        rids, rw, _, _ = O.route(rig.Wh[1], rig.xh[1, 1], 8)
        assert np.array_equal(out.cpu().numpy()[1], rig.oracle_layer(1, 1, rids, rw))
    finally:
        rig.close()
    rig = Rig([16, 16], [Q4, Q6], T=2, admit="off", batch_tables=True, early_issue=True)
    try:
        with pytest.raises(Exception):
            rig.cache.set_streaming(True)               # no norm weights registered
    finally:
        rig.close()
