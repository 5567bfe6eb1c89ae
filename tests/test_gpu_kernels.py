"""GPU parity of the hand-written gfx950 kernels, through the C ABI, against
the CPU oracle on the same seeded inputs.

  generator   device bytes == host bytes (experts, vectors)
  moe_route   ids, slots, gate weights, probabilities and the Q8_K bytes of x
              bit-exact (E = 128 and 256, k = 1/8/16, batches of tokens,
              steering bias, cache prior, integer-valued inputs with ties)
  moe_experts the batch-1 expert chain + combine equal, bit for bit, to the
              oracle's ggml-style dequant+dot path (so within the 1e-3 relative
              L2 bar): Q4_K and Q6_K down, intermediate 768 and 512, experts
              read from HBM slots and from pinned host memory, k = 1..9,
              accumulate
"""
import ctypes

import numpy as np
import pytest
import torch

from gpu_rig import H, Pinned, L, stream, synth_experts_dev
from moe_prefetch import _lib
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def t_(a, dtype=None):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


@pytest.mark.parametrize("dt", [_lib.TYPE_Q4K, _lib.TYPE_Q6K])
@pytest.mark.parametrize("I", [768, 512])
def test_device_generator_matches_host(dt, I):
    eb = L().moe_expert_bytes(H, I, dt)
    dev = torch.empty(3 * eb, dtype=torch.uint8, device=DEV)
    synth_experts_dev(9, 5, 40, 3, I, dt, dev.data_ptr(), eb)
    host = np.zeros(3 * eb, np.uint8)
    _lib.check(L().moe_synth_experts_host(9, 5, 40, 3, H, I, dt, 0.02, host.ctypes.data, eb, 8), "host")
    got = dev.cpu().numpy()
    bad = np.flatnonzero(got != host)
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:5]}"
    v = torch.empty(3 * 5 * 300, dtype=torch.float32, device=DEV)
    _lib.check(L().moe_synth_vec(9, 1, 2, 3, 1, 5, 300, 1.0, v.data_ptr(), stream()), "vec")
    vh = np.empty(v.numel(), np.float32)
    _lib.check(L().moe_synth_vec_host(9, 1, 2, 3, 1, 5, 300, 1.0, vh.ctypes.data), "vec host")
    assert np.array_equal(v.cpu().numpy(), vh)


def run_route(W, x, K, bias=None, prior=None, table=None, dummy=None, probs=True, prior_on_logits=False):
    E, Hh = W.shape
    n_tok = x.shape[0]
    Wd, xd = t_(W), t_(x)
    bd = None if bias is None else t_(bias)
    pd = None if prior is None else t_(prior)
    td = None if table is None else t_(table)
    ids = torch.empty((n_tok, K), dtype=torch.int32, device=DEV)
    w = torch.empty((n_tok, K), dtype=torch.float32, device=DEV)
    slots = torch.empty((n_tok, K), dtype=torch.int32, device=DEV)
    pr = torch.empty((n_tok, E), dtype=torch.float32, device=DEV)
    q8 = torch.empty((n_tok, (Hh // 256) * 292), dtype=torch.uint8, device=DEV)
    ws = torch.zeros(L().moe_route_workspace_bytes(E, n_tok), dtype=torch.uint8, device=DEV)
    d = _lib.RouteDesc(Wd.data_ptr(), xd.data_ptr(), None if bd is None else bd.data_ptr(),
                       None if pd is None else pd.data_ptr(), None if td is None else td.data_ptr(),
                       E if dummy is None else dummy, int(prior_on_logits), E, Hh, K, n_tok, ids.data_ptr(), w.data_ptr(),
                       slots.data_ptr(), pr.data_ptr() if probs else None, q8.data_ptr(), ws.data_ptr())
    _lib.check(L().moe_route(ctypes.byref(d), stream()), "moe_route")
    torch.cuda.synchronize()
    return ids.cpu().numpy(), w.cpu().numpy(), slots.cpu().numpy(), pr.cpu().numpy(), q8.cpu().numpy()


@pytest.mark.parametrize("E,K,n_tok", [(128, 8, 1), (128, 8, 16), (256, 8, 4), (128, 1, 3), (128, 16, 2)])
def test_route_bit_exact(E, K, n_tok):
    rng = np.random.default_rng(E * 100 + K + n_tok)
    for trial in range(4):
        W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        x = rng.standard_normal((n_tok, H)).astype(np.float32)
        bias = prior = table = None
        if trial >= 1:
            table = np.where(rng.random(E) < 0.4, rng.permutation(E).astype(np.int32) % 56, 56).astype(np.int32)
        if trial >= 2:
            prior = np.where(table < 56, 0.01, 0.0).astype(np.float32)
        if trial == 3:
            bias = np.zeros((n_tok, E), np.float32)
            for t in range(n_tok):
                bias[t, rng.choice(E, K, replace=False)] = 12.0
        ids, w, slots, probs, q8 = run_route(W, x, K, bias, prior, table, dummy=56)
        for t in range(n_tok):
            rids, rw, rslots, rprobs = O.route(W, x[t], K, bias=None if bias is None else bias[t],
                                               prior=prior, table=table)
            assert np.array_equal(ids[t], rids), (trial, t)
            assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32)), (trial, t)
            assert np.array_equal(probs[t].view(np.uint32), rprobs.view(np.uint32)), (trial, t)
            if table is not None:
                assert np.array_equal(slots[t], rslots)
            else:
                assert np.all(slots[t] == 56)
            assert np.array_equal(q8[t], O.quant_q8k(x[t]))


def test_route_prior_on_logits_bit_exact():
    rng = np.random.default_rng(8)
    E, K = 128, 8
    for trial in range(4):
        W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
        x = rng.standard_normal((3, H)).astype(np.float32)
        table = np.where(rng.random(E) < 0.5, np.arange(E) % 56, 56).astype(np.int32)
        prior = np.where(table < 56, 0.3, 0.0).astype(np.float32)
        ids, w, slots, probs, _ = run_route(W, x, K, None, prior, table, dummy=56, prior_on_logits=True)
        for t in range(3):
            rids, rw, rslots, _ = O.route(W, x[t], K, prior=prior, table=table, prior_on_logits=True)
            assert np.array_equal(ids[t], rids)
            assert np.array_equal(w[t].view(np.uint32), rw.view(np.uint32))
            assert np.array_equal(slots[t], rslots)
            pids, _, _, _ = O.route(W, x[t], K, prior=prior, table=table)
            # with a 0.3 bonus the two spaces pick differently on these inputs
            if trial == 0 and t == 0:
                assert not np.array_equal(pids, rids)


def test_route_integer_ties_lower_id_wins():
    rng = np.random.default_rng(3)
    E, K = 128, 8
    for trial in range(10):
        W = (rng.integers(-2, 3, size=(E, H)) * (rng.random((E, H)) < 0.004)).astype(np.float32)
        W[9] = W[100]
        W[17] = W[3]
        x = rng.integers(-2, 3, size=(1, H)).astype(np.float32)
        ids, w, _, _, _ = run_route(W, x, K)
        lg = W.astype(np.int64) @ x[0].astype(np.int64)
        order = sorted(range(E), key=lambda e: (-lg[e], e))
        assert list(ids[0]) == order[:K]


def test_route_q8_special_blocks():
    E = 128
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((E, H)) * 0.02).astype(np.float32)
    x = rng.standard_normal((1, H)).astype(np.float32)
    x[0, :256] = 0.0                      # an all-zero block: d = 0
    x[0, 256:512] = 3.0                   # constant block: every value ties for the max
    x[0, 600] = -50.0                     # a negative extreme
    _, _, _, _, q8 = run_route(W, x, 8)
    assert np.array_equal(q8[0], O.quant_q8k(x[0]))


def make_experts(n, I, dt, seed=5, layer=0):
    eb = L().moe_expert_bytes(H, I, dt)
    pool = torch.empty(n * eb, dtype=torch.uint8, device=DEV)
    synth_experts_dev(seed, layer, 0, n, I, dt, pool.data_ptr(), eb)
    store = Pinned(n * eb)
    torch.cuda.synchronize()
    _lib.check(L().moe_memcpy(store.ptr, pool.data_ptr(), n * eb), "copy")
    return pool, store, eb


def run_experts(pool, store, eb, n, I, dt, ids, slots, w, x, accumulate=False, out0=None):
    K = len(ids)
    q8x = t_(O.quant_q8k(x))
    idd, sd, wd = t_(np.asarray(ids, np.int32)), t_(np.asarray(slots, np.int32)), t_(np.asarray(w, np.float32))
    out = t_(out0.copy()) if out0 is not None else torch.zeros(H, dtype=torch.float32, device=DEV)
    ws = torch.zeros(L().moe_experts_workspace_bytes(I, K), dtype=torch.uint8, device=DEV)
    d = _lib.ExpertsDesc(idd.data_ptr(), sd.data_ptr(), wd.data_ptr(), pool.data_ptr(), eb, n, store.dev, eb, n,
                         q8x.data_ptr(), out.data_ptr(), int(accumulate), H, I, K, dt, ws.data_ptr())
    _lib.check(L().moe_experts(ctypes.byref(d), stream()), "moe_experts")
    torch.cuda.synchronize()
    return out.cpu().numpy()


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / np.linalg.norm(b))


@pytest.mark.parametrize("dt", [_lib.TYPE_Q4K, _lib.TYPE_Q6K])
@pytest.mark.parametrize("I", [768, 512])
def test_experts_within_tolerance(dt, I):
    n = 16
    pool, store, eb = make_experts(n, I, dt, seed=11 + I + dt)
    rng = np.random.default_rng(I + dt)
    try:
        for mode in ("hit", "miss", "mixed"):
            for K in (8, 1, 9):
                ids = rng.choice(n, K, replace=False)
                if mode == "hit":
                    slots = ids.copy()
                elif mode == "miss":
                    slots = np.full(K, n)
                else:
                    slots = np.where(np.arange(K) % 2 == 0, ids, n)
                w = rng.random(K).astype(np.float32)
                w /= w.sum()
                x = rng.standard_normal(H).astype(np.float32)
                got = run_experts(pool, store, eb, n, I, dt, ids, slots, w, x)
                want = O.moe_layer(H, I, dt, [store.arr[e * eb:(e + 1) * eb] for e in ids], w, x)
                r = rel_l2(got, want)
                assert r < 1e-3, (mode, K, r)
                # integer dots, and the fp32 steps in the CPU chain's order: bit for bit
                assert np.array_equal(got, want), (mode, K, r)
    finally:
        store.free()


@pytest.mark.parametrize("dt", [_lib.TYPE_Q4K, _lib.TYPE_Q6K])
def test_experts_repeated_ids(dt):
    # the reference's repeated-ids mode (cpp/test-moe-rows.cpp:60-67, mode 3):
    # routed slot k takes expert k % 2, expert 0 resident and expert 1 read
    # from the pinned store; then one expert in every slot, and ids drawn with
    # replacement over mixed sources -- bit for bit as the oracle
    I, n = 768, 16
    pool, store, eb = make_experts(n, I, dt, seed=7 + dt)
    rng = np.random.default_rng(31 + dt)
    try:
        cases = [(np.arange(8) % 2, np.where(np.arange(8) % 2 == 0, 0, n)),
                 (np.full(8, 5), np.full(8, 5)), (np.full(8, 9), np.full(8, n))]
        ids = rng.choice(4, 8, replace=True)
        cases.append((ids, np.where(ids % 2 == 0, ids, n)))
        for ids, slots in cases:
            w = rng.random(8).astype(np.float32)
            w /= w.sum()
            x = rng.standard_normal(H).astype(np.float32)
            got = run_experts(pool, store, eb, n, I, dt, ids, slots, w, x)
            want = O.moe_layer(H, I, dt, [store.arr[e * eb:(e + 1) * eb] for e in ids], w, x)
            assert np.array_equal(got, want), (ids, slots, rel_l2(got, want))
    finally:
        store.free()


def test_experts_accumulate_and_zero_input():
    I, dt, n = 768, _lib.TYPE_Q4K, 8
    pool, store, eb = make_experts(n, I, dt)
    try:
        rng = np.random.default_rng(2)
        ids = np.arange(8)
        w = np.full(8, 0.125, np.float32)
        x = rng.standard_normal(H).astype(np.float32)
        base = rng.standard_normal(H).astype(np.float32)
        got = run_experts(pool, store, eb, n, I, dt, ids, ids, w, x, accumulate=True, out0=base)
        want = O.moe_layer(H, I, dt, [store.arr[e * eb:(e + 1) * eb] for e in ids], w, x)
        assert rel_l2(got - base, want) < 1e-4
        assert np.array_equal(got, base + want)
        z = run_experts(pool, store, eb, n, I, dt, ids, ids, w, np.zeros(H, np.float32))
        assert not z.any()
    finally:
        store.free()


def test_experts_rejects_unmapped_host_memory():
    I, dt, n = 768, _lib.TYPE_Q4K, 2
    pool, store, eb = make_experts(n, I, dt)
    plain = np.zeros(n * eb + 64, np.uint8)          # pageable: never handed to a kernel
    addr = (plain.ctypes.data + 15) // 16 * 16
    try:
        q8x = t_(O.quant_q8k(np.ones(H, np.float32)))
        ids = t_(np.array([0, 1], np.int32))
        w = t_(np.array([0.5, 0.5], np.float32))
        out = torch.zeros(H, dtype=torch.float32, device=DEV)
        ws = torch.zeros(L().moe_experts_workspace_bytes(I, 2), dtype=torch.uint8, device=DEV)
        d = _lib.ExpertsDesc(ids.data_ptr(), ids.data_ptr(), w.data_ptr(), pool.data_ptr(), eb, n, addr, eb, n,
                             q8x.data_ptr(), out.data_ptr(), 0, H, I, 2, dt, ws.data_ptr())
        assert L().moe_experts(ctypes.byref(d), stream()) != 0
        assert b"not device memory" in L().moe_last_error()
    finally:
        store.free()


def test_h2d_batch_copies_three_slices():
    # moe_memcpy_h2d_batch through the C ABI as the reference's upload worker
    # calls ggml_backend_cuda_memcpy_h2d_batch (patches/0006...:52-76,
    # 428-440): the up, gate and down slices of two experts of the pinned
    # store, each to its place in a slot, one synchronisation; read back
    I, dt = 768, _lib.TYPE_Q6K
    eb = L().moe_expert_bytes(H, I, dt)
    gu = I * (H // 256) * 144            # one Q4_K matrix (up or gate)
    store = Pinned(3 * eb)
    try:
        _lib.check(L().moe_synth_experts_host(13, 2, 0, 3, H, I, dt, 0.02, store.ptr, eb, 8), "host")
        slots = torch.zeros(2 * eb, dtype=torch.uint8, device=DEV)
        torch.cuda.synchronize()
        cuts = [(0, gu), (gu, gu), (2 * gu, eb - 2 * gu)]
        dst, src, sizes = [], [], []
        for slot, e in ((0, 2), (1, 0)):          # expert 2 -> slot 0, expert 0 -> slot 1
            for off, n in cuts:
                dst.append(slots.data_ptr() + slot * eb + off)
                src.append(store.ptr + e * eb + off)
                sizes.append(n)
        P = ctypes.c_void_p * 6
        ok = L().moe_memcpy_h2d_batch(0, P(*dst), P(*src), (ctypes.c_size_t * 6)(*sizes), 6)
        assert ok is True, L().moe_last_error()
        got = slots.cpu().numpy()
        assert np.array_equal(got[:eb], store.arr[2 * eb:3 * eb])
        assert np.array_equal(got[eb:], store.arr[:eb])
    finally:
        store.free()
