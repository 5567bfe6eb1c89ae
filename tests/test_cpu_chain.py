"""The host CPU expert chain (moe_cpu_experts: the path that serves experts
absent from the HBM slots on the CPU) against the oracle's chain, bit for bit:
Q4_K and Q6_K down, intermediate 256/512/768, the AVX-512 VNNI dots and the
portable ones, 1..9 experts, 1..8 threads, and inputs with zero, constant and
extreme blocks."""
import ctypes

import numpy as np
import pytest

import moe_prefetch
from moe_prefetch import _lib
from oracle import oracle as O

H = 2048
Q4, Q6 = _lib.TYPE_Q4K, _lib.TYPE_Q6K


def L():
    return moe_prefetch.lib()


def synth(n, I, dt, seed):
    eb = L().moe_expert_bytes(H, I, dt)
    buf = np.empty(n * eb, np.uint8)
    _lib.check(L().moe_synth_experts_host(seed, 0, 0, n, H, I, dt, 0.02, buf.ctypes.data, eb, 4), "synth")
    return buf, eb


def cpu_rows(buf, eb, ks, I, dt, q8x, threads, portable):
    n = len(ks)
    ptrs = (ctypes.c_void_p * n)(*[buf.ctypes.data + int(k) * eb for k in ks])
    rows = np.full((n, H), np.nan, np.float32)
    _lib.check(L().moe_cpu_experts(ctypes.cast(ptrs, ctypes.c_void_p), n, q8x.ctypes.data, H, I, dt,
                                   rows.ctypes.data, threads, int(portable)), "moe_cpu_experts")
    return rows


def paths():
    out = [True]
    if L().moe_cpu_has_vnni():
        out.insert(0, False)
    return out


@pytest.mark.parametrize("dt", [Q4, Q6], ids=["q4k_down", "q6k_down"])
@pytest.mark.parametrize("I", [256, 512, 768])
def test_cpu_chain_matches_oracle(dt, I):
    n = 9
    buf, eb = synth(n, I, dt, seed=100 + I + dt)
    rng = np.random.default_rng(I * 31 + dt)
    x = rng.standard_normal(H).astype(np.float32)
    q8x = O.quant_q8k(x)
    want = np.stack([O.expert_chain(H, I, dt, buf[k * eb:(k + 1) * eb], x)[0] for k in range(n)])
    for portable in paths():
        for threads, ks in ((1, [0]), (3, [4, 1, 7]), (8, list(range(n)))):
            got = cpu_rows(buf, eb, ks, I, dt, q8x, threads, portable)
            for j, k in enumerate(ks):
                assert np.array_equal(got[j], want[k]), (portable, threads, k,
                                                         float(np.abs(got[j] - want[k]).max()))


@pytest.mark.parametrize("dt", [Q4, Q6], ids=["q4k_down", "q6k_down"])
def test_cpu_chain_special_inputs(dt):
    # zero activations, a constant block, one huge value per block, and a
    # block at the edge of fp16-sized magnitudes: the Q8_K of x and of h and
    # every dot follow the oracle exactly
    I, n = 512, 3
    buf, eb = synth(n, I, dt, seed=7)
    cases = [np.zeros(H, np.float32), np.full(H, 0.5, np.float32)]
    spike = np.random.default_rng(3).standard_normal(H).astype(np.float32)
    spike[::256] = 1e4
    cases.append(spike)
    wide = (np.random.default_rng(4).standard_normal(H) * 3e3).astype(np.float32)
    cases.append(wide)
    for x in cases:
        q8x = O.quant_q8k(x)
        for portable in paths():
            got = cpu_rows(buf, eb, range(n), I, dt, q8x, 4, portable)
            for k in range(n):
                want = O.expert_chain(H, I, dt, buf[k * eb:(k + 1) * eb], x)[0]
                assert np.array_equal(got[k], want), (portable, k)


def test_cpu_chain_rejects_bad_shapes():
    buf, eb = synth(1, 512, Q4, seed=1)
    q8x = O.quant_q8k(np.ones(H, np.float32))
    ptrs = (ctypes.c_void_p * 1)(buf.ctypes.data)
    rows = np.empty(H, np.float32)
    assert L().moe_cpu_experts(ctypes.cast(ptrs, ctypes.c_void_p), 1, q8x.ctypes.data, 1024, 512, Q4,
                               rows.ctypes.data, 1, 0) != 0
    assert L().moe_cpu_experts(ctypes.cast(ptrs, ctypes.c_void_p), 1, q8x.ctypes.data, H, 500, Q4,
                               rows.ctypes.data, 1, 0) != 0
    assert L().moe_cpu_experts(ctypes.cast(ptrs, ctypes.c_void_p), 1, q8x.ctypes.data, H, 512, 13,
                               rows.ctypes.data, 1, 0) != 0


@pytest.mark.parametrize("dt", [Q4, Q6], ids=["q4k_down", "q6k_down"])
def test_grouped_tokens_chain_matches_oracle(dt):
    """Groups of tokens sharing an expert (CPU-assisted batched decode): each
    group's rows are read once for all of its tokens; every token's rows equal
    the oracle's chain for that expert and token, bit for bit."""
    I = 512
    buf, eb = synth(5, I, dt, seed=31 + dt)
    groups = [(3, 4), (0, 1), (4, 3), (1, 2), (2, 1)]       # (expert, tokens)
    n = sum(c for _, c in groups)
    rng = np.random.default_rng(17)
    xs = rng.standard_normal((n, H)).astype(np.float32)
    xs[2] *= 40.0                                          # a wide token among them
    q8 = np.stack([O.quant_q8k(x) for x in xs])
    ptrs = (ctypes.c_void_p * len(groups))(*[buf.ctypes.data + e * eb for e, _ in groups])
    count = np.asarray([c for _, c in groups], np.int32)
    for threads in (1, 5):
        rows = np.full((n, H), np.nan, np.float32)
        _lib.check(L().moe_cpu_experts_tokens(ctypes.cast(ptrs, ctypes.c_void_p), len(groups), count.ctypes.data,
                                              q8.ctypes.data, H, I, dt, rows.ctypes.data, threads), "tokens")
        j = 0
        for e, c in groups:
            for _ in range(c):
                want = O.expert_chain(H, I, dt, buf[e * eb:(e + 1) * eb], xs[j])[0]
                assert np.array_equal(rows[j], want), (threads, e, j)
                j += 1
