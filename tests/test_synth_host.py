"""The synthetic generator's weights and vectors (host side, CPU only):
Q4_K / Q6_K blocks from the product generator dequantize (through the oracle)
to within a quantization step of the N(0, sigma) draws they encode; the
normal draws have the stated moments."""
import ctypes

import numpy as np

import moe_prefetch
from moe_prefetch import _lib
from oracle import oracle as O


def synth_host(layer, e0, n, H, I, dt, sigma=0.02, seed=3):
    L = moe_prefetch.lib()
    eb = L.moe_expert_bytes(H, I, dt)
    buf = np.zeros(n * eb, np.uint8)
    _lib.check(L.moe_synth_experts_host(seed, layer, e0, n, H, I, dt, sigma, buf.ctypes.data, eb, 4), "synth")
    return buf, eb


def test_vectors_are_standard_normal_like():
    L = moe_prefetch.lib()
    out = np.empty(200000, np.float32)
    _lib.check(L.moe_synth_vec_host(1, 1, 0, 1, 0, 1, out.size, 1.0, out.ctypes.data), "vec")
    assert abs(out.mean()) < 0.01 and abs(out.std() - 1.0) < 0.01
    assert np.abs(out).max() <= 6.0
    # exactly representable grid of the 12-uniform method: multiples of 1/1024
    assert np.all(out * 1024 == np.round(out * 1024))
    # a different (kind, a, b) is a different stream
    out2 = np.empty(1000, np.float32)
    _lib.check(L.moe_synth_vec_host(1, 1, 0, 1, 1, 1, 1000, 1.0, out2.ctypes.data), "vec")
    assert not np.array_equal(out[:1000], out2)


def test_q4k_q6k_blocks_round_trip():
    H, I = 2048, 256
    for dt in (_lib.TYPE_Q4K, _lib.TYPE_Q6K):
        buf, eb = synth_host(0, 5, 2, H, I, dt)
        upb = I * (H // 256) * 144
        for e in range(2):
            ex = buf[e * eb:(e + 1) * eb]
            up = O.dequant(O.Q4K, ex[:upb], I * H)
            down = O.dequant(dt, ex[2 * upb:], H * I)
            for w in (up, down):
                assert np.isfinite(w).all()
                assert 0.015 < w.std() < 0.025          # N(0, 0.02) survives quantization
            # quantization error: reconstruct the draws from the same stream
            assert abs(up.mean()) < 2e-3


def test_generator_is_deterministic_and_expert_specific():
    a, eb = synth_host(3, 0, 2, 2048, 256, _lib.TYPE_Q4K)
    b, _ = synth_host(3, 0, 2, 2048, 256, _lib.TYPE_Q4K)
    c, _ = synth_host(3, 1, 1, 2048, 256, _lib.TYPE_Q4K)
    assert np.array_equal(a, b)
    assert np.array_equal(a[eb:], c)          # expert 1 is expert 1 whatever the batch
    assert not np.array_equal(a[:eb], a[eb:])
