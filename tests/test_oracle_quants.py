"""Pins for the oracle's block codecs and integer dot products (CPU only).

ggml's K-quant code is not vendored in the reference, so nothing there holds a
quantized block to compare against.  These checks pin the restatement by what
the mathematics fixes:
  * fp16 conversions against numpy's IEEE binary16 (all 65536 codes; RNE);
  * Q8_K: the largest-magnitude value maps to -127, |q| <= 127, the error of
    every element is at most half a step, the group sums are the sums, and an
    all-zero block is d = 0;
  * the integer dot (or_dot_*) against an fp64 dequantise-then-dot of the same
    operands, which is exact up to the fp32 rounding of the block sums;
  * one-hot probes that place a single non-zero code at every position of a
    block and require the dequantised vector to be that one element, so a
    transposed nibble, a wrong half or a wrong scale index fails;
  * special blocks: d = 0, dmin = 0, constant codes.
"""
import numpy as np
import pytest

from oracle import oracle as O

rng = np.random.default_rng(7)


def test_h2f_all_codes():
    codes = np.arange(65536, dtype=np.uint16)
    want = codes.view(np.float16).astype(np.float32)
    got = np.array([O.h2f(int(c)) for c in codes[::7]], np.float32)
    w = want[::7]
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), w[~nan].view(np.uint32))


def test_f2h_round_nearest_even():
    xs = np.concatenate([rng.standard_normal(4000).astype(np.float32) * s
                         for s in (1e-6, 1e-3, 1.0, 1e3, 6e4)])
    edge = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                     3 * 2.0 ** -26, 2.0 ** -14, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], np.float32)
    xs = np.concatenate([xs, edge])
    with np.errstate(over="ignore"):
        want = xs.astype(np.float16).view(np.uint16)
    got = np.array([O.f2h(float(v)) for v in xs], np.uint16)
    assert np.array_equal(got, want)


def _q8_fields(b):
    d = b[:4].view(np.float32)[0]
    qs = b[4:260].view(np.int8)
    bs = b[260:292].view(np.int16)
    return d, qs, bs


def test_q8k_properties():
    for scale in (1e-3, 1.0, 50.0):
        x = (rng.standard_normal(256 * 6) * scale).astype(np.float32)
        x[300] = -7.5 * scale          # block 1 has a negative extreme
        q = O.quant_q8k(x)
        for i in range(6):
            d, qs, bs = _q8_fields(q[i * 292:(i + 1) * 292])
            xb = x[i * 256:(i + 1) * 256]
            j = int(np.argmax(np.abs(xb)))
            assert qs[j] == -127
            assert np.all(np.abs(qs.astype(int)) <= 127)
            err = np.abs(d * qs.astype(np.float64) - xb)
            assert err.max() <= abs(d) * 0.5 * (1 + 1e-5)
            assert np.array_equal(bs, qs.astype(np.int32).reshape(16, 16).sum(1))


def test_q8k_zero_block_and_first_tie():
    x = np.zeros(512, np.float32)
    x[256 + 3] = 2.0
    x[256 + 9] = -2.0                   # same magnitude later: first one wins
    q = O.quant_q8k(x)
    d0, qs0, bs0 = _q8_fields(q[:292])
    assert d0 == 0 and not qs0.any() and not bs0.any()
    d1, qs1, _ = _q8_fields(q[292:])
    assert qs1[3] == -127 and qs1[9] == 127 and d1 < 0


def _rand_q4k(nb, d=0.01, dmin=0.02):
    b = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    b[:, 0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[:, 2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    return b.reshape(-1)


def _rand_q6k(nb, d=0.003):
    b = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    b[:, 208:210] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("wtype", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("n", [256, 768, 2048])
def test_int_dot_vs_f64(wtype, n):
    for _ in range(20):
        w = _rand_q4k(n // 256) if wtype == O.Q4K else _rand_q6k(n // 256)
        x = rng.standard_normal(n).astype(np.float32)
        q8 = O.quant_q8k(x)
        got = O.dot(wtype, n, w, q8)
        ref = O.dot_f64(wtype, n, w, q8)
        # also an independent fp64 path: dequantise each side with numpy
        wd = O.dequant(wtype, w, n).astype(np.float64)
        xd = O.dequant_q8k(q8, n).astype(np.float64)
        assert abs(ref - wd @ xd) <= 1e-5 * (np.abs(wd) @ np.abs(xd))
        assert abs(got - ref) <= 2e-6 * (abs(ref) + 1e-3 * (np.abs(wd) @ np.abs(xd)))


def _q4k_block(d, dmin, sc, mn, codes):
    """Pack a Q4_K block from 8 6-bit scales/mins and 256 4-bit codes, following
    the 12-byte packing: bytes 0-3 low 6 bits of scales 0-3 (top 2 bits carry
    scales 4-7's high bits), bytes 4-7 likewise for mins, bytes 8-11 low nibbles
    of scales 4-7 | mins 4-7 << 4."""
    s = np.zeros(12, np.uint8)
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    qs = np.zeros(128, np.uint8)
    for e in range(256):
        byte = (e // 64) * 32 + e % 32
        qs[byte] |= codes[e] << (4 if e % 64 >= 32 else 0)
    return np.concatenate([np.frombuffer(np.float16(d).tobytes(), np.uint8),
                           np.frombuffer(np.float16(dmin).tobytes(), np.uint8), s, qs])


def test_q4k_one_hot_every_position():
    sc = [1, 2, 3, 5, 7, 11, 13, 63]
    mn = [0] * 8
    for e in range(256):
        codes = np.zeros(256, np.uint8)
        codes[e] = 9
        y = O.dequant(O.Q4K, _q4k_block(0.5, 0.0, sc, mn, codes), 256)
        want = np.zeros(256, np.float32)
        want[e] = 0.5 * sc[e // 32] * 9
        assert np.array_equal(y, want), e


def test_q4k_mins_and_special_blocks():
    sc = [0] * 8
    mn = [1, 2, 4, 8, 16, 32, 63, 40]
    y = O.dequant(O.Q4K, _q4k_block(1.0, 0.25, sc, mn, np.full(256, 15, np.uint8)), 256)
    assert np.array_equal(y, np.repeat(-0.25 * np.array(mn, np.float32), 32))
    # d = 0 and dmin = 0: the block is zero whatever the codes
    z = _q4k_block(0.0, 0.0, [63] * 8, [63] * 8, rng.integers(0, 16, 256).astype(np.uint8))
    assert not O.dequant(O.Q4K, z, 256).any()
    q8 = O.quant_q8k(rng.standard_normal(256).astype(np.float32))
    assert O.dot(O.Q4K, 256, z, q8) == 0.0


def _q6k_block(d, sc, codes):
    """codes: 256 values in 0..63 (stored value = code, dequant = d*sc*(code-32))."""
    ql = np.zeros(128, np.uint8)
    qh = np.zeros(64, np.uint8)
    for e in range(256):
        h, r = divmod(e, 128)
        g, l = divmod(r, 32)
        lo, hi = codes[e] & 15, codes[e] >> 4
        ql[64 * h + l + 32 * (g & 1)] |= lo << (4 if g >= 2 else 0)
        qh[32 * h + l] |= hi << (2 * g)
    return np.concatenate([ql, qh, np.array(sc, np.int8).view(np.uint8),
                           np.frombuffer(np.float16(d).tobytes(), np.uint8)])


def test_q6k_one_hot_every_position():
    sc = [1, -2, 3, -4, 5, 6, 7, 8, 9, 10, -11, 12, 13, 14, 15, -128]
    for e in range(256):
        codes = np.full(256, 32, np.uint8)
        codes[e] = 32 + 17 if e % 2 else 32 - 29
        y = O.dequant(O.Q6K, _q6k_block(0.25, sc, codes), 256)
        want = np.zeros(256, np.float32)
        h, r = divmod(e, 128)
        g, l = divmod(r, 32)
        want[e] = 0.25 * sc[8 * h + l // 16 + 2 * g] * (int(codes[e]) - 32)
        assert np.array_equal(y, want), e


def test_q6k_extremes():
    codes = np.array([0, 63] * 128, np.uint8)
    y = O.dequant(O.Q6K, _q6k_block(1.0, [1] * 16, codes), 256)
    assert np.array_equal(y, np.array([-32.0, 31.0] * 128, np.float32))
