"""GPU parity of the batched path (prefill chunks, decode at batch > 1) through
the C ABI against the oracle on the same seeded inputs.

  moe_dispatch         counts, offsets and the (token, k)-stable permutation
                       bit-exact (uniform, skewed, all-one-expert, ragged,
                       several 4096-pair passes, E = 64/128/256, ids outside
                       [0, E) dropped)
  moe_quant_rows       Q8_K values, scales and group sums bit-exact (f32, bf16,
                       zero rows, ties of the largest magnitude)
  moe_route (logits)   ids / weights / probabilities from given logits
                       bit-exact, with and without a bias
  moe_grouped_experts  every token's output and every pair's SwiGLU
                       activations within 1e-3 relative L2 of the ggml-style
                       oracle, and in fact bit-exact (Q4_K and Q6_K down,
                       intermediate 768/512/256, batch 1..512, tokens crowding
                       a few experts into several passes, experts in HBM slots
                       / a pinned host store / nowhere, super-block sums past
                       2**24)
"""
import zlib

import numpy as np
import pytest
import torch

from gpu_rig import H, L, Pinned, stream, synth_experts_dev
from moe_prefetch import _lib
from moe_prefetch.batched import BatchedMoe
from oracle import oracle as O

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")
TOL = 1e-3   # relative L2 against the oracle, per token / per pair


def t_(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def ref_dispatch(ids, E):
    flat = np.asarray(ids, np.int64).reshape(-1)
    valid = (flat >= 0) & (flat < E)
    counts = np.bincount(flat[valid], minlength=E).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    idx = np.flatnonzero(valid)
    return counts, offsets, idx[np.argsort(flat[valid], kind="stable")].astype(np.int32)


def gpu_dispatch(ids, E):
    T, K = ids.shape
    d_ids = t_(ids.astype(np.int32))
    counts = torch.full((E,), -7, dtype=torch.int32, device=DEV)
    offsets = torch.full((E + 1,), -7, dtype=torch.int32, device=DEV)
    perm = torch.full((max(T * K, 1),), -7, dtype=torch.int32, device=DEV)
    _lib.check(L().moe_dispatch(d_ids.data_ptr(), T, K, E, counts.data_ptr(), offsets.data_ptr(),
                                perm.data_ptr(), stream()), "dispatch")
    torch.cuda.synchronize()
    return counts.cpu().numpy(), offsets.cpu().numpy(), perm.cpu().numpy()


DISPATCH_CASES = {
    "uniform_512x8_e128": (512, 8, 128, "uniform"),
    "single_token": (1, 8, 128, "uniform"),
    "batch16_k9_e256": (16, 9, 256, "uniform"),
    "two_passes_1024x8": (1024, 8, 128, "uniform"),
    "max_pairs_8191x8": (8191, 8, 128, "zipf"),
    "one_expert": (300, 8, 64, "one"),
    "skewed_e64": (777, 6, 64, "zipf"),
}


@pytest.mark.parametrize("case", list(DISPATCH_CASES))
def test_dispatch_bit_exact(case):
    T, K, E, kind = DISPATCH_CASES[case]
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    if kind == "uniform":
        ids = rng.integers(0, E, size=(T, K))
    elif kind == "one":
        ids = np.full((T, K), 5)
    else:
        p = 1.0 / np.arange(1, E + 1) ** 1.2
        ids = rng.choice(E, size=(T, K), p=p / p.sum())
    ids = ids.astype(np.int32)
    c, o, p = gpu_dispatch(ids, E)
    oc, oo, op = O.dispatch(ids, E)
    assert np.array_equal(c, oc) and np.array_equal(o, oo)
    assert np.array_equal(p[:T * K], op)


def test_dispatch_drops_ids_outside_range():
    rng = np.random.default_rng(3)
    ids = rng.integers(-3, 131, size=(200, 8)).astype(np.int32)
    c, o, p = gpu_dispatch(ids, 128)
    rc, ro, rp = ref_dispatch(ids, 128)
    assert np.array_equal(c, rc) and np.array_equal(o, ro)
    assert np.array_equal(p[:ro[-1]], rp)


@pytest.mark.parametrize("src", ["f32", "bf16"])
@pytest.mark.parametrize("n", [2048, 768])
def test_quant_rows_bit_exact(src, n):
    rng = np.random.default_rng(n)
    rows = 37
    x = (rng.standard_normal((rows, n)) * rng.uniform(0.01, 3, size=(rows, 1))).astype(np.float32)
    x[3] = 0.0                                     # all-zero blocks
    x[5, :256] = 0.0
    x[5, 7], x[5, 9] = -2.5, 2.5                   # tie of the largest magnitude: first index wins
    x[6, 300], x[6, 301] = 4.0, -4.0
    xd = t_(x)
    if src == "bf16":
        xd = xd.to(torch.bfloat16)
        x = xd.float().cpu().numpy()
    q16 = torch.empty((rows, n), dtype=torch.int16, device=DEV)
    d = torch.empty((rows, n // 256), dtype=torch.float32, device=DEV)
    bs = torch.empty((rows, n // 16), dtype=torch.int16, device=DEV)
    st = _lib.DTYPE_BF16 if src == "bf16" else _lib.DTYPE_F32
    _lib.check(L().moe_quant_rows(xd.data_ptr(), st, rows, n, q16.data_ptr(), d.data_ptr(), bs.data_ptr(),
                                  stream()), "quant_rows")
    torch.cuda.synchronize()
    qv = q16.cpu().view(torch.float16).float().numpy()
    bv = bs.cpu().view(torch.float16).float().numpy()
    dv = d.cpu().numpy()
    for r in range(rows):
        blocks = O.quant_q8k(x[r]).reshape(-1, 292)
        for b in range(n // 256):
            blk = blocks[b]
            assert dv[r, b].tobytes() == blk[:4].tobytes(), (r, b)
            assert np.array_equal(qv[r, 256 * b:256 * (b + 1)], blk[4:260].view(np.int8).astype(np.float32)), (r, b)
            assert np.array_equal(bv[r, 16 * b:16 * (b + 1)], blk[260:292].view(np.int16).astype(np.float32)), (r, b)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("E,K", [(128, 8), (256, 8), (64, 6)])
def test_route_given_logits_bit_exact(E, K, bias):
    T = 96
    lg = torch.empty((T, E), dtype=torch.float32, device=DEV)
    _lib.check(L().moe_synth_vec(5, 2, 0, T, 0, 1, E, 1.0, lg.data_ptr(), stream()), "logits")
    b = None
    if bias:
        b = t_(np.random.default_rng(E).standard_normal((T, E)).astype(np.float32) * 0.3)
    bm = BatchedMoe(T, n_experts=E, n_expert_used=K)
    ids, w = bm.route(T, logits=lg, bias=b, stream=stream())
    torch.cuda.synchronize()
    lh = lg.cpu().numpy()
    assert lh.min() >= 0.0 and lh.max() < 1.0
    bh = None if b is None else b.cpu().numpy()
    gi, gw = ids.cpu().numpy(), w.cpu().numpy()
    for t in range(T):
        l_ = lh[t] if bh is None else lh[t] + bh[t]
        oi, ow, _ = O.route_logits(l_, K)
        assert np.array_equal(gi[t], oi), t
        assert gw[t].tobytes() == ow.tobytes(), t


# ---- grouped experts ---------------------------------------------------------
class Store:
    """n experts of one layer in HBM (device generator)."""

    def __init__(self, n, I, dt, seed=42, layer=3):
        self.n, self.I, self.dt = n, I, dt
        self.eb = L().moe_expert_bytes(H, I, dt)
        self.t = torch.empty(n * self.eb, dtype=torch.uint8, device=DEV)
        synth_experts_dev(seed, layer, 0, n, I, dt, self.t.data_ptr(), self.eb)
        torch.cuda.synchronize()
        self.host = self.t.cpu().numpy()


def routing(rng, T, K, E, kind):
    if kind == "uniform":
        ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(T)])
    elif kind == "repeat":  # pair i = t*K + k routed to expert i % 2, as the reference's repeated-ids mode
        ids = (np.arange(T * K) % 2).reshape(T, K)   # (cpp/test-moe-rows.cpp:60-67, mode 3)
    elif kind == "dups":    # ids drawn with replacement from 5 experts: repeats inside a token, uneven
        hot = rng.choice(E, size=5, replace=False)
        ids = np.stack([rng.choice(hot, size=K, replace=True) for _ in range(T)])
    elif kind == "edges":   # exact counts at the edges of the two-pass chunks' M tiles: 48 pairs (a
        # second pass of 16, its second tile empty), 49 (17), 33, 64, 65 (a second chunk of 1), 32, 17
        # and 16; the other experts share the rest (ids repeat inside tokens)
        fixed = [48, 49, 33, 64, 65, 32, 17, 16]
        flat = np.concatenate([np.full(c, e) for e, c in enumerate(fixed)] +
                              [rng.choice(np.arange(len(fixed), E), size=T * K - sum(fixed))])
        ids = rng.permutation(flat).reshape(T, K)
        assert [int((ids == e).sum()) for e in range(len(fixed))] == fixed
    else:   # crowd: most tokens share a handful of experts (several passes of 64 pairs)
        hot = rng.choice(E, size=K + 2, replace=False)
        ids = np.stack([rng.choice(hot, size=K, replace=False) if rng.random() < 0.8 else
                        rng.choice(E, size=K, replace=False) for _ in range(T)])
    w = rng.random((T, K)).astype(np.float32) + 0.05
    return ids.astype(np.int32), (w / w.sum(1, keepdims=True)).astype(np.float32)


def rel_l2(a, b):
    return float(np.linalg.norm(a.astype(np.float64) - b) / max(np.linalg.norm(b.astype(np.float64)), 1e-30))


def run_grouped(store, T, K, E, ids, w, x_dtype, table=None, slot_pool=None, slot_bytes=0, n_slots=0,
                store_ptr=None, n_store=None, seed=0, x_host=None):
    if x_host is None:
        xf = torch.empty((T, H), dtype=torch.float32, device=DEV)
        _lib.check(L().moe_synth_vec(seed, 1, 0, T, 7, 1, H, 1.0, xf.data_ptr(), stream()), "x")
    else:
        xf = t_(x_host.astype(np.float32))
    x = xf.to(torch.bfloat16) if x_dtype == "bf16" else xf
    bm = BatchedMoe(T, n_experts=E, n_expert_used=K, intermediate=store.I)
    d_ids, d_w = t_(ids), t_(w)
    bm.dispatch(T, ids=d_ids, stream=stream())
    out = torch.empty((T, H), dtype=torch.float32, device=DEV)
    h_out = torch.empty((T * K, store.I), dtype=torch.float32, device=DEV)
    pair = torch.empty((T * K, H), dtype=torch.float32, device=DEV)
    bm.experts(x, out, T, store.t.data_ptr() if store_ptr is None else store_ptr, store.eb,
               store.n if n_store is None else n_store, store.dt, w=d_w, table=table, slot_pool=slot_pool,
               slot_bytes=slot_bytes, n_slots=n_slots, pair_out=pair, h_out=h_out, stream=stream())
    torch.cuda.synchronize()
    xh = x.float().cpu().numpy()
    return out.cpu().numpy(), h_out.cpu().numpy(), pair.cpu().numpy(), bm.perm[:T * K].cpu().numpy(), xh


GROUPED_CASES = {
    "q4k_i768_t64": (_lib.TYPE_Q4K, 768, 64, 128, "uniform", "bf16"),
    "q6k_i768_t64": (_lib.TYPE_Q6K, 768, 64, 128, "uniform", "bf16"),
    "q4k_i512_t33_f32": (_lib.TYPE_Q4K, 512, 33, 128, "uniform", "f32"),
    "q6k_i512_t1": (_lib.TYPE_Q6K, 512, 1, 128, "uniform", "bf16"),
    "q4k_i768_t512": (_lib.TYPE_Q4K, 768, 512, 128, "uniform", "bf16"),
    "q6k_i768_t200_crowded": (_lib.TYPE_Q6K, 768, 200, 128, "crowd", "bf16"),
    "q4k_i256_t150_e64_crowded": (_lib.TYPE_Q4K, 256, 150, 64, "crowd", "f32"),
    "q4k_i768_t24_repeated_ids": (_lib.TYPE_Q4K, 768, 24, 128, "repeat", "bf16"),
    "q6k_i512_t40_ids_with_replacement": (_lib.TYPE_Q6K, 512, 40, 128, "dups", "f32"),
    # at most 8 pairs per expert on average: one 16-row M tile a pass
    "q4k_i256_t20_one_tile": (_lib.TYPE_Q4K, 256, 20, 128, "uniform", "bf16"),
    "q4k_i512_t100_crowded_one_tile": (_lib.TYPE_Q4K, 512, 100, 128, "crowd", "f32"),
    # more than 16 pairs per expert on average: chunks of two 32-pair passes
    "q6k_i768_t512": (_lib.TYPE_Q6K, 768, 512, 128, "uniform", "bf16"),
    "q6k_i512_t300_crowded": (_lib.TYPE_Q6K, 512, 300, 128, "crowd", "f32"),
    "q6k_i256_t300_e64": (_lib.TYPE_Q6K, 256, 300, 64, "uniform", "bf16"),
    "q4k_i768_t200_e32": (_lib.TYPE_Q4K, 768, 200, 32, "uniform", "bf16"),
    "q4k_i512_t300": (_lib.TYPE_Q4K, 512, 300, 128, "uniform", "f32"),
    "q4k_i768_t300_tile_edges": (_lib.TYPE_Q4K, 768, 300, 128, "edges", "bf16"),
    "q6k_i512_t300_tile_edges": (_lib.TYPE_Q6K, 512, 300, 128, "edges", "f32"),
    "q6k_i512_t200_e32": (_lib.TYPE_Q6K, 512, 200, 32, "uniform", "f32"),
    "q6k_i256_t400_e32_crowded": (_lib.TYPE_Q6K, 256, 400, 32, "crowd", "bf16"),
}


@pytest.mark.parametrize("case", list(GROUPED_CASES))
def test_grouped_experts_vs_oracle(case):
    dt, I, T, E, kind, xt = GROUPED_CASES[case]
    K = 8
    rng = np.random.default_rng(zlib.crc32(case.encode()))
    store = Store(E, I, dt)
    ids, w = routing(rng, T, K, E, kind)
    out, h_out, pair, perm, xh = run_grouped(store, T, K, E, ids, w, xt)
    want, want_h = O.moe_tokens(H, I, dt, store.host, store.eb, E, ids, w, xh, n_threads=16, want_h=True)
    assert all(np.linalg.norm(want[t]) > 0 for t in range(T))
    worst = max(rel_l2(out[t], want[t]) for t in range(T))
    # h in dispatch order: position j holds pair perm[j]
    hw = want_h.reshape(T * K, I)[perm]
    assert all(np.linalg.norm(hw[j]) > 0 for j in range(T * K))
    worst_h = max(rel_l2(h_out[j], hw[j]) for j in range(T * K))
    n_exact = sum(np.array_equal(out[t], want[t]) for t in range(T))
    h_exact = sum(np.array_equal(h_out[j], hw[j]) for j in range(T * K))
    print(f"{case}: worst rel-L2 out {worst:.3e}, h {worst_h:.3e}; bit-exact tokens {n_exact}/{T}, "
          f"pairs {h_exact}/{T * K}")
    assert worst < TOL, worst
    assert worst_h < TOL, worst_h
    # integer products are exact on the matrix cores and the fp32 scale follows
    # the CPU chain's order: the values are the oracle's bit for bit
    assert n_exact == T and h_exact == T * K
    # the per-pair rows summed over k in order give out exactly
    s = pair.reshape(T, K, H)
    acc = s[:, 0].copy()
    for k in range(1, K):
        acc = acc + s[:, k]
    assert np.array_equal(acc, out)


class LargeSumStore:
    """Experts whose Q4_K super-block sums pass 2**24 against near-uniform
    activations: every six-bit scale and min 63 (scale bytes 0xFF), nibbles
    8..15, d = 2**-14, dmin = 0.  A Q6_K down matrix gets scales of the
    largest magnitude (-128..-120, 120..127) and quants 0..3 (q - 32 near -32)."""

    def __init__(self, n, I, dt, seed=5):
        rng = np.random.default_rng(seed)
        self.n, self.I, self.dt = n, I, dt
        self.eb = L().moe_expert_bytes(H, I, dt)
        n_up, n_dn = 2 * I * (H // 256), H * (I // 256)
        d = np.frombuffer(np.float16(2.0 ** -14).tobytes(), np.uint8)
        experts = []
        for _ in range(n):
            q4 = np.zeros((n_up + (n_dn if dt == _lib.TYPE_Q4K else 0), 144), np.uint8)
            q4[:, 0:2] = d
            q4[:, 4:16] = 0xFF
            q4[:, 16:] = rng.integers(8, 16, size=(len(q4), 128)) | (rng.integers(8, 16, size=(len(q4), 128)) << 4)
            parts = [q4.reshape(-1)]
            if dt == _lib.TYPE_Q6K:
                q6 = np.zeros((n_dn, 210), np.uint8)
                q6[:, :128] = rng.integers(0, 4, size=(n_dn, 128)) | (rng.integers(0, 4, size=(n_dn, 128)) << 4)
                sc = rng.integers(120, 129, size=(n_dn, 16)) * rng.choice([-1, 1], size=(n_dn, 16))
                q6[:, 192:208] = np.clip(sc, -128, 127).astype(np.int8).view(np.uint8)
                q6[:, 208:210] = d
                parts.append(q6.reshape(-1))
            e = np.concatenate(parts)
            assert e.size == self.eb
            experts.append(e)
        self.host = np.concatenate(experts)
        self.t = t_(self.host)


@pytest.mark.parametrize("dt,T", [(_lib.TYPE_Q4K, 8), (_lib.TYPE_Q4K, 24), (_lib.TYPE_Q4K, 48),
                                  (_lib.TYPE_Q4K, 96), (_lib.TYPE_Q6K, 48), (_lib.TYPE_Q6K, 96)],
                         ids=["q4k_t8", "q4k_t24", "q4k_t48", "q4k_t96", "q6k_t48", "q6k_t96"])
def test_grouped_experts_sums_past_2_24(dt, T):
    """Super-block integer sums beyond fp32's exact integers (2**24): the
    grouped kernels still equal ggml's (float)sumi bit for bit.  16 experts,
    top-8: 4, 12, 24 and 48 pairs per expert (one-tile passes, one-pass and
    two-pass chunks)."""
    E, K, I = 16, 8, 768
    rng = np.random.default_rng(77 + T)
    store = LargeSumStore(E, I, dt)
    x = (1.0 - 0.06 * rng.random((T, H))).astype(np.float32)      # Q8_K codes -127 .. -119
    ids, w = routing(rng, T, K, E, "uniform")
    # the sums really pass 2**24: gate row 0 of expert ids[0, 0] against token 0
    q8 = O.quant_q8k(x[0]).reshape(H // 256, 292)[:, 4:260].view(np.int8).astype(np.int64)
    row = store.host[ids[0, 0] * store.eb:][:(H // 256) * 144].reshape(H // 256, 144)
    nib = np.stack([row[:, 16:] & 15, row[:, 16:] >> 4], 1)            # [block][lo/hi][128]
    q = np.concatenate([np.concatenate([nib[:, 0, 32 * j:32 * j + 32], nib[:, 1, 32 * j:32 * j + 32]], 1)
                        for j in range(4)], 1).astype(np.int64)        # element order of ggml's Q4_K
    sums = (63 * q * q8).sum(1)
    assert np.abs(sums).max() > 2 ** 24, np.abs(sums).max()
    out, h_out, pair, perm, xh = run_grouped(store, T, K, E, ids, w, "f32", x_host=x)
    want, want_h = O.moe_tokens(H, I, dt, store.host, store.eb, E, ids, w, xh, n_threads=16, want_h=True)
    hw = want_h.reshape(T * K, I)[perm]
    assert np.isfinite(want).all() and np.abs(hw).min() > 0
    n_h = sum(np.array_equal(h_out[j], hw[j]) for j in range(T * K))
    n_out = sum(np.array_equal(out[t], want[t]) for t in range(T))
    print(f"max |super-block sum| {np.abs(sums).max()}; bit-exact pairs {n_h}/{T * K}, tokens {n_out}/{T}")
    assert n_h == T * K and n_out == T


def test_grouped_experts_slots_pinned_and_absent():
    """Experts resident in an HBM slot pool, the rest read from a pinned host
    store, ids past the store contributing zero."""
    dt, I, T, E, K = _lib.TYPE_Q4K, 768, 48, 128, 8
    rng = np.random.default_rng(5)
    store = Store(E, I, dt, layer=1)
    pinned = Pinned(E * store.eb)
    pinned.arr[:] = store.host
    n_slots = 20
    slot_bytes = (store.eb + 255) // 256 * 256
    pool = torch.zeros(n_slots * slot_bytes, dtype=torch.uint8, device=DEV)
    table = np.full(E, n_slots, np.int32)
    resident = rng.choice(E - 10, size=n_slots, replace=False)
    for s, e in enumerate(resident):
        table[e] = s
        pool[s * slot_bytes:s * slot_bytes + store.eb] = store.t[e * store.eb:(e + 1) * store.eb]
    n_store = E - 10                        # the last 10 ids are in no store and not resident
    table[E - 3] = 0 if table[E - 3] == n_slots else table[E - 3]   # one of them resident after all
    ids, w = routing(rng, T, K, E, "uniform")
    ids[0, :3] = [E - 1, E - 2, E - 3]
    try:
        out, h_out, pair, perm, xh = run_grouped(store, T, K, E, ids, w, "bf16", table=t_(table),
                                                 slot_pool=pool.data_ptr(), slot_bytes=slot_bytes,
                                                 n_slots=n_slots, store_ptr=pinned.dev, n_store=n_store)
    finally:
        pinned.free()
    # what each id reads: the bytes its slot holds when the table maps it, else
    # the store (ids below n_store), else nothing (expert E of the padded store)
    src = np.array([resident[table[e]] if table[e] < n_slots else (e if e < n_store else E) for e in range(E)])
    flat_store = np.concatenate([store.host, np.zeros(store.eb, np.uint8)])
    want = O.moe_tokens(H, I, dt, flat_store, store.eb, E, src[ids], w, xh, n_threads=16)
    assert all(np.linalg.norm(want[t]) > 0 for t in range(T))
    worst = max(rel_l2(out[t], want[t]) for t in range(T))
    print(f"slots/pinned/absent: worst rel-L2 {worst:.3e}")
    assert worst < TOL, worst
    assert np.array_equal(out, want)
    # the absent ids of token 0 contribute nothing: its output equals the sum over its other experts
    assert src[E - 1] == E and src[E - 2] == E


def test_combine_accumulates_in_k_order():
    T, K = 9, 8
    rng = np.random.default_rng(2)
    rows = rng.standard_normal((T * K, H)).astype(np.float32)
    base = rng.standard_normal((T, H)).astype(np.float32)
    out = t_(base)
    _lib.check(L().moe_combine(t_(rows).data_ptr(), T, K, H, out.data_ptr(), 1, stream()), "combine")
    s = rows.reshape(T, K, H)
    acc = s[:, 0].copy()
    for k in range(1, K):
        acc = acc + s[:, k]
    assert np.array_equal(out.cpu().numpy(), base + acc)
