"""The batch oracle (or_moe_tokens, which the batched GPU path is compared with) against
the per-token oracle it restates: same expert chain, same k-order combine, so
the two agree bit for bit; an id outside the store contributes zero."""
import numpy as np
import pytest

import moe_prefetch
from moe_prefetch import _lib
from oracle import oracle as O

H = 2048


@pytest.mark.parametrize("dt", [_lib.TYPE_Q4K, _lib.TYPE_Q6K])
def test_moe_tokens_equals_moe_layer(dt):
    I, n_store, T, K = 256, 6, 5, 3
    L = moe_prefetch.lib()
    eb = L.moe_expert_bytes(H, I, dt)
    store = np.zeros(n_store * eb, np.uint8)
    _lib.check(L.moe_synth_experts_host(3, 1, 0, n_store, H, I, dt, 0.02, store.ctypes.data, eb, 4), "synth")
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, H)).astype(np.float32)
    ids = rng.integers(0, n_store, size=(T, K)).astype(np.int32)
    ids[3, 1] = n_store          # outside the store
    ids[4, 0] = -1
    w = rng.random((T, K)).astype(np.float32)
    out, h = O.moe_tokens(H, I, dt, store, eb, n_store, ids, w, x, n_threads=4, want_h=True)
    for t in range(T):
        if t < 3:
            want = O.moe_layer(H, I, dt, [store[e * eb:(e + 1) * eb] for e in ids[t]], w[t], x[t])
            assert np.array_equal(out[t], want), t
        else:
            acc = None
            for k in range(K):
                e = ids[t, k]
                if 0 <= e < n_store:
                    y, hh = O.expert_chain(H, I, dt, store[e * eb:(e + 1) * eb], x[t])
                    v = np.float32(w[t, k]) * y
                    assert np.array_equal(h[t, k], hh)
                else:
                    v = np.zeros(H, np.float32)
                    assert not h[t, k].any()
                acc = v if acc is None else acc + v
            assert np.array_equal(out[t], acc), t
