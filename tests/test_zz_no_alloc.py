"""moe_grouped_experts_static -- the grouped expert chain with its workspace in
a static device array, for callers that cannot allocate -- against
moe_grouped_experts with a caller workspace: captured into a HIP graph and
replayed, outputs, pair rows and h bit for bit on two calls in a row, the
second smaller (the array keeps the first call's contents), and the host-side
refusals."""
import ctypes
import zlib

import numpy as np
import pytest
import torch

from gpu_rig import H, L, stream, synth_experts_dev
from moe_prefetch import _lib
from moe_prefetch.batched import BatchedMoe

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")


def _desc(bm, x, out, n_tok, store, eb, n_store, dt, w, pair_out, h_out, ws, shared=None, kernel_ms=None):
    return _lib.GroupedDesc(bm.offsets.data_ptr(), bm.perm.data_ptr(), w.data_ptr(), x.data_ptr(),
                            _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F32, n_tok, bm.K, bm.E, H,
                            bm.I, dt, None, None, 0, 0, store, eb, n_store, out.data_ptr(), 0,
                            None if pair_out is None else pair_out.data_ptr(),
                            None if h_out is None else h_out.data_ptr(), ws, kernel_ms, shared)


def _call(n_tok, seed, dt, I, shared, rows_out):
    E, K = 128, 8
    rng = np.random.default_rng(seed)
    eb = L().moe_expert_bytes(H, I, dt)
    store = torch.empty((E + 1) * eb, dtype=torch.uint8, device=DEV)
    synth_experts_dev(seed, 2, 0, E + 1, I, dt, store.data_ptr(), eb)       # expert E: the shared one
    xf = torch.empty((n_tok, H), dtype=torch.float32, device=DEV)
    _lib.check(L().moe_synth_vec(seed, 1, 0, n_tok, 3, 1, H, 1.0, xf.data_ptr(), stream()), "x")
    x = xf.to(torch.bfloat16)
    ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, K)).astype(np.float32) + 0.05
    w = torch.from_numpy(w / w.sum(1, keepdims=True)).to(DEV)
    bm = BatchedMoe(n_tok, n_experts=E, n_expert_used=K, intermediate=I)
    bm.dispatch(n_tok, ids=torch.from_numpy(ids).to(DEV), stream=stream())
    sh = store.data_ptr() + E * eb if shared else None
    res = {}
    for kind in ("workspace", "static"):
        out = torch.full((n_tok, H), float("nan"), dtype=torch.float32, device=DEV)
        pair = torch.full((n_tok * K, H), float("nan"), dtype=torch.float32, device=DEV) if rows_out else None
        h = torch.full((n_tok * K, I), float("nan"), dtype=torch.float32, device=DEV) if rows_out else None
        ws = bm.ws.data_ptr() if kind == "workspace" else None
        d = _desc(bm, x, out, n_tok, store.data_ptr(), eb, E, dt, w, pair, h, ws, shared=sh)
        fn = L().moe_grouped_experts if kind == "workspace" else L().moe_grouped_experts_static
        _lib.check(fn(ctypes.byref(d), stream()), kind)
        torch.cuda.synchronize()
        res[kind] = [t.cpu().numpy() for t in (out, pair, h) if t is not None]
    for a, b in zip(res["workspace"], res["static"]):
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
    return bm, x, store, eb, w


def test_static_scratch_under_graph_capture():
    # first in this file: in a fresh process the capture is the first static
    # call on the device, so its scratch-address lookup runs inside the
    # capture.  The captured call is replayed three times, with eager work and
    # synchronisation between the replays; every replay equals the workspace
    # path's result bit for bit
    E, K, I, dt, n_tok = 128, 8, 768, _lib.TYPE_Q4K, 32
    seed = zlib.crc32(b"capture")
    rng = np.random.default_rng(seed)
    eb = L().moe_expert_bytes(H, I, dt)
    store = torch.empty(E * eb, dtype=torch.uint8, device=DEV)
    synth_experts_dev(seed, 4, 0, E, I, dt, store.data_ptr(), eb)
    xf = torch.empty((n_tok, H), dtype=torch.float32, device=DEV)
    _lib.check(L().moe_synth_vec(seed, 1, 0, n_tok, 5, 1, H, 1.0, xf.data_ptr(), stream()), "x")
    x = xf.to(torch.bfloat16)
    ids = np.stack([rng.choice(E, size=K, replace=False) for _ in range(n_tok)]).astype(np.int32)
    w = rng.random((n_tok, K)).astype(np.float32) + 0.05
    w = torch.from_numpy(w / w.sum(1, keepdims=True)).to(DEV)
    bm = BatchedMoe(n_tok, n_experts=E, n_expert_used=K, intermediate=I)
    bm.dispatch(n_tok, ids=torch.from_numpy(ids).to(DEV), stream=stream())
    want = torch.empty((n_tok, H), dtype=torch.float32, device=DEV)
    d = _desc(bm, x, want, n_tok, store.data_ptr(), eb, E, dt, w, None, None, bm.ws.data_ptr())
    _lib.check(L().moe_grouped_experts(ctypes.byref(d), stream()), "workspace")
    torch.cuda.synchronize()
    want_h = want.cpu().numpy()
    out = torch.empty((n_tok, H), dtype=torch.float32, device=DEV)
    ds = _desc(bm, x, out, n_tok, store.data_ptr(), eb, E, dt, w, None, None, None)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    rc = []
    with torch.cuda.graph(g, stream=side, capture_error_mode="thread_local"):
        rc.append(L().moe_grouped_experts_static(ctypes.byref(ds), torch.cuda.current_stream().cuda_stream))
    assert rc == [0], L().moe_last_error()
    for _ in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want_h)
        # eager work between replays: the workspace path again
        _lib.check(L().moe_grouped_experts(ctypes.byref(d), stream()), "workspace")
        torch.cuda.synchronize()
    del g


def test_static_scratch_matches_workspace_two_calls():
    # first call: 64 tokens (batch-64 decode), Q6_K down, I = 768, the shared
    # expert, pair rows and h returned; second call: 17 tokens, Q4_K down,
    # I = 512, no shared expert, pair rows kept in the scratch
    _call(64, zlib.crc32(b"first"), _lib.TYPE_Q6K, 768, True, True)
    _call(17, zlib.crc32(b"second"), _lib.TYPE_Q4K, 512, False, False)


def test_static_scratch_refusals():
    bm, x, store, eb, w = _call(8, 5, _lib.TYPE_Q4K, 768, False, False)
    out = torch.empty((8, H), dtype=torch.float32, device=DEV)
    # a workspace of its own, or timing, is refused
    d = _desc(bm, x, out, 8, store.data_ptr(), eb, 128, _lib.TYPE_Q4K, w, None, None, bm.ws.data_ptr())
    assert L().moe_grouped_experts_static(ctypes.byref(d), stream()) == -1
    ms = (ctypes.c_float * 2)()
    d = _desc(bm, x, out, 8, store.data_ptr(), eb, 128, _lib.TYPE_Q4K, w, None, None, None,
              kernel_ms=ctypes.cast(ms, ctypes.c_void_p))
    assert L().moe_grouped_experts_static(ctypes.byref(d), stream()) == -1
    # a shape whose workspace exceeds the static array: refused before any launch
    n_big = 127
    assert L().moe_grouped_workspace_bytes(n_big, 8, H, 768) > _lib.GROUPED_STATIC_SCRATCH_BYTES
    d = _desc(bm, x, out, n_big, store.data_ptr(), eb, 128, _lib.TYPE_Q4K, w, None, None, None)
    assert L().moe_grouped_experts_static(ctypes.byref(d), stream()) == -1
    assert b"more than the" in L().moe_last_error()
