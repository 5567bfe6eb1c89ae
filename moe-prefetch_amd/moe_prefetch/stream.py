"""Router lookahead and the just-in-time copy planner, over the C ABI.

`Planner` is the mover's earliest-deadline-first copy planner (moe_planner,
patches/0010-team-and-streaming.patch:777-909) exported for inspection;
`route_ahead` runs the batch-1 router with the lookahead of one or two target
layers (k_moe_ahead_scores / k_moe_ahead_post, 0010:382-474) and returns the
posted candidates.  Streaming itself is MoeCache.set_streaming.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib

DROP_NONE, DROP_LATE, DROP_POSTED = 0, 1, 2


class Planner:
    def __init__(self, chunk_bytes=512 * 1024):
        self.h = lib().moe_planner_create(int(chunk_bytes))
        if not self.h:
            raise _lib.MoeError("moe_planner_create failed")

    def close(self):
        if getattr(self, "h", None):
            lib().moe_planner_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def offer(self, target, expert, nbytes, deadline_ns):
        return lib().moe_planner_offer(self.h, int(target), int(expert), int(nbytes), int(deadline_ns))

    def posted(self, target):
        lib().moe_planner_posted(self.h, int(target))

    def next(self, free_at_ns, bytes_per_ns, hold_after=-1):
        c = _lib.StreamChunk()
        if not lib().moe_planner_next(self.h, int(free_at_ns), float(bytes_per_ns), int(hold_after), ctypes.byref(c)):
            return None
        return c.job, c.offset, c.len, bool(c.last)

    def reset(self):
        lib().moe_planner_reset(self.h)

    def size(self):
        return lib().moe_planner_size(self.h)

    def get(self, i):
        j = _lib.PlannerJob()
        if lib().moe_planner_get(self.h, int(i), ctypes.byref(j)) != 0:
            raise IndexError(i)
        return {n: getattr(j, n) for n, _ in _lib.PlannerJob._fields_}

    def counters(self):
        out = np.zeros(4, np.uint64)
        lib().moe_planner_counters(self.h, out.ctypes.data)
        return dict(zip(("offered", "dup", "drop_late", "drop_posted"), (int(v) for v in out)))


def route_ahead(desc, W, r, tbl, dummy, top_k=8, stream=None):
    """desc: a RouteDesc of a batch-1 router GEMV (n_tok 1).  W, r, tbl: lists
    (one or two targets) of device pointers.  Returns [(ids...)] per target."""
    nt = len(W)
    a = _lib.AheadDesc()
    a.n_targets, a.top_k = nt, int(top_k)
    for t in range(nt):
        a.W[t], a.r[t], a.tbl[t], a.dummy[t] = W[t], r[t], tbl[t], int(dummy[t])
    n = np.zeros(2, np.int32)
    ids = np.zeros((2, 8), np.int32)
    check(lib().moe_route_ahead(ctypes.byref(desc), ctypes.byref(a), n.ctypes.data, ids.ctypes.data, stream),
          "moe_route_ahead")
    return [ids[t, :n[t]].copy() for t in range(nt)]
