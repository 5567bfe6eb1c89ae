"""Drop-in `ExpertCache`: a GPU-resident per-layer expert cache fed by async
host->HBM copies (the API of the reference's src/prefetch_engine.py:45-168).

Same constructor and methods, same meaning:
  ExpertCache(n_layers, n_experts, capacity, device="cuda", bytes_per_expert)
  .prefetch(layer, ids) -> number of copies started
  .query(layer, ids)    -> (hit, late, miss) lists; an expert whose copy is
                           still in flight is `late`, not a hit
  .admit(layer, ids)    -> bring computed misses in (moves the bytes)
  .sync(), .vram_bytes(), .summary() with expert_hit_rate, late_rate, gb_moved
Per-layer LRU over `capacity` slots, slots taken from the free list first
(lowest index first, as list.pop() on [0..capacity) pops the last), then the
least recently used expert is evicted.

The slabs live in one HBM pool of the native library (moe_pool_*); every copy
runs on the pool's own non-blocking HIP stream from pinned host staging and
records a per-slot event, which `query` polls.  `staging` is a numpy view of
that pinned memory, [n_experts, bytes_per_expert] uint8 -- the bytes a layer's
experts are uploaded from (one buffer shared by all layers, as in the
reference prototype, where content does not matter to transfer timing).
"""
import ctypes
from collections import OrderedDict

import numpy as np

from ._lib import check, lib

EXPERT_MIB = 2.92
EXPERT_BYTES = int(EXPERT_MIB * 1024 * 1024)


def _device_index(device):
    if isinstance(device, int):
        return device
    s = str(device)
    if ":" in s:
        return int(s.split(":")[1])
    return 0


class ExpertCache:
    """Per-layer LRU cache of experts resident in HBM, with async refill."""

    def __init__(self, n_layers, n_experts, capacity, device="cuda", bytes_per_expert=EXPERT_BYTES):
        self.n_layers = n_layers
        self.n_experts = n_experts
        self.capacity = capacity
        self.device = device
        self.bytes_per_expert = bytes_per_expert
        h = ctypes.c_void_p()
        check(lib().moe_pool_create(n_layers, capacity, bytes_per_expert, _device_index(device),
                                    ctypes.byref(h)), "moe_pool_create")
        self._pool = h.value
        n = n_experts * bytes_per_expert
        self._staging_ptr = lib().moe_host_alloc(n)
        if not self._staging_ptr:
            raise MemoryError(lib().moe_last_error().decode())
        self.staging = np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(self._staging_ptr)).reshape(
            n_experts, bytes_per_expert)
        self.maps = [OrderedDict() for _ in range(n_layers)]    # expert -> slot, LRU first
        self.free = [list(range(capacity)) for _ in range(n_layers)]
        self.pending = set()                                    # (layer, expert) copies not yet seen done
        self.stats = {"hits": 0, "misses": 0, "late": 0, "fetches": 0, "bytes": 0, "evictions": 0}

    def close(self):
        if getattr(self, "_pool", None):
            lib().moe_pool_destroy(self._pool)
            self._pool = None
        if getattr(self, "_staging_ptr", None):
            self.staging = None
            lib().moe_host_free(self._staging_ptr)
            self._staging_ptr = None

    def __del__(self):
        self.close()

    # -- internals ---------------------------------------------------------
    def _slot_for(self, layer, expert):
        m = self.maps[layer]
        if expert in m:
            m.move_to_end(expert)
            return m[expert], False
        if self.free[layer]:
            slot = self.free[layer].pop()
        else:
            old, slot = m.popitem(last=False)
            self.pending.discard((layer, old))
            self.stats["evictions"] += 1
        m[expert] = slot
        return slot, True

    def _fetch(self, layer, expert):
        slot, _ = self._slot_for(layer, expert)
        src = self._staging_ptr + expert * self.bytes_per_expert
        check(lib().moe_pool_copy(self._pool, layer, slot, src, self.bytes_per_expert), "moe_pool_copy")
        self.pending.add((layer, expert))
        self.stats["fetches"] += 1
        self.stats["bytes"] += self.bytes_per_expert

    # -- public ------------------------------------------------------------
    def prefetch(self, layer, expert_ids):
        """Start async copies for `expert_ids` into layer's cache. Returns count."""
        started = 0
        for e in expert_ids:
            e = int(e)
            if e in self.maps[layer]:
                self.maps[layer].move_to_end(e)
                continue
            self._fetch(layer, e)
            started += 1
        return started

    def query(self, layer, expert_ids):
        """Which of `expert_ids` are usable now, without waiting: (hit, late, miss)."""
        hit, late, miss = [], [], []
        for e in expert_ids:
            e = int(e)
            m = self.maps[layer]
            if e not in m:
                miss.append(e)
                continue
            if (layer, e) in self.pending:
                r = lib().moe_pool_ready(self._pool, layer, m[e])
                if r < 0:
                    check(r, "moe_pool_ready")
                if r == 0:
                    late.append(e)
                    continue
                self.pending.discard((layer, e))
            m.move_to_end(e)
            hit.append(e)
        self.stats["hits"] += len(hit)
        self.stats["misses"] += len(miss)
        self.stats["late"] += len(late)
        return hit, late, miss

    def admit(self, layer, expert_ids):
        """A miss was computed elsewhere; bring it in so the next token can use it."""
        for e in expert_ids:
            e = int(e)
            if e in self.maps[layer]:
                self.maps[layer].move_to_end(e)
                continue
            self._fetch(layer, e)

    def sync(self):
        check(lib().moe_pool_sync(self._pool), "moe_pool_sync")

    def slot_ptr(self, layer, slot):
        """Device address of a slot (no counterpart in the prototype, whose slabs were tensors)."""
        return lib().moe_pool_slot_ptr(self._pool, layer, slot)

    def vram_bytes(self):
        return self.n_layers * self.capacity * self.bytes_per_expert

    def summary(self):
        s = dict(self.stats)
        total = s["hits"] + s["misses"] + s["late"]
        s["expert_hit_rate"] = s["hits"] / max(total, 1)
        s["late_rate"] = s["late"] / max(total, 1)
        s["gb_moved"] = s["bytes"] / 1e9
        return s
