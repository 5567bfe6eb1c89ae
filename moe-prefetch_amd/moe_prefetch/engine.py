"""The MoE decode engine: slot cache + routed expert kernels, over the C ABI.

`MoeCache` is the llama-moecache runtime of the reference (patches 0006-0008:
llama_moe_cache_init / lookup / step, the observe callback, map and route
traces) rebuilt around an HBM slot pool on one MI355X.  Knob names and
meanings are the reference's: `n_slots` is --moe-expert-cache, `slot_profile`
LLAMA_MOE_SLOT_PROFILE, `max_inserts` --moe-expert-cache-inserts, `admit`
LLAMA_MOE_ADMIT (off | heat | window), `admit_window` / `admit_half` /
`admit_floor` LLAMA_MOE_ADMIT_*, `batch_tables` LLAMA_MOE_BATCH_TABLES,
`early_issue` LLAMA_MOE_EARLY_ISSUE, `cache_prior` LLAMA_MOE_CACHE_PRIOR (the
delta added to resident experts' selection probabilities; `prior_space="logits"`
adds it to the logits instead), `deterministic`
LLAMA_MOE_DETERMINISTIC.  `MoeCache.from_env()` reads those variables.

`device=-1` builds the state machine alone (no GPU, no weights, every upload
completes at once) -- the CPU-testable core.
"""
import ctypes
import os
import sys

import numpy as np

from . import _lib
from ._lib import check, lib


def _ptr(t):
    """Raw address of a torch tensor, numpy array or int (None -> NULL)."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def parse_slot_profile(spec, n_layers, default):
    """"il:slots,il:slots,..." (patches/0006:447-480) -> per-layer slot counts."""
    slots = [default] * n_layers
    if not spec:
        return slots
    for part in spec.split(","):
        il, n = part.split(":")
        il, n = int(il), int(n)
        if 0 <= il < n_layers and n > 0:
            slots[il] = n
    return slots


class MoeCache:
    def __init__(self, n_layers, n_experts=128, n_expert_used=8, hidden=2048, intermediate=768,
                 n_slots=56, slot_profile=None, down_types=None, max_inserts=2, admit="off",
                 admit_window=8, admit_half=64, admit_floor=1.0, batch_tables=False,
                 early_issue=False, cache_prior=0.0, prior_space="probs", deterministic=False, publish=None,
                 device=0):
        if isinstance(slot_profile, str):
            slot_profile = parse_slot_profile(slot_profile, n_layers, n_slots)
        if isinstance(admit, str):
            if admit not in _lib.ADMIT:
                raise ValueError(f"admit must be off | heat | window, not {admit!r}")
            admit = _lib.ADMIT[admit]
        if publish is None:
            publish = "sorted" if deterministic else "fifo"
        self.n_layers, self.n_experts, self.K = n_layers, n_experts, n_expert_used
        self.H, self.I = hidden, intermediate
        self.slots = list(slot_profile) if slot_profile is not None else [n_slots] * n_layers
        self.down_types = list(down_types) if down_types is not None else [_lib.TYPE_Q4K] * n_layers
        self._slots_arr = np.asarray(self.slots, np.int32)
        self._dt_arr = np.asarray(self.down_types, np.int32)
        cfg = _lib.CacheConfig(n_layers, n_experts, n_expert_used, hidden, intermediate, n_slots,
                               self._slots_arr.ctypes.data, self._dt_arr.ctypes.data, max_inserts, admit,
                               admit_window, admit_half, admit_floor, int(batch_tables),
                               int(early_issue), float(cache_prior), int(prior_space == "logits"),
                               _lib.PUBLISH[publish], device)
        h = ctypes.c_void_p()
        check(lib().moe_cache_create(ctypes.byref(cfg), ctypes.byref(h)), "moe_cache_create")
        self.h = h.value
        self.device = device
        self.cache_prior = cache_prior
        self.prior_space = prior_space

    @classmethod
    def from_env(cls, n_layers, n_slots, max_inserts=2, env=None, **shape):
        """Knobs from the reference's environment variables (patches 0006:501-539, 0007:492-506;
        LLAMA_MOE_SIDECAR / LLAMA_MOE_SIDECAR_THREADS, patches 0009:954-960, 1084-1086)."""
        env = os.environ if env is None else env
        g = env.get
        admit = g("LLAMA_MOE_ADMIT", "off") or "off"
        if admit == "0":
            admit = "off"
        c = cls(n_layers, n_slots=n_slots, max_inserts=max_inserts,
                   slot_profile=parse_slot_profile(g("LLAMA_MOE_SLOT_PROFILE"), n_layers, n_slots),
                   admit=admit,
                   admit_window=max(1, int(g("LLAMA_MOE_ADMIT_WINDOW", "8"))),
                   admit_half=max(1, int(g("LLAMA_MOE_ADMIT_HALF", "64"))),
                   admit_floor=float(g("LLAMA_MOE_ADMIT_FLOOR", "1")),
                   batch_tables=int(g("LLAMA_MOE_BATCH_TABLES", "0")) != 0,
                   early_issue=int(g("LLAMA_MOE_EARLY_ISSUE", "0")) != 0,
                   cache_prior=max(0.0, float(g("LLAMA_MOE_CACHE_PRIOR", "0"))),
                   deterministic=int(g("LLAMA_MOE_DETERMINISTIC", "0")) != 0, **shape)
        # a model that fails to load (or that the cache refuses: a PCA block,
        # another expert count) is reported loudly and serving goes on without
        # it (patches/0006:521-556)
        if g("LLAMA_MOE_EVICTOR"):
            from .moep import MoePredictor
            try:
                c.set_evictor(MoePredictor(g("LLAMA_MOE_EVICTOR")))
            except (_lib.MoeError, OSError) as e:
                print(f"moe-cache: EVICTOR NOT LOADED: {e}", file=sys.stderr, flush=True)
        if g("LLAMA_MOE_PREDICTOR"):
            from .moep import MoePredictor
            try:
                c.set_predictor(MoePredictor(g("LLAMA_MOE_PREDICTOR")),
                                predict_top=int(g("LLAMA_MOE_PREDICT_TOP", "3")),
                                online_lr=float(g("LLAMA_MOE_ONLINE_LR", "0")), save_path=g("LLAMA_MOE_PREDICTOR_SAVE"))
            except (_lib.MoeError, OSError) as e:
                print(f"moe-cache: PREDICTOR NOT LOADED: {e}", file=sys.stderr, flush=True)
        if int(g("LLAMA_MOE_SPEC_PROBATION", "0") or "0") != 0:
            c.set_spec_probation(True)
        if int(g("LLAMA_MOE_UPLOAD_STATS", "0") or "0") != 0:
            c.set_upload_stats(True)
        if int(g("LLAMA_MOE_CACHE_FREEZE", "0") or "0") != 0:
            c.freeze()
        if int(g("LLAMA_MOE_SIDECAR", "0") or "0") != 0:
            c.set_sidecar(max(1, int(g("LLAMA_MOE_SIDECAR_THREADS", "8"))))
        c.stream_knobs = None
        if int(g("LLAMA_MOE_STREAM", "0") or "0") != 0:
            # applied by set_streaming() once routers and norm weights are registered
            c.stream_knobs = dict(per_layer=max(1, int(g("LLAMA_MOE_STREAM_PER_LAYER", "4"))),
                                  reserve=max(0, int(g("LLAMA_MOE_STREAM_RESERVE", "2"))),
                                  top_k=min(8, max(1, int(g("LLAMA_MOE_STREAM_TOPK", "8")))),
                                  gbps=max(1.0, float(g("LLAMA_MOE_STREAM_GBPS", "45.7"))),
                                  chunk_kib=max(0, int(g("LLAMA_MOE_STREAM_CHUNK_KIB", "0"))))
        return c

    def close(self):
        if getattr(self, "h", None):
            lib().moe_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    # -- MOEP predictor / evictor (borrowed models: kept referenced here) ----
    def set_predictor(self, model, predict_top=3, online_lr=0.0, save_path=None):
        """LLAMA_MOE_PREDICTOR / _PREDICT_TOP / _ONLINE_LR / _PREDICTOR_SAVE (patches/0006:501-562):
        speculative next-layer uploads from a MoePredictor; turns early issue on."""
        self._pred = model
        check(lib().moe_cache_set_predictor(self.h, model.h if model is not None else None, predict_top,
                                            float(online_lr), save_path.encode() if save_path else None),
              "set_predictor")

    def set_evictor(self, model):
        """LLAMA_MOE_EVICTOR (patches/0006:521-537): victims by the model's lowest score."""
        self._evict = model
        check(lib().moe_cache_set_evictor(self.h, model.h if model is not None else None), "set_evictor")

    def set_spec_probation(self, on=True):
        """LLAMA_MOE_SPEC_PROBATION (patches/0007:503)."""
        check(lib().moe_cache_set_spec_probation(self.h, int(on)), "set_spec_probation")

    def predictor_stats(self):
        n, r, sp = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_uint64()
        check(lib().moe_cache_predictor_stats(self.h, ctypes.byref(n), ctypes.byref(r), ctypes.byref(sp)),
              "predictor_stats")
        return {"n_updates": n.value, "recall_sum": r.value, "n_spec": sp.value}

    # -- weights -----------------------------------------------------------
    def expert_bytes(self, layer):
        return lib().moe_expert_bytes(self.H, self.I, self.down_types[layer])

    def set_host_store(self, layer, ptr):
        check(lib().moe_cache_set_host_store(self.h, layer, _ptr(ptr), self.expert_bytes(layer)),
              "set_host_store")

    def set_router(self, layer, W):
        check(lib().moe_cache_set_router(self.h, layer, _ptr(W)), "set_router")

    def set_shared(self, layer, expert):
        """Always-on shared expert of `layer` (its [up|gate|down] bytes, host or device); None removes it."""
        check(lib().moe_cache_set_shared(self.h, layer, _ptr(expert), self.expert_bytes(layer) if expert is not None
                                         else 0), "set_shared")

    def lookup(self, layer):
        v = _lib.LayerView()
        check(lib().moe_cache_lookup(self.h, layer, ctypes.byref(v)), "lookup")
        return v

    # -- state machine -------------------------------------------------------
    def trace_open(self, route_path=None, map_path=None):
        check(lib().moe_cache_trace_open(self.h, route_path.encode() if route_path else None,
                                         map_path.encode() if map_path else None), "trace_open")

    def observe(self, layer, ids, n_tok=1):
        ids = np.ascontiguousarray(ids, np.int32)
        check(lib().moe_cache_observe(self.h, layer, ids.ctypes.data, ids.size // n_tok, n_tok), "observe")

    def step(self):
        check(lib().moe_cache_step(self.h), "step")

    def requires_sync(self):
        return bool(lib().moe_cache_requires_sync(self.h))

    def frame(self, layer):
        out = np.empty(self.slots[layer], np.int32)
        check(lib().moe_cache_frame(self.h, layer, out.ctypes.data), "frame")
        return out

    def table(self, layer):
        t = np.empty(self.n_experts, np.int32)
        p = np.empty(self.n_experts, np.float32)
        check(lib().moe_cache_table(self.h, layer, t.ctypes.data, p.ctypes.data), "table")
        return t, p

    def stats(self):
        s = _lib.CacheStats()
        check(lib().moe_cache_stats_get(self.h, ctypes.byref(s)), "stats")
        d = {n: getattr(s, n) for n, _ in _lib.CacheStats._fields_}
        seen = d["n_hit"] + d["n_miss"]
        d["hit_rate"] = d["n_hit"] / seen if seen else 0.0
        steps = max(d["n_steps"], 1)
        d["missed_per_token"] = d["n_miss"] / steps
        d["uploaded_per_token"] = d["n_scheduled"] / steps
        return d

    def sync(self):
        check(lib().moe_cache_sync(self.h), "sync")

    def set_upload_stats(self, on=True):
        """LLAMA_MOE_UPLOAD_STATS (patches/0006:689-703): time every upload's copy on
        its stream (stats n_upload_h2d / n_upload_d2d, upload_h2d_us / upload_d2d_us)."""
        check(lib().moe_cache_set_upload_stats(self.h, int(on)), "set_upload_stats")

    def set_decode_path(self, split=0, graph=True):
        """split: 0 one launch for all routed experts, 1 resident/absent experts on
        two forked streams, 2 resident then absent on one stream, 3 router,
        selection, gate/up and down as four launches.  graph: True/1 a captured
        graph per token (tokens of at most 8 layers without CPU-assisted serving
        or streaming launch directly, which is faster), 2 always the graph,
        False/0 direct launches."""
        check(lib().moe_cache_set_decode_path(self.h, int(split), int(graph)), "set_decode_path")

    def set_wait_bound(self, seconds):
        """Bound of every wait inside the fused decode launch (default 0.5 s):
        past it a workgroup gives up and the token fails (MoeError)."""
        check(lib().moe_cache_set_wait_bound(self.h, float(seconds)), "set_wait_bound")

    def set_timing(self, on=True):
        check(lib().moe_cache_set_timing(self.h, int(on)), "set_timing")

    def set_sidecar(self, n_threads, share=(1, 1)):
        """CPU-assisted serving of absent experts (the reference's sidecar):
        n_threads host threads (0 = off) compute the absent experts whose rank
        r among a layer's absent ones has r % den < num, share = (num, den),
        while the GPU runs the rest.  Same outputs and traces."""
        num, den = share
        check(lib().moe_cache_set_sidecar(self.h, int(n_threads), int(num), int(den)), "set_sidecar")

    def set_sidecar_batch(self, share=None):
        """The host's share (num, den) of the absent experts in decode_batch
        (None: the share given to set_sidecar)."""
        num, den = share if share else (0, 0)
        check(lib().moe_cache_set_sidecar_batch(self.h, int(num), int(den)), "set_sidecar_batch")

    def heat_file(self, path):
        """LLAMA_MOE_HEAT_FILE: count observations, save every 512 steps, and
        warm-start from `path` if it holds this cache's dimensions.  Returns
        (records loaded, experts placed).  After set_host_store, before decoding."""
        nr, npl = ctypes.c_int64(), ctypes.c_int64()
        check(lib().moe_cache_heat_file(self.h, str(path).encode(), ctypes.byref(nr), ctypes.byref(npl)),
              "heat_file")
        return nr.value, npl.value

    def freeze(self):
        """LLAMA_MOE_CACHE_FREEZE: no uploads from now on."""
        check(lib().moe_cache_freeze(self.h), "freeze")

    def map_replay(self, path):
        """LLAMA_MOE_MAP_REPLAY: every step ends with the placement recorded in
        `path` (a trace_open map file).  Freezes the cache."""
        check(lib().moe_cache_map_replay(self.h, str(path).encode()), "map_replay")

    # -- router lookahead and just-in-time streaming ------------------------------
    def set_norm(self, layer, g):
        """The RMS-norm weight g_L [H] behind layer L's router input (host array)."""
        g = np.ascontiguousarray(g, np.float32)
        check(lib().moe_cache_set_norm(self.h, layer, g.ctypes.data, g.size), "set_norm")

    def set_streaming(self, on=True, per_layer=4, reserve=2, top_k=8, gbps=45.7, chunk_kib=0):
        """LLAMA_MOE_STREAM: layer L's router launch predicts layers L+1 and L+2
        from L's input; a mover thread copies the predicted absent experts in
        deadline order and flips their table words as they land.  Needs early
        issue, the routers, the host stores and the norm weights (live cache)."""
        cfg = _lib.StreamConfig(int(bool(on)), int(per_layer), int(reserve), int(top_k), float(gbps), int(chunk_kib))
        check(lib().moe_cache_set_streaming(self.h, ctypes.byref(cfg)), "set_streaming")

    def stream_stats(self):
        s = _lib.StreamStats()
        check(lib().moe_cache_stream_stats(self.h, ctypes.byref(s)), "stream_stats")
        out = {n: getattr(s, n) for n, _ in _lib.StreamStats._fields_ if n not in ("lead_us", "lead_n")}
        out["lead_us"] = [s.lead_us[1], s.lead_us[2]]
        out["lead_n"] = [s.lead_n[1], s.lead_n[2]]
        return out

    def observe_gpu(self, layer, ids, gpu_slots):
        ids = np.ascontiguousarray(ids, np.int32)
        gs = np.ascontiguousarray(gpu_slots, np.int32)
        check(lib().moe_cache_observe_gpu(self.h, layer, ids.ctypes.data, gs.ctypes.data, ids.size), "observe_gpu")

    # scripted streaming (host-only caches): the mover's steps one at a time
    def stream_take(self, layer, targets, n, ids, now_ns, t_ns, expert_bytes):
        targets = np.ascontiguousarray(targets, np.int32)
        n = np.ascontiguousarray(n, np.int32)
        ids = np.ascontiguousarray(ids, np.int32).reshape(16)
        r = lib().moe_cache_stream_take(self.h, layer, targets.ctypes.data, n.ctypes.data, ids.ctypes.data,
                                        int(now_ns), int(t_ns), int(expert_bytes))
        if r < 0:
            check(r, "stream_take")
        return r

    def stream_posted(self, layer):
        check(lib().moe_cache_stream_posted(self.h, layer), "stream_posted")

    def stream_next(self, free_at_ns, hold_after=-1):
        c = _lib.StreamChunk()
        r = lib().moe_cache_stream_next(self.h, int(free_at_ns), int(hold_after), ctypes.byref(c))
        if r < 0:
            check(r, "stream_next")
        return (c.job, c.offset, c.len, bool(c.last)) if r == 1 else None

    def stream_land(self, job):
        check(lib().moe_cache_stream_land(self.h, job), "stream_land")

    def stream_job(self, job):
        li, e = ctypes.c_int32(), ctypes.c_int32()
        slot = lib().moe_cache_stream_job(self.h, job, ctypes.byref(li), ctypes.byref(e))
        return (li.value, e.value, slot) if slot >= 0 else None

    def sidecar_log(self, max_rows=65536):
        """[rows][3] float32: host wait us, host compute us, experts computed,
        per served layer since the last call."""
        out = np.empty((max_rows, 3), np.float32)
        n = lib().moe_cache_sidecar_log(self.h, out.ctypes.data, max_rows)
        return out[:max(n, 0)].copy()

    def set_staging(self, on=True):
        """Uploads of experts a decode token just read from the pinned store are
        copied from an HBM staging area instead of over PCIe (default on)."""
        check(lib().moe_cache_set_staging(self.h, int(on)), "set_staging")

    def kernel_times(self):
        t = _lib.KernelTimes()
        check(lib().moe_cache_kernel_times(self.h, ctypes.byref(t)), "kernel_times")
        return {n: getattr(t, n) for n, _ in _lib.KernelTimes._fields_}

    # -- decode ---------------------------------------------------------------
    def decode_layer(self, layer, x, out, bias=None, ids=None, w=None, stream=None):
        check(lib().moe_decode_layer(self.h, layer, _ptr(x), _ptr(bias), _ptr(out), _ptr(ids), _ptr(w),
                                     _ptr(stream)), "decode_layer")

    def decode_batch(self, x, out, bias=None, stream=None, ids_out=None):
        """x [L, n_tok, H] and out [L, n_tok, H] on the device (bias [L, n_tok, E] or None).
        Returns the routed ids [L, n_tok, K] (host) after the step has been applied."""
        n_tok = x.shape[1]
        ids = ids_out if ids_out is not None else np.empty((self.n_layers, n_tok, self.K), np.int32)
        check(lib().moe_decode_batch(self.h, _ptr(x), _ptr(bias), _ptr(out), n_tok, ids.ctypes.data, _ptr(stream)),
              "decode_batch")
        return ids

    def decode_token(self, x, out, bias=None, stream=None, ids_out=None):
        """x [L, H] and out [L, H] on the device (bias [L, E] or None).  Returns the
        routed ids [L, K] (host) after the step has been applied."""
        ids = ids_out if ids_out is not None else np.empty((self.n_layers, self.K), np.int32)
        check(lib().moe_decode_token(self.h, _ptr(x), _ptr(bias), _ptr(out), ids.ctypes.data, _ptr(stream)),
              "decode_token")
        return ids
