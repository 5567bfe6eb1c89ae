"""ctypes view of liboracle.so -- the CPU restatement of the MoE decode path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always to check the product's results (or as the
CPU baseline timed beside the GPU), never as a product path.  See oracle.h for what each function
restates and what pins it.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

Q4K, Q6K = 12, 14
QK = 256
Q4K_BYTES, Q6K_BYTES, Q8K_BYTES = 144, 210, 292


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


class Knobs(ctypes.Structure):
    _fields_ = [("max_inserts", ctypes.c_int32), ("admit_mode", ctypes.c_int32),
                ("admit_window", ctypes.c_int32), ("admit_half", ctypes.c_int32),
                ("admit_floor", ctypes.c_float), ("batch_tables", ctypes.c_int32),
                ("early_issue", ctypes.c_int32), ("cache_prior", ctypes.c_float),
                ("deterministic", ctypes.c_int32)]


class Stats(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "n_steps", "clock", "n_hit", "n_miss", "n_uploads", "n_scheduled", "n_published",
        "n_admit_ok", "n_admit_denied", "n_table_flushes")]


class Chunk(ctypes.Structure):
    _fields_ = [("job", ctypes.c_int), ("offset", ctypes.c_size_t), ("len", ctypes.c_size_t), ("last", ctypes.c_int)]


class PlannerJob(ctypes.Structure):
    _fields_ = [("target", ctypes.c_int), ("expert", ctypes.c_int32), ("bytes", ctypes.c_size_t),
                ("sent", ctypes.c_size_t), ("deadline_ns", ctypes.c_uint64), ("dropped", ctypes.c_int),
                ("drop", ctypes.c_int)]


class MoepLists(ctypes.Structure):
    _fields_ = [("ids", ctypes.c_void_p * 4), ("n", ctypes.c_int * 4)]


STREAM_STATS = ("records", "offered", "landed", "in_time", "late", "unused", "dropped_late", "dropped_posted",
                "not_sent", "gpu_miss", "bytes")
DROP_NONE, DROP_LATE, DROP_POSTED = 0, 1, 2

P = ctypes.c_void_p
I32 = ctypes.c_int32
I64 = ctypes.c_int64
F32 = ctypes.c_float


def _declare(L):
    def d(name, res, *args):
        f = getattr(L, name)
        f.restype = res
        f.argtypes = list(args)
    d("or_h2f", F32, ctypes.c_uint16)
    d("or_f2h", ctypes.c_uint16, F32)
    d("or_dequant_q4k", None, P, P, I64)
    d("or_dequant_q6k", None, P, P, I64)
    d("or_quant_q8k", None, P, P, I64)
    d("or_dequant_q8k", None, P, P, I64)
    d("or_dot_q4k_q8k", F32, ctypes.c_int, P, P)
    d("or_dot_q6k_q8k", F32, ctypes.c_int, P, P)
    d("or_dot_deq_f64", ctypes.c_double, ctypes.c_int, ctypes.c_int, P, P)
    d("or_expf", F32, F32)
    d("or_route", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P, P, P, P)
    d("or_route_space", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, ctypes.c_int, P, P, P,
      P, P)
    d("or_route_logits", None, ctypes.c_int, ctypes.c_int, P, P, P, P, P)
    d("or_expert_chain", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, P, P)
    d("or_moe_layer", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P,
      ctypes.c_int)
    d("or_expert_bytes", ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int)
    d("or_moe_tokens", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P,
      ctypes.c_size_t, ctypes.c_int, P, P, P, P, P, ctypes.c_int)
    d("or_dispatch", None, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P)
    d("or_cache_create", P, ctypes.c_int, ctypes.c_int, P, ctypes.POINTER(Knobs))
    d("or_cache_destroy", None, P)
    d("or_cache_trace_open", ctypes.c_int, P, ctypes.c_char_p, ctypes.c_char_p)
    d("or_cache_observe", None, P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int)
    d("or_cache_step", None, P)
    d("or_cache_hold_job", None, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_uint64)
    d("or_cache_frame", None, P, ctypes.c_int, P)
    d("or_cache_table", None, P, ctypes.c_int, P, P)
    d("or_cache_stats", None, P, ctypes.POINTER(Stats))
    d("or_cache_heat_file", ctypes.c_int, P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_longlong),
      ctypes.POINTER(ctypes.c_longlong))
    d("or_cache_freeze", None, P)
    d("or_cache_map_replay", ctypes.c_int, P, ctypes.c_char_p)
    d("or_cache_replay_error", ctypes.c_int, P)
    d("or_ahead", ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P, I32, P, P)
    d("or_planner_create", P, ctypes.c_size_t)
    d("or_planner_destroy", None, P)
    d("or_planner_reset", None, P)
    d("or_planner_offer", ctypes.c_int, P, ctypes.c_int, I32, ctypes.c_size_t, ctypes.c_uint64)
    d("or_planner_posted", None, P, ctypes.c_int)
    d("or_planner_next", ctypes.c_int, P, ctypes.c_uint64, ctypes.c_double, ctypes.c_int, ctypes.POINTER(Chunk))
    d("or_planner_size", ctypes.c_int, P)
    d("or_planner_get", None, P, ctypes.c_int, ctypes.POINTER(PlannerJob))
    d("or_planner_counters", None, P, P)
    d("or_cache_stream_enable", ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_double, ctypes.c_size_t)
    d("or_cache_stream_take", ctypes.c_int, P, ctypes.c_int, P, P, P, ctypes.c_uint64, ctypes.c_uint64,
      ctypes.c_size_t)
    d("or_cache_stream_posted", None, P, ctypes.c_int)
    d("or_cache_stream_next", ctypes.c_int, P, ctypes.c_uint64, ctypes.c_int, ctypes.POINTER(Chunk))
    d("or_cache_stream_land", None, P, ctypes.c_int)
    d("or_cache_stream_job", ctypes.c_int, P, ctypes.c_int, P, P)
    d("or_cache_observe_gpu", None, P, ctypes.c_int, P, P, ctypes.c_int)
    d("or_cache_stream_stats", None, P, P)
    d("or_moep_load", P, ctypes.c_char_p)
    d("or_moep_free", None, P)
    d("or_moep_n_expert", ctypes.c_int, P)
    d("or_moep_has_layer", ctypes.c_int, P, ctypes.c_int)
    d("or_moep_score", None, P, ctypes.c_int, ctypes.POINTER(MoepLists), P)
    d("or_moep_top", ctypes.c_int, P, P, ctypes.c_int, P)
    d("or_moep_update", F32, P, ctypes.c_int, ctypes.POINTER(MoepLists), P, ctypes.c_int, F32)
    d("or_cache_set_predictor", None, P, P, ctypes.c_int, F32)
    d("or_cache_set_evictor", None, P, P)
    d("or_cache_set_spec_probation", None, P, ctypes.c_int)
    d("or_cache_predictor_stats", None, P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double),
      ctypes.POINTER(ctypes.c_uint64))


def _p(a):
    return None if a is None else a.ctypes.data


# ---- codecs ---------------------------------------------------------------
def h2f(h):
    return lib().or_h2f(int(h))


def f2h(f):
    return lib().or_f2h(float(f))


def dequant(wtype, blocks, n):
    y = np.empty(n, np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    (lib().or_dequant_q4k if wtype == Q4K else lib().or_dequant_q6k)(_p(blocks), _p(y), n)
    return y


def quant_q8k(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size // QK * Q8K_BYTES, np.uint8)
    lib().or_quant_q8k(_p(x), _p(out), x.size)
    return out


def dequant_q8k(blocks, n):
    y = np.empty(n, np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    lib().or_dequant_q8k(_p(blocks), _p(y), n)
    return y


def dot(wtype, n, w_row, q8):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    f = lib().or_dot_q4k_q8k if wtype == Q4K else lib().or_dot_q6k_q8k
    return f(n, _p(w_row), _p(q8))


def dot_f64(wtype, n, w_row, q8):
    w_row = np.ascontiguousarray(w_row, dtype=np.uint8)
    q8 = np.ascontiguousarray(q8, dtype=np.uint8)
    return lib().or_dot_deq_f64(wtype, n, _p(w_row), _p(q8))


# ---- router ---------------------------------------------------------------
def expf(x):
    return lib().or_expf(float(x))


def route(W, x, K, bias=None, prior=None, table=None, prior_on_logits=False):
    """W [E, H] f32, x [H] f32 -> (ids[K] i32, w[K] f32, slots[K] or None, probs[E])."""
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    E, H = W.shape
    ids = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    probs = np.empty(E, np.float32)
    slots = np.empty(K, np.int32) if table is not None else None
    bias = None if bias is None else np.ascontiguousarray(bias, np.float32)
    prior = None if prior is None else np.ascontiguousarray(prior, np.float32)
    table = None if table is None else np.ascontiguousarray(table, np.int32)
    lib().or_route_space(E, H, K, _p(W), _p(x), _p(bias), _p(prior), int(prior_on_logits), _p(table),
                         _p(ids), _p(w), _p(slots), _p(probs))
    return ids, w, slots, probs


def route_logits(logits, K, prior=None):
    logits = np.ascontiguousarray(logits, np.float32)
    E = logits.size
    ids = np.empty(K, np.int32)
    w = np.empty(K, np.float32)
    probs = np.empty(E, np.float32)
    prior = None if prior is None else np.ascontiguousarray(prior, np.float32)
    lib().or_route_logits(E, K, _p(logits), _p(prior), _p(ids), _p(w), _p(probs))
    return ids, w, probs


def ahead(W, x, r, table, dummy, k=8):
    """Router lookahead: the k best experts of W [E, H] applied to x * r, best
    first, lower id on a tie; those with table[e] == dummy.  -> (ids, scores)."""
    W = np.ascontiguousarray(W, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    r = np.ascontiguousarray(r, np.float32)
    table = np.ascontiguousarray(table, np.int32)
    E, H = W.shape
    ids = np.empty(k, np.int32)
    scores = np.empty(E, np.float32)
    n = lib().or_ahead(E, H, k, _p(W), _p(x), _p(r), _p(table), int(dummy), _p(scores), _p(ids))
    if n < 0:
        raise ValueError("or_ahead: bad sizes")
    return ids[:n].copy(), scores


class Planner:
    """Earliest-deadline-first copy planner (moe_planner)."""

    def __init__(self, chunk_bytes=512 * 1024):
        self.h = lib().or_planner_create(chunk_bytes)

    def close(self):
        if self.h:
            lib().or_planner_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def offer(self, target, expert, nbytes, deadline_ns):
        return lib().or_planner_offer(self.h, target, expert, nbytes, deadline_ns)

    def posted(self, target):
        lib().or_planner_posted(self.h, target)

    def next(self, free_at_ns, bytes_per_ns, hold_after=-1):
        c = Chunk()
        if not lib().or_planner_next(self.h, free_at_ns, bytes_per_ns, hold_after, ctypes.byref(c)):
            return None
        return c.job, c.offset, c.len, bool(c.last)

    def reset(self):
        lib().or_planner_reset(self.h)

    def size(self):
        return lib().or_planner_size(self.h)

    def get(self, i):
        j = PlannerJob()
        lib().or_planner_get(self.h, i, ctypes.byref(j))
        return {n: getattr(j, n) for n, _ in PlannerJob._fields_}

    def counters(self):
        out = np.zeros(4, np.uint64)
        lib().or_planner_counters(self.h, _p(out))
        return dict(zip(("offered", "dup", "drop_late", "drop_posted"), (int(v) for v in out)))


# ---- expert chain -----------------------------------------------------------
def expert_bytes(H, I, down_type):
    return lib().or_expert_bytes(H, I, down_type)


def expert_chain(H, I, down_type, expert, x):
    """expert: uint8 array of one expert's [up | gate | down] bytes."""
    expert = np.ascontiguousarray(expert, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    upb = I * (H // QK) * Q4K_BYTES
    y = np.empty(H, np.float32)
    h = np.empty(I, np.float32)
    base = expert.ctypes.data
    lib().or_expert_chain(H, I, down_type, base, base + upb, base + 2 * upb, _p(x), _p(y), _p(h))
    return y, h


def moe_layer(H, I, down_type, experts, w, x, n_threads=1):
    """experts: list of K uint8 arrays (or raw addresses); out = sum_k w_k y_k."""
    K = len(experts)
    ptrs = (ctypes.c_void_p * K)(*[e if isinstance(e, int) else e.ctypes.data for e in experts])
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(H, np.float32)
    lib().or_moe_layer(H, I, down_type, K, ctypes.cast(ptrs, ctypes.c_void_p), _p(w), _p(x),
                       _p(out), n_threads)
    return out


def moe_tokens(H, I, down_type, store, expert_bytes, n_store, ids, w, x, n_threads=8, want_h=False):
    """Batch oracle: store is a uint8 array (or raw address) of [n_store][expert_bytes];
    ids/w [T][K]; x [T][H] f32.  Returns out [T][H] (and h [T][K][I])."""
    ids = np.ascontiguousarray(ids, np.int32)
    T, K = ids.shape
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty((T, H), np.float32)
    h = np.empty((T, K, I), np.float32) if want_h else None
    base = store if isinstance(store, int) else store.ctypes.data
    lib().or_moe_tokens(H, I, down_type, T, K, base, expert_bytes, n_store, _p(ids), _p(w), _p(x), _p(out),
                        _p(h) if want_h else None, n_threads)
    return (out, h) if want_h else out


def dispatch(ids, E):
    ids = np.ascontiguousarray(ids, np.int32)
    T, K = ids.shape
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    perm = np.empty(T * K, np.int32)
    lib().or_dispatch(T, K, E, _p(ids), _p(counts), _p(offsets), _p(perm))
    return counts, offsets, perm


# ---- state machine ----------------------------------------------------------
ADMIT = {"off": 0, "heat": 1, "window": 2}


class Cache:
    def __init__(self, slots, n_experts=128, max_inserts=2, admit="off", admit_window=8,
                 admit_half=64, admit_floor=1.0, batch_tables=False, early_issue=False,
                 cache_prior=0.0, deterministic=False):
        self.slots = np.ascontiguousarray(slots, np.int32)
        self.n_layers = self.slots.size
        self.n_experts = n_experts
        k = Knobs(max_inserts, ADMIT[admit], admit_window, admit_half, admit_floor,
                  int(batch_tables), int(early_issue), cache_prior, int(deterministic))
        self.h = lib().or_cache_create(self.n_layers, n_experts, _p(self.slots), ctypes.byref(k))

    def close(self):
        if self.h:
            lib().or_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def trace_open(self, route_path=None, map_path=None):
        r = lib().or_cache_trace_open(self.h, route_path.encode() if route_path else None,
                                      map_path.encode() if map_path else None)
        if r != 0:
            raise OSError("trace open failed")

    def observe(self, layer, ids, n_tok=1):
        ids = np.ascontiguousarray(ids, np.int32)
        lib().or_cache_observe(self.h, layer, _p(ids), ids.size // n_tok, n_tok)

    def step(self):
        lib().or_cache_step(self.h)

    def heat_file(self, path):
        """LLAMA_MOE_HEAT_FILE: returns (records loaded, experts placed)."""
        nr, npl = ctypes.c_longlong(), ctypes.c_longlong()
        if lib().or_cache_heat_file(self.h, path.encode(), ctypes.byref(nr), ctypes.byref(npl)) != 0:
            raise OSError(path)
        return nr.value, npl.value

    def freeze(self):
        lib().or_cache_freeze(self.h)

    def map_replay(self, path):
        if lib().or_cache_map_replay(self.h, path.encode()) != 0:
            raise ValueError(f"map replay refused: {path}")

    def replay_error(self):
        return lib().or_cache_replay_error(self.h)

    def hold_job(self, layer, expert, slot, sched_step):
        lib().or_cache_hold_job(self.h, layer, expert, slot, sched_step)

    def frame(self, layer):
        out = np.empty(int(self.slots[layer]), np.int32)
        lib().or_cache_frame(self.h, layer, _p(out))
        return out

    def table(self, layer):
        t = np.empty(self.n_experts, np.int32)
        p = np.empty(self.n_experts, np.float32)
        lib().or_cache_table(self.h, layer, _p(t), _p(p))
        return t, p

    def stats(self):
        s = Stats()
        lib().or_cache_stats(self.h, ctypes.byref(s))
        return {n: getattr(s, n) for n, _ in Stats._fields_}

    # ---- MOEP predictor / evictor hooks (Moep models, borrowed) ----
    def set_predictor(self, model, predict_top=3, online_lr=0.0):
        self._pred = model
        lib().or_cache_set_predictor(self.h, model.h if model else None, predict_top, online_lr)

    def set_evictor(self, model):
        self._evict = model
        lib().or_cache_set_evictor(self.h, model.h if model else None)

    def set_spec_probation(self, on=True):
        lib().or_cache_set_spec_probation(self.h, int(on))

    def predictor_stats(self):
        n, r, sp = ctypes.c_uint64(), ctypes.c_double(), ctypes.c_uint64()
        lib().or_cache_predictor_stats(self.h, ctypes.byref(n), ctypes.byref(r), ctypes.byref(sp))
        return {"n_updates": n.value, "recall_sum": r.value, "n_spec": sp.value}

    # ---- just-in-time streaming ----
    def stream_enable(self, per_layer=4, reserve=2, gbps=45.7, chunk_bytes=512 * 1024):
        if lib().or_cache_stream_enable(self.h, per_layer, reserve, gbps, chunk_bytes) != 0:
            raise ValueError("streaming needs early issue and batched tables, no replay/freeze/deterministic, "
                             "and no open map trace")

    def stream_take(self, layer, targets, n, ids, now_ns, t_ns, expert_bytes):
        targets = np.ascontiguousarray(targets, np.int32)
        n = np.ascontiguousarray(n, np.int32)
        ids = np.ascontiguousarray(ids, np.int32).reshape(16)
        return lib().or_cache_stream_take(self.h, layer, _p(targets), _p(n), _p(ids), now_ns, t_ns, expert_bytes)

    def stream_posted(self, layer):
        lib().or_cache_stream_posted(self.h, layer)

    def stream_next(self, free_at_ns, hold_after=-1):
        c = Chunk()
        if not lib().or_cache_stream_next(self.h, free_at_ns, hold_after, ctypes.byref(c)):
            return None
        return c.job, c.offset, c.len, bool(c.last)

    def stream_land(self, job):
        lib().or_cache_stream_land(self.h, job)

    def stream_job(self, job):
        li, e = ctypes.c_int32(), ctypes.c_int32()
        slot = lib().or_cache_stream_job(self.h, job, ctypes.byref(li), ctypes.byref(e))
        return (li.value, e.value, slot) if slot >= 0 else None

    def observe_gpu(self, layer, ids, gslots):
        ids = np.ascontiguousarray(ids, np.int32)
        gslots = np.ascontiguousarray(gslots, np.int32)
        lib().or_cache_observe_gpu(self.h, layer, _p(ids), _p(gslots), ids.size)

    def stream_stats(self):
        out = np.zeros(11, np.uint64)
        lib().or_cache_stream_stats(self.h, _p(out))
        return dict(zip(STREAM_STATS, (int(v) for v in out)))


# ---- the MOEP predictor / evictor, restated (moep.c) ----
class Moep:
    """The oracle's MOEP model (cpp/moe-predictor.cpp restated)."""

    def __init__(self, path):
        self.h = lib().or_moep_load(str(path).encode())
        if not self.h:
            raise ValueError(f"oracle cannot load MOEP file {path}")
        self.n_expert = lib().or_moep_n_expert(self.h)

    def close(self):
        if getattr(self, "h", None):
            lib().or_moep_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @staticmethod
    def _lists(keep, ids):
        l = MoepLists()
        for b, name in enumerate(("prev", "cur", "below", "self_prev")):
            v = ids.get(name)
            if v is None or len(v) == 0:
                l.ids[b], l.n[b] = None, 0
                continue
            a = np.ascontiguousarray(v, np.int32)
            keep.append(a)
            l.ids[b], l.n[b] = a.ctypes.data, a.size
        return l

    def has_layer(self, layer):
        return bool(lib().or_moep_has_layer(self.h, layer))

    def score(self, layer, **ids):
        keep = []
        l = self._lists(keep, ids)
        out = np.empty(self.n_expert, np.float32)
        lib().or_moep_score(self.h, layer, ctypes.byref(l), out.ctypes.data)
        return out

    def top_k(self, scores, k=8):
        s = np.ascontiguousarray(scores, np.float32)
        out = np.empty(max(k, 0), np.int32)
        n = lib().or_moep_top(self.h, s.ctypes.data, k, out.ctypes.data)
        return out[:n]

    def update(self, layer, truth, lr, **ids):
        keep = []
        l = self._lists(keep, ids)
        t = np.ascontiguousarray(truth, np.int32)
        return lib().or_moep_update(self.h, layer, ctypes.byref(l), t.ctypes.data, t.size, lr)


# ---- the reference's own MOEP predictor (oracle/_ref, built where the reference is) ----
REF_PREDICTOR = os.path.join(HERE, "_ref", "libref_predictor.so")
_ref = None


def ref_predictor_lib():
    """ctypes handle of _ref/libref_predictor.so, or None when it is not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PREDICTOR):
        L = ctypes.CDLL(REF_PREDICTOR)
        I = ctypes.c_int
        L.rp_load.restype, L.rp_load.argtypes = P, [ctypes.c_char_p, ctypes.c_char_p, I]
        L.rp_free.restype, L.rp_free.argtypes = None, [P]
        L.rp_has_layer.restype, L.rp_has_layer.argtypes = I, [P, I]
        L.rp_score.restype, L.rp_score.argtypes = None, [P, I, P, I, P, I, P, I, P, I, P]
        L.rp_top_k.restype, L.rp_top_k.argtypes = I, [P, P, I, P]
        L.rp_update.restype, L.rp_update.argtypes = F32, [P, I, P, I, P, I, P, I, P, I, P, I, F32]
        L.rp_save.restype, L.rp_save.argtypes = I, [P, ctypes.c_char_p, ctypes.c_char_p, I]
        _ref = L
    return _ref


class RefPredictor:
    """The reference's moe_predictor (checker only)."""

    def __init__(self, path):
        L = ref_predictor_lib()
        err = ctypes.create_string_buffer(512)
        self.h = L.rp_load(str(path).encode(), err, 512)
        if not self.h:
            raise ValueError(err.value.decode())
        self.L = L

    def close(self):
        if getattr(self, "h", None):
            self.L.rp_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    @staticmethod
    def _args(keep, ids):
        out = []
        for name in ("prev", "cur", "below", "self_prev"):
            v = ids.get(name)
            if v is None or len(v) == 0:
                out += [None, 0]
            else:
                a = np.ascontiguousarray(v, np.int32)
                keep.append(a)
                out += [a.ctypes.data, a.size]
        return out

    def has_layer(self, layer):
        return bool(self.L.rp_has_layer(self.h, layer))

    def score(self, layer, n_expert, **ids):
        keep = []
        out = np.empty(n_expert, np.float32)
        self.L.rp_score(self.h, layer, *self._args(keep, ids), out.ctypes.data)
        return out

    def top_k(self, scores, k=8):
        s = np.ascontiguousarray(scores, np.float32)
        out = np.empty(k, np.int32)
        n = self.L.rp_top_k(self.h, s.ctypes.data, k, out.ctypes.data)
        return out[:n]

    def update(self, layer, truth, lr, **ids):
        keep = []
        t = np.ascontiguousarray(truth, np.int32)
        return self.L.rp_update(self.h, layer, *self._args(keep, ids), t.ctypes.data, t.size, lr)

    def save(self, path):
        err = ctypes.create_string_buffer(512)
        if self.L.rp_save(self.h, str(path).encode(), err, 512) != 0:
            raise OSError(err.value.decode())
