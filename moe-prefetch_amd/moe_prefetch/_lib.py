"""ctypes binding of libmoeprefetch.so (include/moe_prefetch.h).

The library is built in-tree by moe-prefetch_amd/build.py; importing this
module never falls back to anything else: a missing library raises.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmoeprefetch.so")

MOE_OK = 0
MOE_ERR_ARG, MOE_ERR_HIP, MOE_ERR_NOMEM, MOE_ERR_STATE = -1, -2, -3, -4
TYPE_Q4K, TYPE_Q6K = 12, 14
DTYPE_F32, DTYPE_BF16 = 0, 1
# the static workspace of moe_grouped_experts_static (MOE_GROUPED_STATIC_SCRATCH_BYTES)
GROUPED_STATIC_SCRATCH_BYTES = 16 << 20
ADMIT = {"off": 0, "heat": 1, "window": 2}
PUBLISH = {"fifo": 0, "sorted": 1, "live": 2}

P = ctypes.c_void_p
I32 = ctypes.c_int32
U64 = ctypes.c_uint64
F32 = ctypes.c_float
SZ = ctypes.c_size_t


class MoeError(RuntimeError):
    pass


class RouteDesc(ctypes.Structure):
    _fields_ = [("W", P), ("x", P), ("bias", P), ("prior", P), ("table", P), ("dummy", I32),
                ("prior_on_logits", I32), ("E", I32), ("H", I32), ("K", I32), ("n_tok", I32),
                ("ids", P), ("w", P), ("slots", P), ("probs", P), ("q8x", P), ("workspace", P),
                ("logits", P)]


class ExpertsDesc(ctypes.Structure):
    _fields_ = [("ids", P), ("slots", P), ("w", P), ("slot_pool", P), ("slot_bytes", U64),
                ("n_slots", I32), ("host_store", P), ("expert_bytes", U64), ("n_experts", I32),
                ("q8x", P), ("out", P),
                ("accumulate", I32), ("H", I32), ("I", I32), ("K", I32), ("down_type", I32),
                ("workspace", P), ("shared", P)]


class GroupedDesc(ctypes.Structure):
    _fields_ = [("offsets", P), ("perm", P), ("w", P), ("x", P), ("x_type", I32),
                ("n_tok", I32), ("K", I32), ("E", I32), ("H", I32), ("I", I32), ("down_type", I32),
                ("table", P), ("slot_pool", P), ("slot_bytes", U64), ("n_slots", I32),
                ("store", P), ("expert_bytes", U64), ("n_store", I32),
                ("out", P), ("accumulate", I32), ("pair_out", P), ("h_out", P), ("workspace", P),
                ("kernel_ms", P), ("shared", P)]


class CacheConfig(ctypes.Structure):
    _fields_ = [("n_layers", I32), ("n_experts", I32), ("n_expert_used", I32),
                ("hidden", I32), ("intermediate", I32), ("n_slots", I32),
                ("slot_profile", P), ("down_type", P), ("max_inserts", I32), ("admit_mode", I32),
                ("admit_window", I32), ("admit_half", I32), ("admit_floor", F32),
                ("batch_tables", I32), ("early_issue", I32), ("cache_prior", F32),
                ("prior_on_logits", I32), ("publish", I32), ("device", I32)]


class CacheStats(ctypes.Structure):
    _fields_ = [(n, U64) for n in ("n_steps", "clock", "n_hit", "n_miss", "n_uploads", "n_scheduled",
                                   "n_copied", "n_published", "n_admit_ok", "n_admit_denied",
                                   "n_table_flushes", "bytes_uploaded")] + \
               [("publication_wait_us", ctypes.c_double), ("n_staged", ctypes.c_uint64),
                ("n_cpu_served", ctypes.c_uint64), ("sidecar_wait_us", ctypes.c_double),
                ("sidecar_cpu_us", ctypes.c_double), ("host_boundary_us", ctypes.c_double),
                ("n_evicted", ctypes.c_uint64), ("n_upload_h2d", ctypes.c_uint64), ("n_upload_d2d", ctypes.c_uint64),
                ("upload_h2d_us", ctypes.c_double), ("upload_d2d_us", ctypes.c_double)]


class LayerView(ctypes.Structure):
    _fields_ = [("il", I32), ("n_slots", I32), ("n_experts", I32), ("down_type", I32),
                ("slot_bytes", U64), ("expert_bytes", U64), ("slot_pool", P), ("dev_table", P),
                ("prior", P), ("host_store", P), ("router", P)]


class KernelTimes(ctypes.Structure):
    _fields_ = [(n, ctypes.c_double) for n in ("route_ms", "gateup_hbm_ms", "down_hbm_ms", "gateup_host_ms",
                                               "down_host_ms")] + \
               [(n, U64) for n in ("n_layers", "gateup_hbm_bytes", "down_hbm_bytes", "gateup_host_bytes",
                                   "down_host_bytes")] + \
               [("layer_ms", ctypes.c_double), ("layer_hbm_bytes", U64), ("layer_host_bytes", U64)] + \
               [(n, ctypes.c_double) for n in ("grouped_gateup_ms", "grouped_down_ms")] + \
               [(n, U64) for n in ("grouped_launches", "grouped_pairs", "grouped_gateup_hbm_bytes",
                                   "grouped_down_hbm_bytes", "grouped_gateup_host_bytes", "grouped_down_host_bytes")]


class StreamConfig(ctypes.Structure):
    _fields_ = [("on", I32), ("per_layer", I32), ("reserve", I32), ("top_k", I32), ("gbps", ctypes.c_double),
                ("chunk_kib", I32)]


class StreamStats(ctypes.Structure):
    _fields_ = [(n, U64) for n in ("records", "offered", "landed", "in_time", "late", "unused", "dropped_late",
                                   "dropped_posted", "not_sent", "gpu_miss", "bytes")] + \
               [("lead_us", ctypes.c_double * 3), ("lead_n", U64 * 3), ("tau_us", ctypes.c_double),
                ("failed", I32)]


class StreamChunk(ctypes.Structure):
    _fields_ = [("job", I32), ("offset", U64), ("len", U64), ("last", I32)]


class AheadDesc(ctypes.Structure):
    _fields_ = [("n_targets", I32), ("top_k", I32), ("W", P * 2), ("r", P * 2), ("tbl", P * 2),
                ("dummy", I32 * 2)]


class PlannerJob(ctypes.Structure):
    _fields_ = [("target", I32), ("expert", I32), ("bytes", U64), ("sent", U64), ("deadline_ns", U64),
                ("dropped", I32), ("drop", I32)]


class PredictorInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_expert", "n_layers", "feat_dim", "top_k", "d_model", "n_comp",
                                               "n_present")] + \
               [(n, I32) for n in ("has_pca", "off_pca", "off_prev", "off_cur", "off_below", "off_self_prev")]


class PredictorLists(ctypes.Structure):
    _fields_ = [("ids", P * 4), ("n", I32 * 4)]


# name -> (restype, argtypes); mirrors include/moe_prefetch.h one to one
SIGNATURES = {
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_abi_version": (ctypes.c_int, []),
    "moe_host_alloc": (P, [SZ]),
    "moe_host_free": (ctypes.c_int, [P]),
    "moe_host_device_ptr": (P, [P]),
    "moe_device_alloc": (P, [SZ]),
    "moe_device_free": (ctypes.c_int, [P]),
    "moe_device_synchronize": (ctypes.c_int, []),
    "moe_memcpy": (ctypes.c_int, [P, P, SZ]),
    "moe_memcpy_h2d_batch": (ctypes.c_bool, [ctypes.c_int, P, P, P, ctypes.c_int]),
    "moe_synth_experts": (ctypes.c_int, [U64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_int, F32, P, SZ, P]),
    "moe_synth_experts_host": (ctypes.c_int, [U64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int, F32, P, SZ, ctypes.c_int]),
    "moe_synth_vec": (ctypes.c_int, [U64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                     ctypes.c_int, ctypes.c_int, F32, P, P]),
    "moe_synth_vec_host": (ctypes.c_int, [U64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, F32, P]),
    "moe_expert_bytes": (SZ, [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "moe_route_workspace_bytes": (SZ, [ctypes.c_int, ctypes.c_int]),
    "moe_experts_workspace_bytes": (SZ, [ctypes.c_int, ctypes.c_int]),
    "moe_cpu_experts_tokens": (ctypes.c_int, [P, ctypes.c_int, P, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P,
                                               ctypes.c_int]),
    "moe_cpu_experts": (ctypes.c_int, [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P,
                                       ctypes.c_int, ctypes.c_int]),
    "moe_cpu_has_vnni": (ctypes.c_int, []),
    "moe_route": (ctypes.c_int, [ctypes.POINTER(RouteDesc), P]),
    "moe_experts": (ctypes.c_int, [ctypes.POINTER(ExpertsDesc), P]),
    "moe_cache_create": (ctypes.c_int, [ctypes.POINTER(CacheConfig), ctypes.POINTER(P)]),
    "moe_cache_destroy": (ctypes.c_int, [P]),
    "moe_cache_set_host_store": (ctypes.c_int, [P, ctypes.c_int, P, SZ]),
    "moe_cache_set_router": (ctypes.c_int, [P, ctypes.c_int, P]),
    "moe_cache_set_shared": (ctypes.c_int, [P, ctypes.c_int, P, SZ]),
    "moe_cache_lookup": (ctypes.c_int, [P, ctypes.c_int, ctypes.POINTER(LayerView)]),
    "moe_cache_trace_open": (ctypes.c_int, [P, ctypes.c_char_p, ctypes.c_char_p]),
    "moe_cache_observe": (ctypes.c_int, [P, ctypes.c_int, P, ctypes.c_int, ctypes.c_int]),
    "moe_cache_step": (ctypes.c_int, [P]),
    "moe_cache_requires_sync": (ctypes.c_int, [P]),
    "moe_cache_frame": (ctypes.c_int, [P, ctypes.c_int, P]),
    "moe_cache_table": (ctypes.c_int, [P, ctypes.c_int, P, P]),
    "moe_cache_stats_get": (ctypes.c_int, [P, ctypes.POINTER(CacheStats)]),
    "moe_cache_sync": (ctypes.c_int, [P]),
    "moe_cache_set_upload_stats": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_sidecar_selftest": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_double,
                                                  ctypes.POINTER(ctypes.c_int)]),
    "moe_cache_set_timing": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_set_decode_path": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int]),
    "moe_cache_set_wait_bound": (ctypes.c_int, [P, ctypes.c_double]),
    "moe_cache_set_staging": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_set_sidecar": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "moe_cache_set_sidecar_batch": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int]),
    "moe_cache_sidecar_log": (ctypes.c_int, [P, P, ctypes.c_int]),
    "moe_cache_heat_file": (ctypes.c_int, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64),
                                           ctypes.POINTER(ctypes.c_int64)]),
    "moe_cache_freeze": (ctypes.c_int, [P]),
    "moe_probe_stream_read": (ctypes.c_int, [P, SZ, SZ, ctypes.c_int, ctypes.POINTER(ctypes.c_double), P]),
    "moe_cache_map_replay": (ctypes.c_int, [P, ctypes.c_char_p]),
    "moe_cache_set_norm": (ctypes.c_int, [P, ctypes.c_int, P, ctypes.c_int]),
    "moe_cache_set_streaming": (ctypes.c_int, [P, ctypes.POINTER(StreamConfig)]),
    "moe_cache_stream_stats": (ctypes.c_int, [P, ctypes.POINTER(StreamStats)]),
    "moe_cache_observe_gpu": (ctypes.c_int, [P, ctypes.c_int, P, P, ctypes.c_int]),
    "moe_cache_stream_take": (ctypes.c_int, [P, ctypes.c_int, P, P, P, U64, U64, U64]),
    "moe_cache_stream_posted": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_stream_next": (ctypes.c_int, [P, U64, ctypes.c_int, ctypes.POINTER(StreamChunk)]),
    "moe_cache_stream_land": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_stream_job": (ctypes.c_int, [P, ctypes.c_int, ctypes.POINTER(I32), ctypes.POINTER(I32)]),
    "moe_route_ahead": (ctypes.c_int, [ctypes.POINTER(RouteDesc), ctypes.POINTER(AheadDesc), P, P, P]),
    "moe_predictor_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(P)]),
    "moe_predictor_free": (None, [P]),
    "moe_predictor_info_get": (ctypes.c_int, [P, ctypes.POINTER(PredictorInfo)]),
    "moe_predictor_has_layer": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_predictor_score": (ctypes.c_int, [P, ctypes.c_int, ctypes.POINTER(PredictorLists), P]),
    "moe_predictor_top_k": (ctypes.c_int, [P, P, ctypes.c_int, P]),
    "moe_predictor_update": (ctypes.c_int, [P, ctypes.c_int, ctypes.POINTER(PredictorLists), P, ctypes.c_int, F32,
                                            ctypes.POINTER(F32)]),
    "moe_predictor_save": (ctypes.c_int, [P, ctypes.c_char_p]),
    "moe_cache_set_predictor": (ctypes.c_int, [P, P, ctypes.c_int, ctypes.c_float, ctypes.c_char_p]),
    "moe_cache_set_evictor": (ctypes.c_int, [P, P]),
    "moe_cache_set_spec_probation": (ctypes.c_int, [P, ctypes.c_int]),
    "moe_cache_predictor_stats": (ctypes.c_int, [P, ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double),
                                                 ctypes.POINTER(ctypes.c_uint64)]),
    "moe_planner_create": (P, [U64]),
    "moe_planner_destroy": (None, [P]),
    "moe_planner_reset": (None, [P]),
    "moe_planner_offer": (ctypes.c_int, [P, ctypes.c_int, I32, U64, U64]),
    "moe_planner_posted": (None, [P, ctypes.c_int]),
    "moe_planner_next": (ctypes.c_int, [P, U64, ctypes.c_double, ctypes.c_int, ctypes.POINTER(StreamChunk)]),
    "moe_planner_size": (ctypes.c_int, [P]),
    "moe_planner_get": (ctypes.c_int, [P, ctypes.c_int, ctypes.POINTER(PlannerJob)]),
    "moe_planner_counters": (None, [P, P]),
    "moe_cache_kernel_times": (ctypes.c_int, [P, ctypes.POINTER(KernelTimes)]),
    "moe_decode_layer": (ctypes.c_int, [P, ctypes.c_int, P, P, P, P, P, P]),
    "moe_decode_token": (ctypes.c_int, [P, P, P, P, P, P]),
    "moe_decode_batch": (ctypes.c_int, [P, P, P, P, ctypes.c_int, P, P]),
    "moe_dispatch": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P]),
    "moe_quant_rows": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, P, P, P]),
    "moe_grouped_workspace_bytes": (SZ, [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "moe_grouped_experts": (ctypes.c_int, [ctypes.POINTER(GroupedDesc), P]),
    "moe_grouped_experts_static": (ctypes.c_int, [ctypes.POINTER(GroupedDesc), P]),
    "moe_combine": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, ctypes.c_int, P, ctypes.c_int, P]),
    "moe_pool_create": (ctypes.c_int, [ctypes.c_int, ctypes.c_int, SZ, ctypes.c_int, ctypes.POINTER(P)]),
    "moe_pool_destroy": (ctypes.c_int, [P]),
    "moe_pool_copy": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int, P, SZ]),
    "moe_pool_ready": (ctypes.c_int, [P, ctypes.c_int, ctypes.c_int]),
    "moe_pool_sync": (ctypes.c_int, [P]),
    "moe_pool_slot_ptr": (P, [P, ctypes.c_int, ctypes.c_int]),
}

_lib = None


def lib():
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MoeError(f"{LIB_PATH} is missing: run `python moe-prefetch_amd/build.py` "
                           "(or __graft_entry__.build()) first")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def check(rc, what=""):
    if rc != MOE_OK:
        msg = lib().moe_last_error().decode(errors="replace")
        raise MoeError(f"{what}: status {rc}: {msg}")
    return rc
