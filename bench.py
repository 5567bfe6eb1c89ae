#!/usr/bin/env python3
"""Decode throughput of the MoE hot path on one MI355X.

Workload (default, the stacked Qwen3-30B-A3B shape): 48 MoE layers, hidden
2048, 128 experts, top-8, SwiGLU intermediate 768; gate/up Q4_K, down Q6_K in
odd layers and Q4_K in even ones; a 56-slot HBM cache per layer over a pinned
host store holding all 128 experts of every layer; routing steered to a
per-layer Zipf(1.1) popularity with reuse p = 0.6; window (second-miss)
admission, batched table writes, max 2 inserts per layer per step.  A step is
one batch-1 decode token through all 48 layers (router, experts from HBM slots
or the pinned store, combine, routed ids back, cache step with uploads on the
side stream).  The synthetic sequence is 512 tokens: --warmup tokens warm the
cache, the next --steps tokens are timed.

Prints ONE JSON line (rank 0, N = 1).  Inputs are resident before timing:
weights in the pinned store / HBM, activations and steering on the device.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "moe-prefetch_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "MoE decode tok/s @bs1 (48 layers, 56 slots) + achieved HBM GB/s; cache hit %"
HBM_PEAK_GBS = 8000.0


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=448)
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--layers", type=int, default=48)
    ap.add_argument("--slots", type=int, default=56)
    ap.add_argument("--admit", default="window")
    ap.add_argument("--cache-prior", type=float, default=0.0)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="bounded CPU-baseline sample")
    ap.add_argument("--kernel-steps", type=int, default=64, help="eager tokens timed per kernel")
    ap.add_argument("--path", type=int, default=0, help="0 fused, 1 fork/join, 2 serial expert launches")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="end with a plain 256 MiB device copy (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-check", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode in this build "
              "(the expert-sharded design is described in DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import ctypes

    import numpy as np
    import torch

    import moe_prefetch
    from moe_prefetch import MoeCache, _lib
    from moe_prefetch.workload import KIND_ROUTER, KIND_X, down_types, steering_bias, zipf_targets

    L = moe_prefetch.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream().cuda_stream
    H, E, K, I = 2048, 128, 8, 768
    NL, T = args.layers, args.warmup + args.steps
    dts = down_types(NL)
    eb = [L.moe_expert_bytes(H, I, dt) for dt in dts]

    t_setup = time.time()
    log(f"[bench] setup: {NL} layers x {E} experts, store {sum(eb) * E / 1e9:.2f} GB pinned")
    stores, views = [], []
    for l in range(NL):
        p = L.moe_host_alloc(E * eb[l])
        if not p:
            raise MemoryError(L.moe_last_error())
        stores.append(p)
        dptr = L.moe_host_device_ptr(p)
        _lib.check(L.moe_synth_experts(args.seed, l, 0, E, H, I, dts[l], 0.02, dptr, eb[l], stream), "synth")
    W = torch.empty((NL, E, H), dtype=torch.float32, device=dev)
    _lib.check(L.moe_synth_vec(args.seed, KIND_ROUTER, 0, NL, 0, E, H, 0.02, W.data_ptr(), stream), "W")
    x = torch.empty((T, NL, H), dtype=torch.float32, device=dev)
    _lib.check(L.moe_synth_vec(args.seed, KIND_X, 0, T, 0, NL, H, 1.0, x.data_ptr(), stream), "x")
    steer = args.cache_prior == 0.0
    bias = None
    if steer:
        tg = [zipf_targets(args.seed, l, T, s=1.1, reuse=0.6) for l in range(NL)]
        bias = torch.from_numpy(steering_bias(tg)).to(dev)
    torch.cuda.synchronize()
    cache = MoeCache(NL, intermediate=I, n_slots=args.slots, down_types=dts, admit=args.admit,
                     batch_tables=True, cache_prior=args.cache_prior, device=0)
    for l in range(NL):
        cache.set_host_store(l, stores[l])
        cache.set_router(l, W[l])
    cache.set_decode_path(split=args.path, graph=True)
    log(f"[bench] setup done in {time.time() - t_setup:.1f}s")

    out = torch.empty((NL, H), dtype=torch.float32, device=dev)
    ids_log = np.empty((T, NL, K), np.int32)
    keep = {}
    check_tokens = {args.warmup, T - 1}

    def token(t):
        b = None if bias is None else bias[t]
        cache.decode_token(x[t], out, bias=b, stream=stream, ids_out=ids_log[t])
        if t in check_tokens:
            keep[t] = out.cpu().numpy().copy()

    for t in range(args.warmup):
        token(t)
    s0 = cache.stats()
    torch.cuda.synchronize()
    log(f"[bench] warmup {args.warmup} tokens done; timing {args.steps}")
    t0 = time.perf_counter()
    for t in range(args.warmup, T):
        token(t)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    s1 = cache.stats()
    frames_after = [cache.frame(l) for l in range(NL)]
    log(f"[bench] timed {args.steps} tokens in {elapsed:.2f}s")

    # Per-kernel durations: HIP events on each launch's stream cannot be read
    # from inside a graph, so the same cache continues for --kernel-steps more
    # tokens launched eagerly with events around every launch (not in `value`).
    kernel_tokens = min(args.kernel_steps, args.steps)
    cache.set_decode_path(split=2, graph=False)   # resident and absent experts timed apart
    cache.set_timing(True)
    xs = torch.empty((kernel_tokens, NL, H), dtype=torch.float32, device=dev)
    _lib.check(L.moe_synth_vec(args.seed, KIND_X, T, kernel_tokens, 0, NL, H, 1.0, xs.data_ptr(), stream), "x2")
    if bias is not None:
        tg2 = [zipf_targets(args.seed + 1, l, kernel_tokens, s=1.1, reuse=0.6) for l in range(NL)]
        bias2 = torch.from_numpy(steering_bias(tg2)).to(dev)
    for t in range(kernel_tokens):
        cache.decode_token(xs[t], out, bias=None if bias is None else bias2[t], stream=stream)
    torch.cuda.synchronize()
    kt = cache.kernel_times()
    cache.set_timing(False)
    log(f"[bench] per-kernel timing pass: {kernel_tokens} tokens")

    tok_s = args.steps / elapsed
    seen = (s1["n_hit"] - s0["n_hit"]) + (s1["n_miss"] - s0["n_miss"])
    hit = (s1["n_hit"] - s0["n_hit"]) / max(seen, 1)
    miss_tok = (s1["n_miss"] - s0["n_miss"]) / args.steps
    upl_tok = (s1["n_scheduled"] - s0["n_scheduled"]) / args.steps
    n = max(kt["n_layers"], 1)
    # HBM-bound launches (experts resident in slots) carry the roofline; the
    # absent experts' launches stream the pinned store over PCIe
    hbm = {"gateup_hbm": (kt["gateup_hbm_ms"], kt["gateup_hbm_bytes"]),
           "down_hbm": (kt["down_hbm_ms"], kt["down_hbm_bytes"])}
    host = {"gateup_host": (kt["gateup_host_ms"], kt["gateup_host_bytes"]),
            "down_host": (kt["down_host_ms"], kt["down_host_bytes"])}
    dom = max(hbm, key=lambda k: hbm[k][0])
    dom_ms, dom_bytes = hbm[dom]
    avg_ms = dom_ms / n
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9 if dom_ms > 0 else 0.0
    host_ms = sum(v[0] for v in host.values())
    host_gbs = sum(v[1] for v in host.values()) / (host_ms * 1e-3) / 1e9 if host_ms > 0 else 0.0
    times = {"route": kt["route_ms"], **{k: v[0] for k, v in hbm.items()}, **{k: v[0] for k, v in host.items()}}
    nt = max(kernel_tokens, 1)
    # HBM bytes per launch of this kernel: the (read + write) / algorithmic
    # ratio measured with rocprofv3 PMC counters (profiles/traffic.json) times
    # this run's algorithmic bytes per launch
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f).get(dom)
        if tr:
            ratio = (tr["hbm_read_bytes_per_launch"] + tr["hbm_write_bytes_per_launch"]) / \
                tr["algorithmic_bytes_per_launch"]
            traffic = round(ratio * dom_bytes / n)
    result = {
        "metric": METRIC, "value": round(tok_s, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * elapsed / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8_k int8-dot, fp32 scale (router fp32)",
        "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K/Q6_K, N(0,1) activations)",
        "config": {"workload": f"stacked{NL}: {NL} layers x {E} experts, H {H}, I {I}, top-{K}, "
                               f"{args.slots} HBM slots/layer over a pinned store, Q6_K down in odd layers, "
                               f"Zipf(1.1) reuse 0.6, admission {args.admit}, batched tables, "
                               f"{T} tokens ({args.warmup} warmup)",
                   "batch": 1, "layers": NL, "slots": args.slots, "cache_prior": args.cache_prior},
        "cache": {"hit_rate": round(hit, 4), "missed_per_token": round(miss_tok, 2),
                  "uploaded_per_token": round(upl_tok, 2),
                  "publication_wait_ms_per_token": round((s1["publication_wait_us"] - s0["publication_wait_us"])
                                                         / 1e3 / args.steps, 4)},
        "kernels_ms_per_token": {k: round(v / nt, 4) for k, v in times.items()},
        "kernel_timing": f"HIP events around each launch on its stream, {kernel_tokens} eager tokens after the "
                         f"timed ones, resident and absent experts launched one after the other "
                         f"(graph replay cannot carry per-kernel events)",
        "decode_path": {0: "fused", 1: "fork/join", 2: "serial"}[args.path] + " expert launches, HIP graph per token",
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": round(dom_bytes / n), "avg_launch_us": round(avg_ms * 1e3, 2),
                     "launches": n},
        "hbm_kernels": {k: {"bytes_per_launch": round(v[1] / n), "avg_launch_us": round(v[0] / n * 1e3, 2),
                            "gbs": round(v[1] / (v[0] * 1e-3) / 1e9, 1) if v[0] > 0 else 0.0}
                        for k, v in hbm.items()},
        "pcie": {"kernels": "gateup_host + down_host (absent experts read from the pinned store)",
                 "achieved": round(host_gbs, 1), "unit": "GB/s", "peak_nominal": 64.0,
                 "ms_per_token": round(host_ms / nt, 4),
                 "upload_gb_per_token": round((s1["bytes_uploaded"] - s0["bytes_uploaded"]) / 1e9 / args.steps, 4)},
    }

    if not args.no_check:
        log("[bench] checking the full-size run against the oracle (outside the timed region)")
        from oracle import oracle as O
        oc = O.Cache([args.slots] * NL, admit=args.admit, batch_tables=True, cache_prior=args.cache_prior)
        Wh = W.cpu().numpy()
        xh = x.cpu().numpy()
        bh = None if bias is None else bias.cpu().numpy()
        bad_ids = 0
        worst = 0.0
        store_arr = [np.ctypeslib.as_array((ctypes.c_uint8 * (E * eb[l])).from_address(stores[l]))
                     for l in range(NL)]
        for t in range(T):
            for l in range(NL):
                if args.cache_prior > 0 or t in check_tokens or l == t % NL:
                    tbl, prior = oc.table(l)
                    rids, rw, _, _ = O.route(Wh[l], xh[t, l], K, bias=None if bh is None else bh[t, l],
                                             prior=prior if args.cache_prior > 0 else None, table=tbl)
                    bad_ids += not np.array_equal(rids, ids_log[t, l])
                    if t in check_tokens:
                        want = O.moe_layer(H, I, dts[l], [store_arr[l][e * eb[l]:(e + 1) * eb[l]] for e in rids],
                                           rw, xh[t, l], n_threads=8)
                        r = float(np.linalg.norm(keep[t][l].astype(np.float64) - want) / np.linalg.norm(want))
                        worst = max(worst, r)
                oc.observe(l, ids_log[t, l])
            oc.step()
        frames_equal = all(np.array_equal(oc.frame(l), frames_after[l]) for l in range(NL))
        os_ = oc.stats()
        counters_equal = all(os_[k] == s1[k] for k in ("n_hit", "n_miss", "n_scheduled", "n_published",
                                                         "n_admit_ok", "n_admit_denied", "n_table_flushes"))
        result["check"] = {"ids_mismatched": int(bad_ids), "frames_equal": bool(frames_equal),
                           "counters_equal": bool(counters_equal), "worst_rel_l2": worst,
                           "outputs_checked": len(check_tokens) * NL}
        del store_arr
        log(f"[bench] check: {result['check']}")

    if not args.no_cpu:
        from oracle import oracle as O
        cores = min(len(os.sched_getaffinity(0)), 16)
        Wh = W.cpu().numpy()
        xh = x.cpu().numpy()
        bh = None if bias is None else bias.cpu().numpy()
        addrs = [stores[l] for l in range(NL)]
        log(f"[bench] CPU baseline: oracle decode on {cores} threads for ~{args.cpu_seconds}s")
        t0 = time.perf_counter()
        done = 0
        while done < T and (time.perf_counter() - t0) < args.cpu_seconds:
            t = done
            for l in range(NL):
                rids, rw, _, _ = O.route(Wh[l], xh[t, l], K, bias=None if bh is None else bh[t, l])
                O.moe_layer(H, I, dts[l], [addrs[l] + int(e) * eb[l] for e in rids], rw, xh[t, l],
                            n_threads=cores)
            done += 1
        cpu_el = time.perf_counter() - t0
        result["cpu_baseline"] = {"value": round(done / cpu_el, 3), "unit": "tok/s", "cores": cores,
                                  "kind": "port",
                                  "sample": f"{done} tokens x {NL} layers of the same workload, every routed "
                                            f"expert computed on the host from the pinned store (Q8_K "
                                            f"activations, integer dots, OpenMP over rows), {cpu_el:.1f}s"}

    cache.close()
    for p in stores:
        L.moe_host_free(p)
    if args.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device=dev)
        for _ in range(3):
            dst = src.clone()
        torch.cuda.synchronize()
        del src, dst
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
