#!/usr/bin/env python3
"""Decode throughput of the MoE hot path on one MI355X.

The line's `value` is configuration 2 (stacked48): 48 MoE layers of the
Qwen3-30B-A3B shape -- hidden 2048, 128 experts, top-8, SwiGLU intermediate
768, gate/up Q4_K, down Q6_K in odd layers and Q4_K in even ones -- with a
56-slot HBM cache per layer over a pinned host store holding all 128 experts
of every layer.  Routing is steered to a per-layer Zipf(1.1) popularity with
reuse p = 0.6; window (second-miss) admission, batched table writes, max 2
inserts per layer per step.  A step is one batch-1 decode token through all 48
layers (each layer one fused launch: router, selection, experts from HBM
slots, combine; the routed ids back, cache step with uploads on the side
stream), replayed as one HIP graph.  Experts absent from the slots are
computed by the host CPU (14 threads; the reference's sidecar) while the GPU
runs the resident ones; `gpu_only` is the same decode with the GPU reading
absent experts from the pinned store over PCIe.

The synthetic sequence is 512 tokens.  --warmup tokens warm the cache and the
next --steps are timed for `value`; the run then continues to token 511 and
`steady` reports tokens 64..511 (the cache full: evictions and admission
denials in every step).  Beside it, in the same line:

  config1  one layer, all 128 experts resident, 256 steps: GB/s and the
           fraction of 8 TB/s of the fused layer launch on 21,233,664 expert
           bytes + 1 MiB of router per step
  config3  the single-layer shape stacked 48 deep, 512 tokens at delta = 0,
           0.01 on probabilities and 0.01 on logits: change in hit rate,
           relative L2 of the block outputs against delta = 0
  config4  batched layers (48, all experts in HBM): a 512-token prefill chunk
           and batch-64 decode on the matrix cores, GB/s and MFMA utilisation
  config5  40 layers x 256 experts + 1 shared, I 512, 96 slots, delta 0.01:
           1024 tokens at batch 1, then 128 at batch 16
  cpu_baseline  the host chain (AVX-512 VNNI integer dots, the same numerics)
           swept over {1, 4, 8, all} threads: us per expert, per layer of 8,
           tok/s of configuration 2 with every expert on the CPU

Other --workload values print their own line: prefill48, prior48, wide40,
residual48 (router lookahead + just-in-time streaming), single1.

Inputs are resident before timing: weights in the pinned store / HBM slots,
activations and steering on the device.
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
H, E, K, I = 2048, 128, 8, 768
COUNTERS = ("n_hit", "n_miss", "n_scheduled", "n_published", "n_admit_ok", "n_admit_denied", "n_table_flushes")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Workload:
    """Pinned expert stores, router weights, activations and (optionally) a
    shared expert per layer in HBM for one stacked decode run.  `T1` tokens
    are decoded one at a time, the `T - T1` after them in batches."""

    def __init__(self, args, steer, n_experts=E, inter=I, shared=False, zipf_s=1.1, reuse=0.6, slots=None,
                 batch_tokens=0, T=None):
        import torch
        import moe_prefetch
        from moe_prefetch import _lib
        from moe_prefetch.workload import KIND_ROUTER, KIND_X, down_types, steering_bias, zipf_targets
        self.torch, self._lib, self.args = torch, _lib, args
        self.L = L = moe_prefetch.lib()
        self.dev = dev = torch.device("cuda:0")
        self.stream = stream = torch.cuda.current_stream().cuda_stream
        self.E, self.I, self.zipf_s, self.reuse = n_experts, inter, zipf_s, reuse
        self.slots = args.slots if slots is None else slots
        self.NL = NL = args.layers
        self.T1 = args.warmup + args.steps
        self.T = T = max(self.T1 + batch_tokens, T or 0)
        self.dts = down_types(NL)
        self.eb = [L.moe_expert_bytes(H, inter, dt) for dt in self.dts]
        self.zipf_targets, self.steering_bias, self.KIND_X = zipf_targets, steering_bias, KIND_X
        t0 = time.time()
        log(f"[bench] setup: {NL} layers x {n_experts} experts{' + shared' if shared else ''}, "
            f"store {sum(self.eb) * n_experts / 1e9:.2f} GB pinned")
        self.stores, self.shared = [], []
        for l in range(NL):
            p = L.moe_host_alloc(n_experts * self.eb[l])
            if not p:
                raise MemoryError(L.moe_last_error())
            self.stores.append(p)
            _lib.check(L.moe_synth_experts(args.seed, l, 0, n_experts, H, inter, self.dts[l], 0.02,
                                           L.moe_host_device_ptr(p), self.eb[l], stream), "synth")
            if shared:     # the generator's expert index n_experts, kept in HBM
                sh = torch.empty(self.eb[l], dtype=torch.uint8, device=dev)
                _lib.check(L.moe_synth_experts(args.seed, l, n_experts, 1, H, inter, self.dts[l], 0.02,
                                               sh.data_ptr(), self.eb[l], stream), "synth shared")
                self.shared.append(sh)
            else:
                self.shared.append(None)
        self.W = torch.empty((NL, n_experts, H), dtype=torch.float32, device=dev)
        _lib.check(L.moe_synth_vec(args.seed, KIND_ROUTER, 0, NL, 0, n_experts, H, 0.02, self.W.data_ptr(), stream),
                   "W")
        self.x = torch.empty((T, NL, H), dtype=torch.float32, device=dev)
        _lib.check(L.moe_synth_vec(args.seed, KIND_X, 0, T, 0, NL, H, 1.0, self.x.data_ptr(), stream), "x")
        self.bias = None
        if steer:
            tg = [zipf_targets(args.seed, l, T, n_experts=n_experts, s=zipf_s, reuse=reuse) for l in range(NL)]
            self.bias = torch.from_numpy(steering_bias(tg, n_experts=n_experts)).to(dev)
        torch.cuda.synchronize()
        self.shared_h = [None if sh is None else sh.cpu().numpy() for sh in self.shared]
        log(f"[bench] setup done in {time.time() - t0:.1f}s")

    def oracle_layer(self, stores, l, rids, rw, x, n_threads):
        """The oracle's layer output: routed experts in k order, then the shared
        expert with weight 1."""
        import numpy as np
        from oracle import oracle as O
        eb, base = self.eb[l], stores[l]
        experts = [base + int(e) * eb if isinstance(base, int) else base[e * eb:(e + 1) * eb] for e in rids]
        w = list(rw)
        if self.shared_h[l] is not None:
            experts.append(self.shared_h[l])
            w.append(1.0)
        return O.moe_layer(H, self.I, self.dts[l], experts, np.asarray(w, np.float32), x, n_threads=n_threads)

    def cache(self, **knobs):
        from moe_prefetch import MoeCache
        c = MoeCache(self.NL, n_experts=self.E, intermediate=self.I, n_slots=self.slots, down_types=self.dts,
                     batch_tables=True, device=0, **knobs)
        for l in range(self.NL):
            c.set_host_store(l, self.stores[l])
            c.set_router(l, self.W[l])
            if self.shared[l] is not None:
                c.set_shared(l, self.shared[l])
        return c

    def residual(self):
        """Router inputs and norm weights of the residual-stream workload (the
        lookahead workload): x [T][L][H], g [L][H] on the device."""
        if getattr(self, "x_res", None) is None:
            from moe_prefetch.workload import residual_stream
            t0 = time.time()
            self.x_res, self.g_res = residual_stream(self.args.seed, self.T, self.NL, self.torch, self.dev,
                                                     self.stream)
            self.torch.cuda.synchronize()
            self.g_res_h = self.g_res.cpu().numpy()
            log(f"[bench] residual stream of {self.T} tokens x {self.NL} layers in {time.time() - t0:.1f}s")
        return self.x_res, self.g_res_h

    def decode(self, cache, keep=(), all_out=None, x=None, steer=True):
        """Warm up, then time the rest of the sequence.  Returns (elapsed s, stats
        before / after the timed tokens, ids [T][L][K], kept outputs, frames).
        x: other router inputs [T][L][H]; steer=False: no steering bias."""
        import numpy as np
        torch = self.torch
        out = torch.empty((self.NL, H), dtype=torch.float32, device=self.dev)
        ids_log = np.empty((self.T, self.NL, K), np.int32)     # batched tokens are filled in by decode_batches
        kept = {}
        xs = self.x if x is None else x
        bias = self.bias if steer else None

        def token(t):
            dst = all_out[t] if all_out is not None else out
            cache.decode_token(xs[t], dst, bias=None if bias is None else bias[t],
                               stream=self.stream, ids_out=ids_log[t])
            if t in keep:
                kept[t] = dst.cpu().numpy().copy()

        for t in range(self.args.warmup):
            token(t)
        s0 = cache.stats()
        torch.cuda.synchronize()
        log(f"[bench] warmup {self.args.warmup} tokens done; timing {self.args.steps}")
        t0 = time.perf_counter()
        for t in range(self.args.warmup, self.T1):
            token(t)
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        s1 = cache.stats()
        frames = [cache.frame(l) for l in range(self.NL)]
        log(f"[bench] timed {self.args.steps} tokens in {elapsed:.2f}s")
        return elapsed, s0, s1, ids_log, kept, frames

    def tokens(self, cache, t0, t1, ids_log, keep=(), kept=None, all_out=None, x=None, steer=True):
        """Decode tokens [t0, t1) one at a time (graph replay); returns the
        elapsed seconds, synchronised on both sides."""
        torch = self.torch
        out = torch.empty((self.NL, H), dtype=torch.float32, device=self.dev)
        xs = self.x if x is None else x
        bias = self.bias if steer else None
        torch.cuda.synchronize()
        tic = time.perf_counter()
        for t in range(t0, t1):
            dst = all_out[t] if all_out is not None else out
            cache.decode_token(xs[t], dst, bias=None if bias is None else bias[t], stream=self.stream,
                               ids_out=ids_log[t])
            if t in keep:
                kept[t] = dst.cpu().numpy().copy()
        torch.cuda.synchronize()
        return time.perf_counter() - tic

    def tokens_per_layer(self, cache, t0, t1, ids_log, xin, outs):
        """Decode tokens [t0, t1) as a model drives the per-layer op: layer l's
        input is x_l = x_{l-1} + out_{l-1} (x_0 the token's first activation;
        one add on the stream per layer, the caller's residual), every layer
        one moe_decode_layer call (the fused launch; the host's share of the
        absent experts served inside the call), the ids copied back once, each
        layer observed, one step.  xin [T][L][H] and outs [T][L][H] keep every
        layer's input and output for the check.  Returns the elapsed seconds,
        synchronised on both sides."""
        torch = self.torch
        ids_dev = torch.empty((self.NL, K), dtype=torch.int32, device=self.dev)
        bias = self.bias
        torch.cuda.synchronize()
        tic = time.perf_counter()
        for t in range(t0, t1):
            xin[t, 0].copy_(self.x[t, 0])
            for l in range(self.NL):
                cache.decode_layer(l, xin[t, l], outs[t, l], bias=None if bias is None else bias[t, l],
                                   ids=ids_dev[l], stream=self.stream)
                if l + 1 < self.NL:
                    torch.add(xin[t, l], outs[t, l], out=xin[t, l + 1])
            ids_log[t] = ids_dev.cpu().numpy()
            for l in range(self.NL):
                cache.observe(l, ids_log[t, l])
            cache.step()
        torch.cuda.synchronize()
        return time.perf_counter() - tic

    def kernel_pass(self, cache, split=2, keep_serving=False):
        """Per-kernel durations: the same cache continues for --kernel-steps more
        tokens launched eagerly (HIP events cannot be read from graph nodes).
        split 2: resident and absent experts as separate launches, GPU only;
        split 0 with keep_serving: the fused layer launch as the decode runs it
        (absent experts on the host CPU)."""
        torch, L, _lib = self.torch, self.L, self._lib
        n = min(self.args.kernel_steps, max(self.args.steps, 16))
        if not keep_serving:
            cache.set_sidecar(0)                # GPU kernels only
        cache.set_decode_path(split=split, graph=False)
        cache.set_timing(True)
        xs = torch.empty((n, self.NL, H), dtype=torch.float32, device=self.dev)
        _lib.check(L.moe_synth_vec(self.args.seed, self.KIND_X, self.T, n, 0, self.NL, H, 1.0, xs.data_ptr(),
                                   self.stream), "x2")
        b2 = None
        if self.bias is not None:
            tg2 = [self.zipf_targets(self.args.seed + 1, l, n, n_experts=self.E, s=self.zipf_s, reuse=self.reuse)
                   for l in range(self.NL)]
            b2 = torch.from_numpy(self.steering_bias(tg2, n_experts=self.E)).to(self.dev)
        out = torch.empty((self.NL, H), dtype=torch.float32, device=self.dev)
        cache.set_upload_stats(True)            # each upload's copy timed on its stream as well
        u0 = cache.stats()
        for t in range(n):
            cache.decode_token(xs[t], out, bias=None if b2 is None else b2[t], stream=self.stream)
        torch.cuda.synchronize()
        u1 = cache.stats()
        cache.set_upload_stats(False)
        self.upload_in_decode = {}
        for kind in ("h2d", "d2d"):
            nu = u1[f"n_upload_{kind}"] - u0[f"n_upload_{kind}"]
            us = u1[f"upload_{kind}_us"] - u0[f"upload_{kind}_us"]
            self.upload_in_decode[kind] = {"n": nu, "us_per_upload": round(us / nu, 1) if nu else None}
        kt = cache.kernel_times()
        cache.set_timing(False)
        log(f"[bench] per-kernel timing pass: {n} tokens")
        return kt, n

    def batch_kernel_pass(self, cache, B, n_batches=4):
        """Per-kernel durations of the batched decode: the batched tokens'
        first n_batches batches decoded again on the same cache with timing on
        (each layer's grouped launches waited for)."""
        torch = self.torch
        cache.set_timing(True)
        out = torch.empty((self.NL, B, H), dtype=torch.float32, device=self.dev)
        for i in range(n_batches):
            t0 = self.T1 + B * i
            if t0 + B > self.T:
                break
            xb = self.x[t0:t0 + B].transpose(0, 1).contiguous()
            bb = None if self.bias is None else self.bias[t0:t0 + B].transpose(0, 1).contiguous()
            cache.decode_batch(xb, out, bias=bb, stream=self.stream)
        torch.cuda.synchronize()
        kt = cache.kernel_times()
        cache.set_timing(False)
        log(f"[bench] batched per-kernel timing pass: {n_batches} batches of {B}")
        return kt

    def decode_batches(self, cache, B, keep=()):
        """Tokens T1.. decoded B at a time with moe_decode_batch.  Returns
        (elapsed s, per-batch ms, stats before / after, ids [T-T1][L][K], kept
        outputs)."""
        import numpy as np
        torch = self.torch
        n = self.T - self.T1
        xb, bb = [], []
        for t0 in range(self.T1, self.T, B):
            xb.append(self.x[t0:t0 + B].transpose(0, 1).contiguous())
            bb.append(None if self.bias is None else self.bias[t0:t0 + B].transpose(0, 1).contiguous())
        out = torch.empty((self.NL, B, H), dtype=torch.float32, device=self.dev)
        ids = np.empty((n // B, self.NL, B, K), np.int32)
        kept, per = {}, []
        s0 = cache.stats()
        torch.cuda.synchronize()
        log(f"[bench] timing {n} tokens at batch {B}")
        t0 = time.perf_counter()
        for i in range(n // B):
            ti = time.perf_counter()
            cache.decode_batch(xb[i], out, bias=bb[i], stream=self.stream, ids_out=ids[i])
            per.append(round(1e3 * (time.perf_counter() - ti), 3))
            for j in range(B):
                if self.T1 + B * i + j in keep:
                    kept[self.T1 + B * i + j] = out[:, j].cpu().numpy().copy()
        torch.cuda.synchronize()
        elapsed = time.perf_counter() - t0
        s1 = cache.stats()
        log(f"[bench] timed {n} batched tokens in {elapsed:.3f}s")
        return elapsed, per, s0, s1, ids.transpose(0, 2, 1, 3).reshape(n, self.NL, K), kept

    def check(self, ids_log, kept, frames, s1, knobs, every=False, batch=1, steer=True, T=None, heat=None,
              x_host=None):
        """Full-size properties against the oracle, outside every timed region:
        routed ids (every token and layer when `every` or a prior is on, else
        one layer per token), frames, counters, and the kept outputs.  Tokens
        from T1 on were decoded `batch` at a time: observed together, one step
        per batch, no prior (it biases single-token selection only).  x_host:
        the layers' inputs [T][L][H] when they are not the workload's own."""
        import ctypes
        import numpy as np
        from oracle import oracle as O
        prior_on = knobs.get("cache_prior", 0.0) > 0
        logits_space = knobs.get("prior_space", "probs") == "logits"
        oc = O.Cache([self.slots] * self.NL, n_experts=self.E, admit=knobs.get("admit", "off"), batch_tables=True,
                     cache_prior=knobs.get("cache_prior", 0.0))
        if heat:
            oc.heat_file(heat)
        Wh, xh = self.W.cpu().numpy(), self.x.cpu().numpy() if x_host is None else x_host
        bh = None if (self.bias is None or not steer) else self.bias.cpu().numpy()
        stores = [np.ctypeslib.as_array((ctypes.c_uint8 * (self.E * self.eb[l])).from_address(self.stores[l]))
                  for l in range(self.NL)]
        bad, worst, checked = 0, 0.0, 0
        t = 0
        T = self.T if T is None else T
        while t < T:
            n = 1 if t < self.T1 else batch
            for l in range(self.NL):
                tbl, prior = oc.table(l)
                use_prior = prior if prior_on and n == 1 else None
                for tt in range(t, t + n):
                    if every or prior_on or tt in kept or l == tt % self.NL:
                        rids, rw, _, _ = O.route(Wh[l], xh[tt, l], K, bias=None if bh is None else bh[tt, l],
                                                 prior=use_prior, table=tbl, prior_on_logits=logits_space)
                        bad += not np.array_equal(rids, ids_log[tt, l])
                        checked += 1
                        if tt in kept:
                            want = self.oracle_layer(stores, l, rids, rw, xh[tt, l], 8)
                            worst = max(worst, float(np.linalg.norm(kept[tt][l].astype(np.float64) - want)
                                                     / np.linalg.norm(want)))
                oc.observe(l, np.ascontiguousarray(ids_log[t:t + n, l]), n_tok=n)
            oc.step()
            t += n
        os_ = oc.stats()
        res = {"ids_checked": checked, "ids_mismatched": int(bad),
               "frames_equal": bool(all(np.array_equal(oc.frame(l), frames[l]) for l in range(self.NL))),
               "counters_equal": bool(all(os_[k] == s1[k] for k in COUNTERS)),
               "worst_rel_l2": worst, "outputs_checked": len(kept) * self.NL}
        oc.close()
        return res

    def cpu_baseline(self, seconds):
        """The host expert chain (moe_cpu_experts: Q8_K activations, AVX-512
        VNNI integer dots, fp32 steps in the CPU chain's order -- the numerics
        of the reference's CPU path, experiments/x2_cpu_expert_cost.cpp:115-156)
        timed as that experiment times it: a tour over experts of the pinned
        store (cold in the CPU's caches), one expert per call and a layer's 8
        per call, for 1, 4, 8 and all threads (p50 of the calls)."""
        import ctypes
        import numpy as np
        from oracle import oracle as O
        L = self.L
        nproc = os.cpu_count() or 1
        usable = len(os.sched_getaffinity(0))
        phys = set()
        for c in os.sched_getaffinity(0):
            try:
                base = f"/sys/devices/system/cpu/cpu{c}/topology/"
                phys.add((open(base + "physical_package_id").read().strip(), open(base + "core_id").read().strip()))
            except OSError:
                phys.add((c,))
        threads = sorted({1, 4, 8, usable} & set(range(1, usable + 1)) | {usable})
        rng = np.random.default_rng(self.args.seed)
        # Q8_K of one activation (any: the arithmetic per byte does not depend on it)
        q8 = O.quant_q8k(self.x[0, 0].cpu().numpy())
        tour = [(int(l), int(e)) for l, e in zip(rng.integers(0, self.NL, 4096), rng.integers(0, self.E, 4096))]
        budget = seconds / (2 * len(threads))
        rows, pos = [], 0
        log(f"[bench] CPU baseline: host chain, threads {threads}, ~{seconds:.0f}s")
        for th in threads:
            for m in (1, 8):
                # one warm-up call starts the thread team
                times = []
                tic = time.perf_counter()
                while time.perf_counter() - tic < budget or len(times) < 3:
                    l = tour[pos % len(tour)][0]
                    ptrs = (ctypes.c_void_p * m)(*[self.stores[l] + tour[(pos + j) % len(tour)][1] * self.eb[l]
                                                   for j in range(m)])
                    pos += m
                    rows_out = np.empty((m, H), np.float32)
                    t0 = time.perf_counter()
                    self._lib.check(L.moe_cpu_experts(ptrs, m, q8.ctypes.data, H, self.I, self.dts[l],
                                                      rows_out.ctypes.data, th, 0), "cpu experts")
                    times.append(time.perf_counter() - t0)
                t = np.array(times[1:]) * 1e6
                rows.append({"threads": th, "experts_per_call": m, "us_p50": round(float(np.median(t)), 1),
                             "us_p90": round(float(np.percentile(t, 90)), 1), "calls": len(t)})
        best = min((r for r in rows if r["experts_per_call"] == 8), key=lambda r: r["us_p50"])
        one = min((r for r in rows if r["experts_per_call"] == 1), key=lambda r: r["us_p50"])
        # a token through the stacked decode with every routed expert on the CPU: K experts per layer
        tok_s = 1e6 / (self.NL * best["us_p50"])
        return {"value": round(tok_s, 2), "unit": "tok/s", "cores": best["threads"], "kind": "port",
                "sample": f"{sum(r['calls'] for r in rows)} host-chain calls over a tour of the pinned store's "
                          f"experts ({len(threads)} thread counts x 1 and 8 experts per call, ~{seconds:.0f}s); "
                          f"tok/s = 1 / ({self.NL} layers x the best 8-expert call); the router is not included",
                "nproc": nproc, "usable_cpus": usable, "physical_cores": len(phys),
                "us_per_expert": one["us_p50"], "us_per_expert_threads": one["threads"],
                "us_per_layer_k8": best["us_p50"], "us_per_layer_k8_threads": best["threads"],
                "sweep": rows,
                "engine": "moe_cpu_experts (the library's host chain: AVX-512 VNNI dots when present; results "
                          "equal the oracle's bit for bit)" + ("" if L.moe_cpu_has_vnni() else ", portable path")}

    def close(self):
        for p in self.stores:
            self.L.moe_host_free(p)
        self.stores = []


def upload_cost(expert_bytes, n=300):
    """One expert's upload, measured as experiments/e1_upload_cost.py measures
    it ('pinned, dedicated stream': a pinned host buffer copied to HBM on a
    stream of its own, synchronised per expert, n times), and the staged
    device-to-device copy of the same bytes.  Host wall time per expert and the
    copy's own duration from events on the stream."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.empty(expert_bytes, dtype=torch.uint8, pin_memory=True)
    src.fill_(3)
    dst = torch.empty(expert_bytes, dtype=torch.uint8, device=dev)
    dst2 = torch.empty(expert_bytes, dtype=torch.uint8, device=dev)
    s = torch.cuda.Stream()
    out = {"expert_bytes": expert_bytes, "n": n}
    for name, a, b in (("pinned_h2d", dst, src), ("staged_d2d", dst2, dst)):
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
        with torch.cuda.stream(s):
            for _ in range(10):
                a.copy_(b, non_blocking=True)
            s.synchronize()
            t0 = time.perf_counter()
            for e0, e1 in evs:
                e0.record(s)
                a.copy_(b, non_blocking=True)
                e1.record(s)
                s.synchronize()
            wall = (time.perf_counter() - t0) / n * 1e6
        dev_us = sum(e0.elapsed_time(e1) for e0, e1 in evs) / n * 1e3
        out[name] = {"us_wall": round(wall, 2), "us_copy": round(dev_us, 2),
                     "gbs_copy": round(expert_bytes / (dev_us * 1e-6) / 1e9, 1)}
    return out


def size_matched(roof, iters=50):
    """The same bytes per launch read by a plain streaming-read kernel, each
    launch from a fresh window of a 4 GiB buffer, timed the same way: the
    ceiling a kernel of this size can reach on this GPU."""
    import ctypes
    import torch
    import moe_prefetch
    from moe_prefetch import _lib
    L = moe_prefetch.lib()
    buf = torch.empty(4 << 30, dtype=torch.uint8, device="cuda:0")
    buf.fill_(1)
    us = ctypes.c_double()
    b = int(roof["bytes_per_launch"])
    _lib.check(L.moe_probe_stream_read(buf.data_ptr(), buf.numel(), b, iters, ctypes.byref(us),
                                       torch.cuda.current_stream().cuda_stream), "probe")
    del buf
    torch.cuda.synchronize()
    gbs = b / (us.value * 1e-6) / 1e9
    return {"bytes": b, "avg_launch_us": round(us.value, 2), "gbs": round(gbs, 1),
            "frac": round(roof["achieved"] / gbs, 4),
            "what": "plain streaming-read kernel (8 x 16 B loads in flight per thread) over the same bytes, a cold "
                    "window per launch, dispatch-stamped events"}


def cache_summary(s0, s1, steps):
    seen = (s1["n_hit"] - s0["n_hit"]) + (s1["n_miss"] - s0["n_miss"])
    return {"hit_rate": round((s1["n_hit"] - s0["n_hit"]) / max(seen, 1), 4),
            "missed_per_token": round((s1["n_miss"] - s0["n_miss"]) / steps, 2),
            "uploaded_per_token": round((s1["n_scheduled"] - s0["n_scheduled"]) / steps, 2),
            "publication_wait_ms_per_token": round((s1["publication_wait_us"] - s0["publication_wait_us"])
                                                   / 1e3 / steps, 4),
            "host_boundary_ms_per_token": round((s1["host_boundary_us"] - s0["host_boundary_us"]) / 1e3 / steps, 4)}


def kernel_report(kt, n_tok, steps, s0, s1):
    """Per-kernel figures and the roofline of the dominant HBM-bound kernel (the
    launches over experts resident in slots; the absent experts' launches
    stream the pinned store over PCIe and are reported beside it)."""
    n = max(kt["n_layers"], 1)
    hbm = {"gateup_hbm": (kt["gateup_hbm_ms"], kt["gateup_hbm_bytes"]),
           "down_hbm": (kt["down_hbm_ms"], kt["down_hbm_bytes"])}
    host = {"gateup_host": (kt["gateup_host_ms"], kt["gateup_host_bytes"]),
            "down_host": (kt["down_host_ms"], kt["down_host_bytes"])}
    dom = max(hbm, key=lambda k: hbm[k][0])
    dom_ms, dom_bytes = hbm[dom]
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9 if dom_ms > 0 else 0.0
    host_ms = sum(v[0] for v in host.values())
    host_gbs = sum(v[1] for v in host.values()) / (host_ms * 1e-3) / 1e9 if host_ms > 0 else 0.0
    # HBM bytes per launch: the (read + write) / algorithmic ratio measured with
    # rocprofv3 PMC counters (profiles/traffic.json) times this run's bytes
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f).get(dom)
        if tr:
            ratio = (tr["hbm_read_bytes_per_launch"] + tr["hbm_write_bytes_per_launch"]) / \
                tr["algorithmic_bytes_per_launch"]
            traffic = round(ratio * dom_bytes / n)
    times = {"route": kt["route_ms"], **{k: v[0] for k, v in hbm.items()}, **{k: v[0] for k, v in host.items()}}
    nt = max(n_tok, 1)
    return {
        "kernels_ms_per_token": {k: round(v / nt, 4) for k, v in times.items()},
        "kernel_timing": f"HIP events stamped by each dispatch (hipExtLaunchKernelGGL) on its stream, {n_tok} "
                         f"eager tokens after the timed ones, resident and absent experts launched one after the "
                         f"other (graph replay cannot carry per-kernel events)",
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "bytes_per_launch": round(dom_bytes / n), "avg_launch_us": round(dom_ms / n * 1e3, 2),
                     "launches": n},
        "hbm_kernels": {k: {"bytes_per_launch": round(v[1] / n), "avg_launch_us": round(v[0] / n * 1e3, 2),
                            "gbs": round(v[1] / (v[0] * 1e-3) / 1e9, 1) if v[0] > 0 else 0.0}
                        for k, v in hbm.items()},
        "pcie": {"kernels": "gateup_host + down_host (absent experts read from the pinned store)",
                 "achieved": round(host_gbs, 1), "unit": "GB/s", "peak_nominal": 64.0,
                 "ms_per_token": round(host_ms / nt, 4),
                 "upload_gb_per_token": round((s1["bytes_uploaded"] - s0["bytes_uploaded"]) / 1e9 / steps, 4)},
    }


# the rocprofv3 PMC runs behind roofline.traffic, per workload (profiles/traffic.json)
TRAFFIC_KEYS = {"single1": ("fused_layer", "profiles/fused_layer_traffic.md"),
                "stacked48": ("fused_layer_stacked48", "profiles/fused_layer_stacked48_traffic.md")}


def fused_report(kt, n_tok, workload="stacked48"):
    """Roofline of the fused layer launch (router rows + the resident experts'
    bytes it reads, over its dispatch-stamped duration).  traffic: this run's
    bytes per launch times the (FETCH_SIZE + WRITE_SIZE) / algorithmic ratio
    of the committed PMC run on the same workload (on the 48-layer decode for a
    workload without one of its own)."""
    n = max(kt["n_layers"], 1)
    ms, hb, pb = kt["layer_ms"], kt["layer_hbm_bytes"], kt["layer_host_bytes"]
    achieved = hb / (ms * 1e-3) / 1e9 if ms > 0 else 0.0
    traffic, tsrc = None, None
    key, doc = TRAFFIC_KEYS.get(workload, TRAFFIC_KEYS["stacked48"])
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f).get(key)
        if tr:
            ratio = (tr["hbm_read_bytes_per_launch"] + tr["hbm_write_bytes_per_launch"]) / \
                tr["algorithmic_bytes_per_launch"]
            traffic = round(ratio * hb / n)
            tsrc = (f"pmc: this run's bytes per launch x {ratio:.3f}, the (FETCH_SIZE + WRITE_SIZE) / algorithmic "
                    f"ratio of the committed rocprofv3 run on the {key.replace('fused_layer_', '').replace('fused_layer', 'single1')} "
                    f"workload ({doc})")
    return {
        "kernels_ms_per_token": {"fused_layer": round(ms / max(n_tok, 1), 4)},
        "kernel_timing": f"HIP events stamped by each dispatch (hipExtLaunchKernelGGL) on its stream, {n_tok} "
                         f"eager tokens after the timed ones on the same cache and serving path (graph replay "
                         f"cannot carry per-kernel events)",
        "roofline": {"bound": "hbm", "kernel": "fused_layer", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": tsrc, "bytes_per_launch": round(hb / n), "avg_launch_us": round(ms / n * 1e3, 2),
                     "launches": n,
                     "bytes": "router rows (1 MiB) + the resident routed experts' weights the launch reads "
                              "(2,654,208 B per expert with Q4_K down, 3,059,712 with Q6_K); absent experts are "
                              "computed by the host and not read"},
        "pcie_bytes_per_launch": round(pb / n),
    }


def window(s0, s1, steps, t0_s=None):
    """Cache and throughput figures between two stats snapshots."""
    seen = (s1["n_hit"] - s0["n_hit"]) + (s1["n_miss"] - s0["n_miss"])
    return {"hit_rate": round((s1["n_hit"] - s0["n_hit"]) / max(seen, 1), 4),
            "missed_per_token": round((s1["n_miss"] - s0["n_miss"]) / steps, 2),
            "uploaded_per_token": round((s1["n_scheduled"] - s0["n_scheduled"]) / steps, 2),
            "evicted_per_token": round((s1["n_evicted"] - s0["n_evicted"]) / steps, 2),
            "admit_denied_per_token": round((s1["n_admit_denied"] - s0["n_admit_denied"]) / steps, 2),
            "cpu_served_per_token": round((s1["n_cpu_served"] - s0["n_cpu_served"]) / steps, 2),
            "publication_wait_ms_per_token": round((s1["publication_wait_us"] - s0["publication_wait_us"])
                                                   / 1e3 / steps, 4),
            "host_boundary_ms_per_token": round((s1["host_boundary_us"] - s0["host_boundary_us"]) / 1e3 / steps, 4)}


def run_default(args):
    """Configuration 2 as the line's value, steady state, GPU-only, the
    oracle check, the fused launch's roofline, the CPU baseline, then
    configurations 3, 1, 4 and 5 as keys."""
    import numpy as np
    T_SEQ, STEADY0 = 512, 64
    wl = Workload(args, steer=True, T=T_SEQ)
    T = wl.T
    W, Kt = args.warmup, args.steps
    knobs = dict(admit=args.admit)
    cache = wl.cache(**knobs)
    cache.set_decode_path(split=args.path, graph=True)
    sidecar_setup(args, cache)
    ids_log = np.empty((T, wl.NL, K), np.int32)
    kept = {}
    keep = {W, W + Kt - 1, T - 1}
    snaps = {}
    wl.tokens(cache, 0, W, ids_log, keep, kept)
    snaps[W] = cache.stats()
    log(f"[bench] warmup {W} tokens done; timing {Kt}")
    el = wl.tokens(cache, W, W + Kt, ids_log, keep, kept)
    snaps[W + Kt] = cache.stats()
    log(f"[bench] timed {Kt} tokens in {el:.3f}s")
    # the rest of the 512-token sequence; tokens 64..511 are the steady window
    s_lo = max(STEADY0, W + Kt)
    if s_lo > W + Kt:
        wl.tokens(cache, W + Kt, s_lo, ids_log, keep, kept)
    snaps[s_lo] = cache.stats()
    el_s = wl.tokens(cache, s_lo, T, ids_log, keep, kept) if T > s_lo else 0.0
    snaps[T] = cache.stats()
    frames = [cache.frame(l) for l in range(wl.NL)]
    sc = args.sidecar > 0
    result = {
        "metric": METRIC, "value": round(Kt / el, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": Kt, "warmup": W, "ms_per_step": round(1e3 * el / Kt, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8_k int8-dot, fp32 scale (router fp32)",
        "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K/Q6_K, N(0,1) activations)",
        "config": {"workload": f"stacked{wl.NL} (configuration 2): {wl.NL} layers x {E} experts, H {H}, I {I}, "
                               f"top-{K}, {wl.slots} HBM slots/layer over a pinned store of all experts, Q6_K down "
                               f"in odd layers, Zipf(1.1) reuse 0.6, admission {args.admit}, batched tables; "
                               + (f"experts absent from the slots computed by the host CPU ({args.sidecar} threads, "
                                  f"share {args.share}), resident ones by the GPU" if sc else
                                  "absent experts read by the GPU from the pinned store over PCIe")
                               + f"; tokens {W}..{W + Kt - 1} of a {T}-token sequence timed ({W} warmup, cache "
                                 f"still filling)",
                   "batch": 1, "layers": wl.NL, "slots": wl.slots},
        "decode_path": {0: "fused layer launch", 1: "fork/join", 2: "serial", 3: "unfused"}[args.path]
                       + ", HIP graph per token",
        "cache": window(snaps[W], snaps[W + Kt], Kt),
    }
    if T > s_lo:
        result["steady"] = {"tokens": f"{s_lo}..{T - 1}", "value": round((T - s_lo) / el_s, 2), "unit": "tok/s",
                            "ms_per_token": round(1e3 * el_s / (T - s_lo), 4), **window(snaps[s_lo], snaps[T], T - s_lo)}
    result["sidecar"] = sidecar_report(args, snaps[W], snaps[W + Kt], Kt,
                                       cache.sidecar_log() if sc else None)
    kt, n_kt = wl.kernel_pass(cache, split=args.path, keep_serving=sc)
    result.update(fused_report(kt, n_kt) if args.path == 0 else kernel_report(kt, n_kt, Kt, snaps[W], snaps[W + Kt]))
    result["roofline"]["size_matched"] = size_matched(result["roofline"])
    cache.close()
    if not args.no_check:
        log("[bench] checking the 512-token run against the oracle (outside the timed regions)")
        result["check"] = wl.check(ids_log, kept, frames, snaps[T], knobs)
        result["check"]["tokens"] = T
        log(f"[bench] check: {result['check']}")
    if sc and not args.no_gpu_only:
        log("[bench] the same decode with the GPU alone serving absent experts")
        c2 = wl.cache(**knobs)
        c2.set_decode_path(split=args.path, graph=True)
        ids2 = np.empty_like(ids_log)
        wl.tokens(c2, 0, W, ids2)
        e1 = wl.tokens(c2, W, W + Kt, ids2)
        if s_lo > W + Kt:
            wl.tokens(c2, W + Kt, s_lo, ids2)
        g0 = c2.stats()
        e2 = wl.tokens(c2, s_lo, T, ids2) if T > s_lo else 0.0
        g1 = c2.stats()
        c2.close()
        result["gpu_only"] = {"value": round(Kt / e1, 2), "unit": "tok/s",
                              "steady": {"tokens": f"{s_lo}..{T - 1}",
                                         "value": round((T - s_lo) / e2, 2) if e2 else None, **window(g0, g1, T - s_lo)}
                              if T > s_lo else None,
                              "ids_equal": bool((ids2 == ids_log).all()),
                              "path": "absent experts read by the fused launch from the pinned store over PCIe "
                                      "(and staged, so their uploads are HBM copies)"}
    up = upload_cost(max(wl.eb))
    up["in_decode"] = wl.upload_in_decode
    up["context"] = "reference: 85.8 us per 3.06 MB expert pinned on a dedicated stream, RTX 5070 PCIe"
    result["uploads"] = up
    if not args.no_per_layer:
        result["per_layer"] = run_per_layer(args, wl, knobs, W, Kt, s_lo, T, ids_log)
    if not args.no_cpu:
        result["cpu_baseline"] = wl.cpu_baseline(args.cpu_seconds)
    if not args.no_extra:
        result["config3"] = config3(args, wl)
    wl.close()
    del wl
    if not args.no_extra:
        result["config1"] = config1(args)
        result["config4"] = config4(args)
        result["config5"] = config5(args)
    return result


def run_per_layer(args, wl, knobs, W, Kt, s_lo, T, ids_tok):
    """Configuration 2 decoded as a model drives the per-layer op
    (moe_decode_layer per layer, x_{l+1} = x_l + out_l, observe, step): the
    same windows as the token figures, the fused launch's time per layer from
    a timing pass after the sequence, and the oracle's check of the whole
    sequence (every layer's routing against the inputs the chain produced)."""
    import numpy as np
    torch = wl.torch
    c = wl.cache(**knobs)
    c.set_decode_path(split=args.path, graph=False)
    sidecar_setup(args, c)
    xin = torch.empty((T, wl.NL, H), dtype=torch.float32, device=wl.dev)
    outs = torch.empty((T, wl.NL, H), dtype=torch.float32, device=wl.dev)
    ids = np.empty((T, wl.NL, K), np.int32)
    log("[bench] per-layer decode (moe_decode_layer, residual inputs)")
    wl.tokens_per_layer(c, 0, W, ids, xin, outs)
    a0 = c.stats()
    el = wl.tokens_per_layer(c, W, W + Kt, ids, xin, outs)
    a1 = c.stats()
    if s_lo > W + Kt:
        wl.tokens_per_layer(c, W + Kt, s_lo, ids, xin, outs)
    b0 = c.stats()
    el_s = wl.tokens_per_layer(c, s_lo, T, ids, xin, outs) if T > s_lo else 0.0
    b1 = c.stats()
    frames = [c.frame(l) for l in range(wl.NL)]
    res = {"value": round(Kt / el, 2), "unit": "tok/s", "tokens": f"{W}..{W + Kt - 1}",
           "hit_rate": window(a0, a1, Kt)["hit_rate"]}
    if T > s_lo:
        res["steady"] = {"tokens": f"{s_lo}..{T - 1}", "value": round((T - s_lo) / el_s, 2),
                         "hit_rate": window(b0, b1, T - s_lo)["hit_rate"]}
    if not args.no_check:
        keep = {W, T - 1}
        kept = {t: outs[t].cpu().numpy() for t in keep}
        log("[bench] per-layer: checking every routed id and two tokens' outputs against the oracle")
        chk = wl.check(ids, kept, frames, b1, knobs, every=True, x_host=xin.cpu().numpy())
        res["check"] = compact_check(chk)
    del xin, outs
    # the fused launch's time per layer, a timing pass over the sequence's first tokens again
    n = min(args.kernel_steps, 64)
    c.set_timing(True)
    xin = torch.empty((n, wl.NL, H), dtype=torch.float32, device=wl.dev)
    outs = torch.empty((n, wl.NL, H), dtype=torch.float32, device=wl.dev)
    wl.tokens_per_layer(c, 0, n, np.empty((n, wl.NL, K), np.int32), xin, outs)
    kt = c.kernel_times()
    c.close()
    res["fused_us"] = round(kt["layer_ms"] / max(kt["n_layers"], 1) * 1e3, 2)
    res["fused_gbs"] = round(kt["layer_hbm_bytes"] / max(kt["layer_ms"] * 1e-3, 1e-12) / 1e9, 1)
    log(f"[bench] per-layer: {res}")
    return res


def compact_check(c):
    """A check result in a few characters: ids checked/mismatched, frames and
    counters equal, outputs checked and the worst relative L2."""
    out = {"ids": f"{c.get('ids_checked', 0)}/{c.get('ids_mismatched', 0)}",
           "outputs": f"{c.get('outputs_checked', 0)}, worst rel-L2 {c.get('worst_rel_l2', 0.0):.2g}"}
    if "frames_equal" in c:
        out["frames_counters_equal"] = bool(c["frames_equal"] and c.get("counters_equal", True))
    return out


def _sub(args, **kw):
    a = argparse.Namespace(**vars(args))
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def config3(args, wl):
    """Cache-aware routing on the single-layer shape stacked 48 deep (no
    steering), 512 tokens: delta 0, 0.01 on probabilities, 0.01 on logits."""
    r = run_prior(_sub(args, warmup=64, steps=448), wl, steer=False)
    runs = r["runs"]
    out = {"workload": "single-layer shape (N(0,0.02) router, no steering) stacked 48 deep over 56 slots, "
                       "512 tokens; hit rate over tokens 64..511",
           "delta0_hit_rate": runs["delta0"]["cache"]["hit_rate"]}
    for name in ("delta0.01", "delta0.01_logits"):
        out[name] = {"hit_rate": runs[name]["cache"]["hit_rate"], "delta_hit": runs[name]["hit_rate_change"],
                     "rel_l2_vs_delta0": round(runs[name]["rel_l2_vs_delta0"], 4), "tok_s": runs[name]["tok_s"]}
    out["check"] = {n: runs[n].get("check") for n in runs}
    return out


def config1(args):
    r = run_single(_sub(args, warmup=8, steps=256))
    keep = ("value", "unit", "config", "roofline", "step", "check")
    return {k: r[k] for k in keep if k in r}


def config4(args):
    out = {}
    for B in (512, 64):
        r = run_prefill(_sub(args, layers=48, batch=B, warmup=2, steps=10, no_cpu=True))
        out[f"batch{B}"] = {"tok_s": r["value"], "ms_per_chunk": r["ms_per_step"], "roofline": r["roofline"],
                            "mfma": r["mfma"], "hbm": r["hbm"], "check": r.get("check")}
    out["workload"] = ("48 batched layers, all 128 experts in HBM; 512-token prefill chunk and 64-token decode batch "
                       "(bf16 N(0,1) activations, uniform router logits, top-8): route, dispatch, grouped up/gate + "
                       "SwiGLU and down on fp16 matrix cores (exact integer products), combine; HIP graph per chunk")
    return out


def config5(args):
    a = _sub(args, layers=40, slots=96, warmup=64, steps=960, batch=16, batch_tokens=128)
    wl = Workload(a, steer=True, n_experts=256, inter=512, shared=True, zipf_s=1.0, reuse=0.5,
                  batch_tokens=a.batch_tokens)
    try:
        r = run_wide(a, wl)
    finally:
        wl.close()
    return {"workload": r["config"]["workload"], "batch1": {"tok_s": r["value"], "cache": r["cache"]},
            "batch16": r["batch16"], "check": r.get("check"),
            "roofline": r.get("roofline")}


def sidecar_setup(args, cache):
    if args.sidecar > 0:
        num, den = (int(v) for v in args.share.split("/"))
        cache.set_sidecar(args.sidecar, (num, den))


def sidecar_report(args, s0, s1, steps, log_rows=None):
    if args.sidecar <= 0:
        return {"threads": 0}
    extra = {}
    if log_rows is not None and len(log_rows):
        import numpy as np
        for n in (1, 2, 3):
            sel = log_rows[log_rows[:, 2] == n]
            if len(sel):
                extra[f"cpu_us_{n}_experts_p50_p90_max"] = [round(float(np.percentile(sel[:, 1], q)), 1)
                                                           for q in (50, 90, 100)]
        extra["wait_us_p50_p90_max"] = [round(float(np.percentile(log_rows[:, 0], q)), 1) for q in (50, 90, 100)]
    return {"threads": args.sidecar, "share": args.share, **extra,
            "cpu_served_per_token": round((s1["n_cpu_served"] - s0["n_cpu_served"]) / steps, 2),
            "host_wait_ms_per_token": round((s1["sidecar_wait_us"] - s0["sidecar_wait_us"]) / 1e3 / steps, 4),
            "host_cpu_ms_per_token": round((s1["sidecar_cpu_us"] - s0["sidecar_cpu_us"]) / 1e3 / steps, 4),
            "path": "absent experts assigned to the host computed by its CPU team (AVX-512 VNNI integer dots) "
                    "from the pinned store while the GPU runs the rest; posted / joined through mapped memory"}


def lookahead_compare(args, wl):
    """Router lookahead + just-in-time streaming (LLAMA_MOE_STREAM) on the
    residual-stream workload: the same decode with streaming on and off (CPU-
    assisted serving and early issue in both), same stores and routers as
    stacked48.  Returns the 'lookahead' object (stream-on tok/s and the
    comparison, the mover's counters per token, what it achieved)."""
    import numpy as np
    x, g = wl.residual()
    knobs = dict(admit=args.admit, early_issue=True)
    runs = {}
    T = args.warmup + args.steps
    keep = {args.warmup, T - 1}
    for on in (True, False):
        c = wl.cache(**knobs)
        for l in range(wl.NL):
            c.set_norm(l, g[l])
        c.set_decode_path(split=args.path, graph=True)
        if args.sidecar > 0:
            num, den = (int(v) for v in args.share.split("/"))
            c.set_sidecar(max(1, args.sidecar - 1) if on else args.sidecar, (num, den))   # the mover takes a core
        if on:
            c.set_streaming(True, per_layer=args.stream_per_layer, reserve=args.stream_reserve, top_k=8,
                            gbps=args.stream_gbps, chunk_kib=args.stream_chunk_kib)
        log(f"[bench] lookahead: residual48 decode, streaming {'on' if on else 'off'}")
        el, s0, s1, ids, kept, frames = wl.decode(c, keep=keep, x=x, steer=False)
        ss = c.stream_stats() if on else None
        runs[on] = (el, s0, s1, ids, kept, ss)
        c.close()
    el_on, s0, s1, ids_on, kept_on, ss = runs[True]
    el_off, o0, o1, ids_off, kept_off, _ = runs[False]
    steps = args.steps
    check = {"ids_checked": 0, "ids_mismatched": 0, "outputs_checked": 0, "outputs_bit_exact": True}
    if not args.no_check:
        # the oracle on the kept tokens, every layer (outside the timed regions)
        import ctypes
        from oracle import oracle as O
        Wh, xh = wl.W.cpu().numpy(), x.cpu().numpy()
        stores = [np.ctypeslib.as_array((ctypes.c_uint8 * (wl.E * wl.eb[l])).from_address(wl.stores[l]))
                  for l in range(wl.NL)]
        for t in sorted(keep):
            for l in range(wl.NL):
                rids, rw, _, _ = O.route(Wh[l], xh[t, l], K)
                check["ids_checked"] += 1
                check["ids_mismatched"] += int(not np.array_equal(rids, ids_on[t, l]))
                want = wl.oracle_layer(stores, l, rids, rw, xh[t, l], 8)
                check["outputs_checked"] += 1
                check["outputs_bit_exact"] &= bool(np.array_equal(kept_on[t][l], want))
    per = {k: round(ss[k] / T, 3) for k in ("offered", "landed", "in_time", "late", "unused", "dropped_late",
                                            "dropped_posted", "not_sent", "gpu_miss")}
    served = ss["in_time"] / max(1, ss["in_time"] + ss["gpu_miss"])
    res = {
        "workload": f"residual48: stacked48's shape and stores ({args.layers} layers x {E} experts, {args.slots} "
                    f"slots), routed by the routers on a synthetic residual stream (MU 1.2, RHO 0.7, BETA 0.975, "
                    f"norm weights 1 + 0.1 N(0,1)); early issue, admission {args.admit}, "
                    + ("CPU-assisted serving" if args.sidecar > 0 else "absent experts read by the GPU over PCIe"),
        "value": round(steps / el_on, 2), "unit": "tok/s",
        "stream_off": round(steps / el_off, 2),
        "speedup": round(el_off / el_on, 4),
        "ids_equal": bool((ids_on == ids_off).all()),
        "outputs_equal": bool(all(np.array_equal(kept_on[t], kept_off[t]) for t in keep)),
        "check": check,
        "hit_rate_on": cache_summary(s0, s1, steps)["hit_rate"],
        "hit_rate_off": cache_summary(o0, o1, steps)["hit_rate"],
        "stream_per_token": per,
        "served_from_vram": round(served, 4),
        "landed_used_in_time": round(ss["in_time"] / max(1, ss["landed"]), 4),
        "copied_mib_per_token": round(ss["bytes"] / T / 1048576, 2),
        "lead_us_d1_d2": [round(v, 1) for v in ss["lead_us"]],
        "tau_us": round(ss["tau_us"], 1),
        "failed": int(ss["failed"]),
        "knobs": {"per_layer": args.stream_per_layer, "reserve": args.stream_reserve, "top_k": 8,
                  "gbps": args.stream_gbps, "chunk_kib": args.stream_chunk_kib,
                  "sidecar_threads_on_off": [max(1, args.sidecar - 1) if args.sidecar > 0 else 0, args.sidecar]},
    }
    log(f"[bench] lookahead: {res['value']} tok/s on, {res['stream_off']} off; served from VRAM "
        f"{res['served_from_vram']}, landed used {res['landed_used_in_time']}")
    return res


def run_residual(args, wl):
    """The lookahead workload as the line's own metric: residual48 with
    streaming on, with the comparison against streaming off."""
    la = lookahead_compare(args, wl)
    wl.x = wl.x_res                     # the CPU baseline routes the same inputs
    T = args.warmup + args.steps
    return {
        "metric": "MoE decode tok/s @bs1 (48 layers, 56 slots), router lookahead + just-in-time streaming",
        "value": la["value"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 / la["value"], 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k/q6_k x q8_k int8-dot, fp32 scale (router fp32)",
        "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K/Q6_K, residual-stream router inputs)",
        "config": {"workload": la["workload"] + f", {T} tokens ({args.warmup} warmup)", "batch": 1,
                   "layers": args.layers, "slots": args.slots},
        "lookahead": la,
    }


def run_prior(args, wl, steer=False):
    """The three cache-prior runs over tokens [0, warmup + steps) of wl (no
    steering): delta 0, delta 0.01 on the selection probabilities (the
    reference's LLAMA_MOE_CACHE_PRIOR), delta 0.01 on the logits; each id of
    each run replayed through the oracle with the oracle's own tables."""
    import numpy as np
    torch = wl.torch
    W, T = args.warmup, args.warmup + args.steps
    runs, outs = {}, {}
    for name, knobs in (("delta0", dict(admit=args.admit)),
                        ("delta0.01", dict(admit=args.admit, cache_prior=0.01)),
                        ("delta0.01_logits", dict(admit=args.admit, cache_prior=0.01, prior_space="logits"))):
        log(f"[bench] cache prior run {name}")
        cache = wl.cache(**knobs)
        cache.set_decode_path(split=args.path, graph=True)
        sidecar_setup(args, cache)
        all_out = torch.empty((T, wl.NL, H), dtype=torch.float32, device=wl.dev)
        ids_log = np.empty((T, wl.NL, K), np.int32)
        kept = {}
        wl.tokens(cache, 0, W, ids_log, all_out=all_out, steer=steer)
        s0 = cache.stats()
        elapsed = wl.tokens(cache, W, T, ids_log, keep={T - 1}, kept=kept, all_out=all_out, steer=steer)
        s1 = cache.stats()
        frames = [cache.frame(l) for l in range(wl.NL)]
        r = {"tok_s": round(args.steps / elapsed, 2), "cache": cache_summary(s0, s1, args.steps),
             "hit_rate_all_tokens": round(s1["n_hit"] / max(s1["n_hit"] + s1["n_miss"], 1), 4)}
        if not args.no_check:
            log(f"[bench] {name}: replaying every routed id through the oracle")
            r["check"] = wl.check(ids_log, kept, frames, s1, knobs, every=True, steer=steer, T=T)
            log(f"[bench] check: {r['check']}")
        runs[name], outs[name] = r, all_out
        cache.close()
    ref = outs["delta0"].double()
    for name in ("delta0.01", "delta0.01_logits"):
        runs[name]["rel_l2_vs_delta0"] = float(torch.linalg.norm(outs[name].double() - ref) / torch.linalg.norm(ref))
        runs[name]["hit_rate_change"] = round(runs[name]["cache"]["hit_rate"] - runs["delta0"]["cache"]["hit_rate"], 4)
    main_run = runs["delta0.01"]
    return {
        "metric": METRIC, "value": main_run["tok_s"], "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(1e3 / main_run["tok_s"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "q4_k/q6_k x q8_k int8-dot, fp32 scale (router fp32)",
        "data": "synthetic (seeded N(0,0.02) router and experts, N(0,1) activations, no steering)",
        "config": {"workload": f"prior{wl.NL}: single-layer shape stacked {wl.NL} deep, {wl.slots} "
                               f"slots/layer, admission {args.admit}, batched tables, {T} tokens ({args.warmup} "
                               f"warmup); delta 0, 0.01 on probabilities (value), 0.01 on logits",
                   "batch": 1, "layers": wl.NL, "slots": wl.slots, "cache_prior": 0.01},
        "runs": runs,
    }


def run_single(args):
    """Configuration 1: one layer with all 128 experts resident (a heat-file
    warm start puts every expert in a slot), independent batch-1 decode steps
    on N(0,1) inputs (router N(0,0.02), no steering), GPU only.  The roofline
    is the fused layer launch's: 21,233,664 expert bytes (8 Q4_K experts) +
    1 MiB of router per step over its dispatch-stamped duration."""
    import tempfile
    import numpy as np
    # one layer: the timing pass affords as many launches as the timed steps
    a = _sub(args, layers=1, slots=E, sidecar=0, kernel_steps=max(args.kernel_steps, args.steps))
    wl = Workload(a, steer=False)
    try:
        cache = wl.cache(admit="window")
        # every expert with a count (halved on load, so >= 2), hottest first
        # the cache saves its counts back to its heat file (on close, and every
        # 512 steps), so the oracle's check warm-starts from a copy of it
        heat_text = f"moe-heat 1 1 {E}\n" + "".join(f"0 {e} {2 * (E - e)}\n" for e in range(E))
        with tempfile.NamedTemporaryFile("w", suffix=".heat", delete=False) as f:
            f.write(heat_text)
            hp = f.name
        with tempfile.NamedTemporaryFile("w", suffix=".heat", delete=False) as f:
            f.write(heat_text)
            hp_check = f.name
        n_rec, n_placed = cache.heat_file(hp)
        if n_placed != E:
            raise RuntimeError(f"warm start placed {n_placed} of {E} experts")
        cache.set_decode_path(split=0, graph=True)
        T, W = wl.T, a.warmup
        ids_log = np.empty((T, 1, K), np.int32)
        kept = {}
        wl.tokens(cache, 0, W, ids_log)
        s0 = cache.stats()
        el = wl.tokens(cache, W, T, ids_log, keep={W, T - 1}, kept=kept)
        s1 = cache.stats()
        frames = [cache.frame(0)]
        kt, n_kt = wl.kernel_pass(cache, split=0)
        rep = fused_report(kt, n_kt, "single1")
        n = max(kt["n_layers"], 1)
        us = kt["layer_ms"] / n * 1e3
        expert_bytes = K * wl.eb[0]
        out = {"value": round(a.steps / el, 1), "unit": "steps/s",
               "config": {"workload": f"one layer x {E} experts all resident, H {H}, I {I}, top-{K}, Q4_K gate/up/down, "
                                      f"router N(0,0.02), x N(0,1); {a.steps} independent steps timed ({W} warmup)"},
               "step": {"us_wall": round(1e6 * el / a.steps, 2), "hit_rate": window(s0, s1, a.steps)["hit_rate"],
                        "what": "decode_token per step: the layer launched directly (graph mode launches tokens of at most 8 layers directly), routed ids back, cache step"},
               "roofline": {**rep["roofline"], "expert_bytes_per_step": expert_bytes,
                            "expert_gbs": round(expert_bytes / (us * 1e-6) / 1e9, 1),
                            "expert_frac": round(expert_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}}
        out["roofline"]["size_matched"] = size_matched(out["roofline"])
        cache.close()
        if not args.no_check:
            out["check"] = wl.check(ids_log, kept, frames, s1, dict(admit="window"), every=True, steer=False,
                                    heat=hp_check)
        os.unlink(hp)
        os.unlink(hp_check)
        return out
    finally:
        wl.close()


def run_wide(args, wl):
    """256 routed experts + 1 shared per layer: --warmup + --steps tokens at
    batch 1, then the next tokens --batch at a time through moe_decode_batch,
    on the same cache (delta = 0.01 on selection probabilities, window
    admission)."""
    B = args.batch
    knobs = dict(admit=args.admit, cache_prior=0.01)
    cache = wl.cache(**knobs)
    cache.set_decode_path(split=args.path, graph=True)
    sidecar_setup(args, cache)
    if args.sidecar > 0 and args.batch_share:
        cache.set_sidecar_batch(tuple(int(v) for v in args.batch_share.split("/")))
    T1, n_b = wl.T1, wl.T - wl.T1
    el1, s0, s1, ids_log, kept, _ = wl.decode(cache, keep={args.warmup, T1 - 1})
    el2, per, s2, s3, ids_b, kept_b = wl.decode_batches(cache, B, keep={T1, wl.T - 1})
    ids_log[T1:] = ids_b
    kept.update(kept_b)
    frames = [cache.frame(l) for l in range(wl.NL)]
    result = {
        "metric": f"MoE decode tok/s @bs1 ({wl.NL} layers x {wl.E} experts + shared, {wl.slots} slots) + achieved "
                  f"HBM GB/s; cache hit %",
        "value": round(args.steps / el1, 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * el1 / args.steps, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "q4_k/q6_k x q8_k int8-dot, fp32 scale (router fp32)",
        "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K/Q6_K, N(0,1) activations)",
        "config": {"workload": f"wide{wl.NL}: {wl.NL} layers x {wl.E} routed experts + 1 shared (HBM), H {H}, "
                               f"I {wl.I}, top-{K}, {wl.slots} HBM slots/layer over a pinned store, Q6_K down in "
                               f"odd layers, Zipf({wl.zipf_s}) reuse {wl.reuse}, delta 0.01, admission "
                               f"{args.admit}, batched tables; {T1} tokens at batch 1 ({args.warmup} warmup), "
                               f"then {n_b} at batch {B}",
                   "batch": 1, "layers": wl.NL, "slots": wl.slots, "cache_prior": 0.01},
        "decode_path": {0: "fused", 1: "fork/join", 2: "serial"}[args.path] + " expert launches, HIP graph per token",
        "cache": cache_summary(s0, s1, args.steps),
        "sidecar": sidecar_report(args, s0, s1, args.steps),
        f"batch{B}": {"tok_s": round(n_b / el2, 2), "tokens": n_b, "ms_per_batch": per,
                      "cache": cache_summary(s2, s3, n_b),
                      "path": "moe_decode_batch: route, dispatch, grouped up/gate + SwiGLU and down on the matrix "
                              "cores from slots" + (
                                  "; the pairs of experts absent from the slots computed by the host CPU team from "
                                  "the pinned store while the GPU runs the rest, their rows combined in k order"
                                  if args.sidecar > 0 else " or the pinned store") +
                              ", shared expert, combine; ids back, one cache step per batch (batch buffers "
                              "allocated in the first call)"},
    }
    if args.sidecar > 0:
        nb_ = max(n_b // B, 1)
        result[f"batch{B}"]["sidecar"] = {"share": args.batch_share or args.share,
            "cpu_pairs_per_token": round((s3["n_cpu_served"] - s2["n_cpu_served"]) / n_b, 2),
            "host_wait_ms_per_batch": round((s3["sidecar_wait_us"] - s2["sidecar_wait_us"]) / 1e3 / nb_, 3),
            "host_cpu_ms_per_batch": round((s3["sidecar_cpu_us"] - s2["sidecar_cpu_us"]) / 1e3 / nb_, 3)}
    result[f"batch{B}"]["kernels"] = grouped_report(wl.batch_kernel_pass(cache, B), wl.I)
    # the batch-1 launches as the timed decode ran them (the fused launch, the
    # host serving its share of the absent experts)
    kt, n_kt = wl.kernel_pass(cache, split=args.path, keep_serving=args.sidecar > 0)
    result.update(fused_report(kt, n_kt) if args.path == 0 else kernel_report(kt, n_kt, args.steps, s0, s1))
    result["roofline"]["size_matched"] = size_matched(result["roofline"])
    if not args.no_check:
        log("[bench] replaying every routed id of both phases through the oracle (outside the timed region)")
        result["check"] = wl.check(ids_log, kept, frames, s3, knobs, every=True, batch=B)
        log(f"[bench] check: {result['check']}")
    cache.close()
    return result


MFMA_PEAK_TFLOPS = 2500.0   # dense fp16/bf16


def grouped_report(kt, inter):
    """GB/s and matrix-core utilisation of the batched decode's grouped
    launches: weights read once per expert with pairs on the GPU (slots in HBM,
    or the pinned store over PCIe), useful FLOPs 2 x pairs x (2 I H) up/gate and
    2 x pairs x I H down."""
    n = max(kt["grouped_launches"], 1)
    out = {"launches": kt["grouped_launches"], "pairs_per_launch": round(kt["grouped_pairs"] / n, 1)}
    for part, ms, hb, pb, fl in (("gateup", kt["grouped_gateup_ms"], kt["grouped_gateup_hbm_bytes"],
                                  kt["grouped_gateup_host_bytes"], 4 * inter * H),
                                 ("down", kt["grouped_down_ms"], kt["grouped_down_hbm_bytes"],
                                  kt["grouped_down_host_bytes"], 2 * inter * H)):
        sec = max(ms * 1e-3, 1e-12)
        tfl = fl * kt["grouped_pairs"] / sec / 1e12
        out[part] = {"us": round(ms / n * 1e3, 2), "hbm_mb": round(hb / n / 1e6, 2), "pcie_mb": round(pb / n / 1e6, 2),
                     "gbs": round((hb + pb) / sec / 1e9, 1), "hbm_frac": round((hb + pb) / sec / 1e9 / HBM_PEAK_GBS, 4),
                     "tflops": round(tfl, 2), "mfma_util": round(tfl / MFMA_PEAK_TFLOPS, 4)}
    return out


def run_prefill(args):
    """Batched MoE layers: a chunk of --batch tokens (bf16 N(0,1) activations,
    seeded uniform router logits, top-8 of 128) through --layers layers whose
    128 experts all sit in HBM.  A step = route -> dispatch -> grouped experts
    -> combine for every layer, replayed as one HIP graph."""
    import numpy as np
    import torch
    import moe_prefetch
    from moe_prefetch import _lib
    from moe_prefetch.batched import BatchedMoe
    from moe_prefetch.workload import KIND_X, down_types
    L = moe_prefetch.lib()
    dev = torch.device("cuda:0")
    NL, T = args.layers, args.batch
    dts = down_types(NL)
    eb = [L.moe_expert_bytes(H, I, dt) for dt in dts]
    t0 = time.time()
    log(f"[bench] prefill setup: {NL} layers x {E} experts in HBM ({sum(eb) * E / 1e9:.2f} GB), chunk {T}")
    stream = torch.cuda.current_stream().cuda_stream
    stores = []
    for l in range(NL):
        st = torch.empty(E * eb[l], dtype=torch.uint8, device=dev)
        _lib.check(L.moe_synth_experts(args.seed, l, 0, E, H, I, dts[l], 0.02, st.data_ptr(), eb[l], stream), "synth")
        stores.append(st)
    xs = torch.empty((T, NL, H), dtype=torch.float32, device=dev)
    _lib.check(L.moe_synth_vec(args.seed, KIND_X, 0, T, 0, NL, H, 1.0, xs.data_ptr(), stream), "x")
    x = xs.transpose(0, 1).contiguous().to(torch.bfloat16)           # [L][T][H] bf16
    del xs
    lg = torch.empty((T, NL, E), dtype=torch.float32, device=dev)
    _lib.check(L.moe_synth_vec(args.seed, 2, 0, T, 0, NL, E, 1.0, lg.data_ptr(), stream), "logits")
    logits = lg.transpose(0, 1).contiguous()                         # [L][T][E]
    del lg
    out = torch.empty((NL, T, H), dtype=torch.float32, device=dev)
    bm = BatchedMoe(T, E, K, H, I)
    torch.cuda.synchronize()
    log(f"[bench] setup done in {time.time() - t0:.1f}s")

    def step(st):
        for l in range(NL):
            bm.route(T, logits=logits[l], stream=st)
            bm.dispatch(T, stream=st)
            bm.experts(x[l], out[l], T, stores[l].data_ptr(), eb[l], E, dts[l], stream=st)

    for _ in range(2):
        step(stream)
    torch.cuda.synchronize()
    g = None
    try:
        cap = torch.cuda.Stream()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(cap):
            with torch.cuda.graph(g, stream=cap):
                step(cap.cuda_stream)
        torch.cuda.synchronize()
    except Exception as ex:        # capture refused: time eager launches instead
        log(f"[bench] graph capture failed ({ex}); timing eager launches")
        g = None
        torch.cuda.synchronize()
    run = g.replay if g is not None else (lambda: step(stream))
    for _ in range(args.warmup):
        run()
    torch.cuda.synchronize()
    log(f"[bench] timing {args.steps} chunks ({'graph' if g is not None else 'eager'})")
    t1 = time.perf_counter()
    for _ in range(args.steps):
        run()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t1
    tok_s = T * args.steps / elapsed

    # per-kernel durations (HIP events stamped by the dispatches), one eager pass
    gu_ms = dn_ms = 0.0
    touched = pairs = 0
    gu_bytes = dn_bytes = 0
    counts_all = []
    for l in range(NL):
        bm.route(T, logits=logits[l], stream=stream)
        c, _, _ = bm.dispatch(T, stream=stream)
        a, b = bm.experts(x[l], out[l], T, stores[l].data_ptr(), eb[l], E, dts[l], timing=True, stream=stream)
        gu_ms += a
        dn_ms += b
        cnt = c.cpu().numpy()
        counts_all.append(cnt)
        n_t = int((cnt > 0).sum())
        touched += n_t
        pairs += int(cnt.sum())
        gu_bytes += n_t * 2 * I * (H // 256) * 144
        dn_bytes += n_t * (eb[l] - 2 * I * (H // 256) * 144)
    gu_flops = 2.0 * pairs * 2 * I * H
    dn_flops = 2.0 * pairs * I * H
    torch.cuda.synchronize()
    gu_gbs = gu_bytes / (gu_ms * 1e-3) / 1e9
    dn_gbs = dn_bytes / (dn_ms * 1e-3) / 1e9
    dom = "gateup_grouped" if gu_ms >= dn_ms else "down_grouped"
    d_ms, d_bytes, d_flops = (gu_ms, gu_bytes, gu_flops) if dom == "gateup_grouped" else (dn_ms, dn_bytes, dn_flops)
    result = {
        "metric": f"MoE batched tok/s ({NL} layers, {T}-token chunk) + achieved HBM GB/s; MFMA utilisation",
        "value": round(tok_s, 1), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "q4_k/q6_k x q8_k on fp16 MFMA (exact integer products), fp32 scale",
        "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K/Q6_K, bf16 N(0,1) activations, uniform "
                "router logits)",
        "config": {"workload": f"prefill{NL}: {NL} layers x {E} experts in HBM, H {H}, I {I}, top-{K}, "
                               f"{T}-token chunk, Q6_K down in odd layers; route from logits, dispatch, grouped "
                               f"up/gate + SwiGLU, grouped down, combine; "
                               f"{'one HIP graph per chunk' if g is not None else 'eager launches'}",
                   "batch": T, "layers": NL},
        "kernels_ms_per_step": {"gateup_grouped": round(gu_ms, 4), "down_grouped": round(dn_ms, 4)},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(d_bytes / (d_ms * 1e-3) / 1e9, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(d_bytes / (d_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                     "bytes_per_launch": round(d_bytes / NL), "avg_launch_us": round(d_ms / NL * 1e3, 2),
                     "launches": NL},
        "mfma": {"gateup_tflops": round(gu_flops / (gu_ms * 1e-3) / 1e12, 1),
                 "down_tflops": round(dn_flops / (dn_ms * 1e-3) / 1e12, 1), "peak_tflops": MFMA_PEAK_TFLOPS,
                 "gateup_util": round(gu_flops / (gu_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                 "down_util": round(dn_flops / (dn_ms * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                 "flops": "useful: 2 x pairs x (2 I H) up/gate, 2 x pairs x I H down"},
        "hbm": {"gateup_gbs": round(gu_gbs, 1), "down_gbs": round(dn_gbs, 1),
                "experts_touched_per_layer": round(touched / NL, 1), "pairs_per_layer": pairs // NL},
    }
    # HBM bytes per launch: the (read + write) / algorithmic ratio of the rocprofv3
    # PMC runs on this chunk size (profiles/traffic.json) times this run's bytes
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tr = json.load(f).get(f"{dom}_t{T}")
        if tr:
            ratio = (tr["hbm_read_bytes_per_launch"] + tr["hbm_write_bytes_per_launch"]) / \
                tr["algorithmic_bytes_per_launch"]
            result["roofline"]["traffic"] = round(ratio * d_bytes / NL)
            result["roofline"]["traffic_source"] = (f"pmc: this run's bytes per launch x {ratio:.3f}, the "
                                                    f"(FETCH_SIZE + WRITE_SIZE) / algorithmic ratio of the committed "
                                                    f"rocprofv3 runs at {T} tokens ({tr['source']})")
    result["roofline"]["size_matched"] = size_matched(result["roofline"], iters=10)
    if not args.no_check:
        from oracle import oracle as O
        log("[bench] checking routing and dispatch of every layer, outputs of two layers, against the oracle")
        lh = logits.cpu().numpy()
        bad_ids = bad_disp = 0
        worst = 0.0
        for l in range(NL):
            bm.route(T, logits=logits[l], stream=stream)
            _, offs, perm = bm.dispatch(T, stream=stream)
            ids = bm.ids[:T].cpu().numpy()
            w = bm.w[:T].cpu().numpy()
            for t in range(T):
                oi, ow, _ = O.route_logits(lh[l, t], K)
                bad_ids += not (np.array_equal(oi, ids[t]) and ow.tobytes() == w[t].tobytes())
            oc, oo, op = O.dispatch(ids, E)
            bad_disp += not (np.array_equal(oo, offs.cpu().numpy()) and np.array_equal(op, perm.cpu().numpy()))
            if l < 2:
                bm.experts(x[l], out[l], T, stores[l].data_ptr(), eb[l], E, dts[l], stream=stream)
                got = out[l].cpu().numpy()
                want = O.moe_tokens(H, I, dts[l], stores[l].cpu().numpy(), eb[l], E, ids, w,
                                    x[l].float().cpu().numpy(), n_threads=min(len(os.sched_getaffinity(0)), 16))
                worst = max(worst, max(float(np.linalg.norm(got[t].astype(np.float64) - want[t]) /
                                             np.linalg.norm(want[t])) for t in range(T)))
        result["check"] = {"ids_mismatched_tokens": bad_ids, "dispatch_mismatched_layers": bad_disp,
                           "worst_rel_l2": worst, "outputs_checked": 2 * T}
        log(f"[bench] check: {result['check']}")
    if not args.no_cpu:
        from oracle import oracle as O
        cores = min(len(os.sched_getaffinity(0)), 16)
        host0 = stores[0].cpu().numpy()
        xh = x[0].float().cpu().numpy()
        bm.route(T, logits=logits[0], stream=stream)
        ids, w = bm.ids[:T].cpu().numpy(), bm.w[:T].cpu().numpy()
        log(f"[bench] CPU baseline: oracle batch on {cores} threads for ~{args.cpu_seconds}s")
        t2 = time.perf_counter()
        done = i0 = 0
        while time.perf_counter() - t2 < args.cpu_seconds:
            n = min(4 * cores, T - i0)
            O.moe_tokens(H, I, dts[0], host0, eb[0], E, ids[i0:i0 + n], w[i0:i0 + n], xh[i0:i0 + n],
                         n_threads=cores)
            done += n
            i0 = (i0 + n) % T
        el = time.perf_counter() - t2
        result["cpu_baseline"] = {"value": round(done / el / NL, 3), "unit": "tok/s", "cores": cores, "kind": "port",
                                  "sample": f"{done} token-layers (tokens of layer 0's chunk, cycled) through the "
                                            f"oracle's batch chain (Q8_K activations, integer dots, OpenMP over "
                                            f"tokens) in {el:.1f}s, divided by {NL} layers"}
    return result


def parse_args(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed batch-1 tokens (448; wide40: 960)")
    ap.add_argument("--warmup", type=int, default=64)
    ap.add_argument("--workload", default="stacked48",
                    choices=["stacked48", "prior48", "prefill48", "wide40", "residual48", "single1"])
    ap.add_argument("--batch", type=int, default=None, help="tokens per chunk (prefill48: 512) or per batched "
                                                            "decode step (wide40: 16)")
    ap.add_argument("--batch-tokens", type=int, default=128, help="wide40: tokens decoded in batches")
    ap.add_argument("--layers", type=int, default=None, help="48; wide40: 40")
    ap.add_argument("--slots", type=int, default=None, help="56; wide40: 96")
    ap.add_argument("--admit", default="window")
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--cpu-seconds", type=float, default=16.0, help="bounded CPU-baseline sample")
    ap.add_argument("--kernel-steps", type=int, default=64, help="eager tokens timed per kernel")
    ap.add_argument("--path", type=int, default=0,
                    help="0 fused layer launch, 1 fork/join, 2 serial expert launches, 3 unfused launches")
    ap.add_argument("--sidecar", type=int, default=-1,
                    help="host threads serving absent experts (0: GPU only; default: 14 on a 16-CPU host)")
    ap.add_argument("--batch-share", default="3/4", help="num/den: the host's share of absent experts in batched "
                                                          "decode (wide40's batch phase; empty: --share)")
    ap.add_argument("--share", default="1/1", help="num/den: absent experts of rank r with r %% den < num go to "
                                                   "the CPU")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="end with a plain 256 MiB device copy (scale for rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gpu-only", action="store_true", help="skip the GPU-only decode beside the default one")
    ap.add_argument("--no-per-layer", action="store_true", help="skip the decode through the per-layer op")
    ap.add_argument("--no-check", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="stacked48: only configuration 2 (no config1/3/4/5)")
    ap.add_argument("--no-lookahead", action="store_true", help="residual48: skip the streaming-off comparison")
    ap.add_argument("--stream-per-layer", type=int, default=4)
    ap.add_argument("--stream-reserve", type=int, default=2)
    ap.add_argument("--stream-gbps", type=float, default=45.7)
    ap.add_argument("--stream-chunk-kib", type=int, default=0, help="0: a whole expert per copy")
    args = ap.parse_args(argv)
    if args.sidecar < 0:
        n_cpu = len(os.sched_getaffinity(0))
        args.sidecar = 14 if n_cpu >= 16 else (n_cpu - 2 if n_cpu >= 8 else 0)
    wide = args.workload == "wide40"
    if args.steps is None:
        args.steps = 960 if wide else 448
    if args.layers is None:
        args.layers = 40 if wide else 48
    if args.slots is None:
        args.slots = 96 if wide else 56
    if args.batch is None:
        args.batch = 16 if wide else 512
    return args


# long descriptions go to stderr; the one stdout line keeps every figure and
# stays short enough for a log tail of ~10 KB
_DROP = {"what", "path", "engine", "kernel_timing", "flops", "ms_per_batch", "sweep"}


def compact(v, key=None):
    """The result without its long descriptive strings: checks as short
    summaries, the CPU sweep as [threads, experts per call, p50 us] rows,
    workload texts cut at 160 characters."""
    if isinstance(v, dict):
        if "ids_checked" in v:
            return compact_check(v)
        out = {}
        for k, x in v.items():
            if k in _DROP:
                continue
            if k == "bytes" and isinstance(x, str):
                continue
            if k == "traffic_source" and isinstance(x, str):
                out[k] = x if x.startswith("pmc") else "PMC ratio of profiles/traffic.json x bytes"
                continue
            out[k] = compact(x, k)
        if key == "cpu_baseline" and "sweep" in v:
            out["sweep_thr_experts_p50us"] = [[r["threads"], r["experts_per_call"], r["us_p50"]] for r in v["sweep"]]
        return out
    if isinstance(v, str) and key in ("workload", "sample") and len(v) > 160:
        return v[:157] + "..."
    if isinstance(v, list):
        return [compact(x) for x in v]
    return v


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode (the expert-sharded "
              "design is documented, not built); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    wide = args.workload == "wide40"
    import torch
    wl = None
    if args.workload == "stacked48":
        result = run_default(args)
    elif args.workload == "prefill48":
        result = run_prefill(args)
    elif args.workload == "single1":
        r = run_single(args)
        result = {"metric": "MoE layer steps/s (1 layer, 128 experts resident, batch 1) + achieved HBM GB/s",
                  "value": r["value"], "unit": r["unit"], "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
                  "ms_per_step": round(r["step"]["us_wall"] / 1e3, 5), "higher_is_better": True, "scaling": "weak",
                  "vs_baseline": None, "dtype": "q4_k x q8_k int8-dot, fp32 scale (router fp32)",
                  "data": "synthetic (seeded N(0,0.02) experts quantized to Q4_K, N(0,1) activations)", **r}
    elif wide:
        if args.batch_tokens % args.batch:
            sys.exit("--batch-tokens must be a multiple of --batch")
        wl = Workload(args, steer=True, n_experts=256, inter=512, shared=True, zipf_s=1.0, reuse=0.5,
                      batch_tokens=args.batch_tokens)
        result = run_wide(args, wl)
    elif args.workload == "residual48":
        wl = Workload(args, steer=False)
        result = run_residual(args, wl)
    else:
        wl = Workload(args, steer=False)
        result = run_prior(args, wl)
    if wl is not None:
        if not args.no_cpu:
            result["cpu_baseline"] = wl.cpu_baseline(args.cpu_seconds)
        wl.close()
    if args.calibrate_copy:
        src = torch.ones(256 << 20, dtype=torch.uint8, device="cuda:0")
        for _ in range(3):
            dst = src.clone()
        torch.cuda.synchronize()
        del src, dst
    log("[bench] full result: " + json.dumps(result))
    print(json.dumps(compact(result)), flush=True)


if __name__ == "__main__":
    main()
