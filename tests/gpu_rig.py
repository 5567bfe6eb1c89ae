"""Shared set-up of the GPU parity tests: seeded synthetic experts in pinned
host stores (written by the device generator through their mapped addresses),
router weights, activations and optional Zipf steering on the device, and a
MoeCache over them.  The oracle side reads the same bytes back on the host."""
import ctypes

import numpy as np
import torch

import moe_prefetch
from moe_prefetch import MoeCache, _lib
from moe_prefetch.workload import KIND_ROUTER, KIND_X, residual_stream, steering_bias, zipf_targets
from oracle import oracle as O

H, E, K = 2048, 128, 8


def L():
    return moe_prefetch.lib()


def stream():
    return torch.cuda.current_stream().cuda_stream


class Pinned:
    """moe_host_alloc'd memory with a numpy view and its device address."""

    def __init__(self, nbytes):
        self.n = nbytes
        self.ptr = L().moe_host_alloc(nbytes)
        assert self.ptr, L().moe_last_error()
        self.arr = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(self.ptr))
        self.dev = L().moe_host_device_ptr(self.ptr)
        assert self.dev, L().moe_last_error()

    def free(self):
        if self.ptr:
            self.arr = None
            L().moe_host_free(self.ptr)
            self.ptr = None


def synth_experts_dev(seed, layer, e0, n, I, dt, out_ptr, stride):
    _lib.check(L().moe_synth_experts(seed, layer, e0, n, H, I, dt, 0.02, out_ptr, stride, stream()), "synth")


class Rig:
    def __init__(self, slots, down_types, T, I=768, seed=42, steer=True, zipf_s=1.1, reuse=0.6, E=E, shared=False,
                 residual=False, skip_router=(), **knobs):
        self.nl = len(slots)
        self.slots, self.down_types, self.T, self.I, self.seed = list(slots), list(down_types), T, I, seed
        self.E = E
        self.dev = torch.device("cuda:0")
        self.eb = [L().moe_expert_bytes(H, I, dt) for dt in self.down_types]
        self.stores = []
        self.shared = []        # per layer: uint8 tensor in HBM (expert index E of the generator) or None
        for l in range(self.nl):
            st = Pinned(E * self.eb[l])
            synth_experts_dev(seed, l, 0, E, I, self.down_types[l], st.dev, self.eb[l])
            self.stores.append(st)
            if shared:
                sh = torch.empty(self.eb[l], dtype=torch.uint8, device=self.dev)
                synth_experts_dev(seed, l, E, 1, I, self.down_types[l], sh.data_ptr(), self.eb[l])
                self.shared.append(sh)
            else:
                self.shared.append(None)
        self.W = torch.empty((self.nl, E, H), dtype=torch.float32, device=self.dev)
        _lib.check(L().moe_synth_vec(seed, KIND_ROUTER, 0, self.nl, 0, E, H, 0.02, self.W.data_ptr(), stream()), "W")
        self.g = None
        if residual:            # routing by the routers on a residual stream (lookahead workload)
            self.x, self.g = residual_stream(seed, T, self.nl, torch, self.dev, stream())
            steer = False
        else:
            self.x = torch.empty((T, self.nl, H), dtype=torch.float32, device=self.dev)
            _lib.check(L().moe_synth_vec(seed, KIND_X, 0, T, 0, self.nl, H, 1.0, self.x.data_ptr(), stream()), "x")
        self.bias = None
        if steer:
            tg = [zipf_targets(seed, l, T, n_experts=E, s=zipf_s, reuse=reuse) for l in range(self.nl)]
            self.bias = torch.from_numpy(steering_bias(tg, n_experts=E)).to(self.dev)
        torch.cuda.synchronize()
        self.knobs = knobs
        self.cache = MoeCache(self.nl, n_experts=E, intermediate=I, slot_profile=self.slots,
                              down_types=self.down_types, device=0, **knobs)
        for l in range(self.nl):
            self.cache.set_host_store(l, self.stores[l].ptr)
            if l not in skip_router:
                self.cache.set_router(l, self.W[l])
            if self.shared[l] is not None:
                self.cache.set_shared(l, self.shared[l])
            if self.g is not None:
                self.cache.set_norm(l, self.g[l].cpu().numpy())
        self.shared_h = [None if sh is None else sh.cpu().numpy() for sh in self.shared]
        self.Wh = self.W.cpu().numpy()
        self.xh = self.x.cpu().numpy()
        self.bh = None if self.bias is None else self.bias.cpu().numpy()

    def run(self, tokens=None, keep_out=None):
        tokens = range(self.T) if tokens is None else tokens
        ids_all, outs, frames = {}, {}, {}
        out = torch.empty((self.nl, H), dtype=torch.float32, device=self.dev)
        for t in tokens:
            b = None if self.bias is None else self.bias[t]
            ids_all[t] = self.cache.decode_token(self.x[t], out, bias=b, stream=stream()).copy()
            frames[t] = [self.cache.frame(l) for l in range(self.nl)]
            if keep_out is None or t in keep_out:
                outs[t] = out.cpu().numpy().copy()
        return ids_all, outs, frames

    def oracle_cache(self):
        kn = dict(self.knobs)
        kn.pop("prior_space", None)         # the space only changes the routing (O.route's prior_on_logits)
        kn.setdefault("admit", "off")
        return O.Cache(self.slots, n_experts=self.E, **kn)

    def oracle_layer(self, t, l, ids, w, x=None):
        """Routed experts in k order, then the shared expert with weight 1."""
        st, eb = self.stores[l].arr, self.eb[l]
        experts = [st[e * eb:(e + 1) * eb] for e in ids]
        w = list(w)
        if self.shared_h[l] is not None:
            experts.append(self.shared_h[l])
            w.append(1.0)
        return O.moe_layer(H, self.I, self.down_types[l], experts, np.asarray(w, np.float32),
                           self.xh[t, l] if x is None else x)

    def prior_on_logits(self):
        return self.knobs.get("prior_space") == "logits"

    def close(self):
        self.cache.close()
        for s in self.stores:
            s.free()
