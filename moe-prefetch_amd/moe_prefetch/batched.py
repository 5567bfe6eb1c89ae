"""The batched MoE layer (prefill chunks, decode at batch > 1) over the C ABI.

    route     moe_route: softmax / top-k / renormalised weights of W.x, or of
              given logits (build_moe_ffn's router at n_tokens > 1)
    dispatch  moe_dispatch: per-expert histogram, exclusive scan and the stable
              permutation of the (token, k) pairs -- the row mapping ggml's
              mul_mat_id builds (patches/0008-fused-cpu-moe-rows.patch:157-167)
    experts   moe_grouped_experts: Q8_K of x, up/gate per expert on the matrix
              cores with the SwiGLU, Q8_K of h, down times the gate weight,
              and the sum over k in order (patches/0009-moe-sidecar.patch:697-703)

Device buffers are torch tensors (torch is only the allocator here); every
computation is the library's.
"""
import ctypes

import torch

from . import _lib
from ._lib import check, lib

DTYPES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16}


def _ptr(t):
    if t is None:
        return None
    if isinstance(t, int):
        return t
    return t.data_ptr()


class BatchedMoe:
    def __init__(self, n_tok_max, n_experts=128, n_expert_used=8, hidden=2048, intermediate=768, device=0):
        self.T, self.E, self.K, self.H, self.I = n_tok_max, n_experts, n_expert_used, hidden, intermediate
        dev = torch.device("cuda", device)
        self.dev = dev
        i32, f32 = torch.int32, torch.float32
        self.ids = torch.empty((n_tok_max, n_expert_used), dtype=i32, device=dev)
        self.w = torch.empty((n_tok_max, n_expert_used), dtype=f32, device=dev)
        self.slots = torch.empty((n_tok_max, n_expert_used), dtype=i32, device=dev)
        self.counts = torch.empty(n_experts, dtype=i32, device=dev)
        self.offsets = torch.empty(n_experts + 1, dtype=i32, device=dev)
        self.perm = torch.empty(n_tok_max * n_expert_used, dtype=i32, device=dev)
        self.route_ws = torch.zeros(lib().moe_route_workspace_bytes(n_experts, n_tok_max), dtype=torch.uint8,
                                    device=dev)
        self.q8x = torch.empty((n_tok_max, hidden // 256 * 292), dtype=torch.uint8, device=dev)
        ws = lib().moe_grouped_workspace_bytes(n_tok_max, n_expert_used, hidden, intermediate)
        self.ws = torch.empty(ws, dtype=torch.uint8, device=dev)

    def route(self, n_tok, logits=None, W=None, x=None, bias=None, prior=None, table=None, stream=None):
        """ids/w for n_tok tokens from given logits [n_tok][E], or from W [E][H] . x [n_tok][H] (f32)."""
        if n_tok > self.T:
            raise ValueError(f"n_tok {n_tok} > {self.T}")
        d = _lib.RouteDesc(_ptr(W), _ptr(x), _ptr(bias), _ptr(prior), _ptr(table), self.E, 0, self.E, self.H,
                           self.K, n_tok, _ptr(self.ids), _ptr(self.w), _ptr(self.slots), None,
                           _ptr(self.q8x) if logits is None else None, _ptr(self.route_ws), _ptr(logits))
        check(lib().moe_route(ctypes.byref(d), _ptr(stream)), "moe_route")
        return self.ids[:n_tok], self.w[:n_tok]

    def dispatch(self, n_tok, ids=None, stream=None):
        ids = self.ids if ids is None else ids
        check(lib().moe_dispatch(_ptr(ids), n_tok, self.K, self.E, _ptr(self.counts), _ptr(self.offsets),
                                 _ptr(self.perm), _ptr(stream)), "moe_dispatch")
        return self.counts, self.offsets, self.perm[:n_tok * self.K]

    def experts(self, x, out, n_tok, store, expert_bytes, n_store, down_type, w=None, table=None, slot_pool=None,
                slot_bytes=0, n_slots=0, accumulate=False, pair_out=None, h_out=None, timing=False, stream=None):
        """x [n_tok][H] f32 or bf16 on the device; out [n_tok][H] f32.  store: device address of
        [n_store][expert_bytes] (HBM, or pinned memory through moe_host_device_ptr).  With timing,
        returns the (up/gate, down) kernel milliseconds."""
        w = self.w if w is None else w
        ms = (ctypes.c_float * 2)() if timing else None
        d = _lib.GroupedDesc(_ptr(self.offsets), _ptr(self.perm), _ptr(w), _ptr(x), DTYPES[x.dtype], n_tok,
                             self.K, self.E, self.H, self.I, down_type, _ptr(table), _ptr(slot_pool), slot_bytes,
                             n_slots, _ptr(store), expert_bytes, n_store, _ptr(out), int(accumulate),
                             _ptr(pair_out), _ptr(h_out), _ptr(self.ws),
                             ctypes.cast(ms, ctypes.c_void_p) if timing else None)
        check(lib().moe_grouped_experts(ctypes.byref(d), _ptr(stream)), "moe_grouped_experts")
        return (ms[0], ms[1]) if timing else None

    def forward(self, x, out, store, expert_bytes, n_store, down_type, logits=None, W=None, xf32=None, bias=None,
                stream=None, **kw):
        """route -> dispatch -> experts for x.shape[0] tokens."""
        n_tok = x.shape[0]
        self.route(n_tok, logits=logits, W=W, x=xf32, bias=bias, stream=stream)
        self.dispatch(n_tok, stream=stream)
        return self.experts(x, out, n_tok, store, expert_bytes, n_store, down_type, stream=stream, **kw)

