"""Synthetic decode workloads of the Qwen3-30B-A3B-shaped MoE path.

Shapes (hidden 2048, 128 experts, top-8, intermediate 768; the 256-expert
variant uses intermediate 512):

  single_layer   one layer, all 128 experts resident, x ~ N(0, 1),
                 router W ~ N(0, 0.02), experts N(0, 0.02) -> Q4_K
  stacked48      48 layers, 56 slots per layer over a pinned host store of all
                 128 experts, Q6_K down in odd layers; routing steered to a
                 per-layer Zipf(s) popularity with reuse p of the previous
                 token's experts
  prior48        the single-layer shape stacked 48 deep with the cache prior
                 delta on resident experts (no steering)
  residual48     stacked48's shape routed by the routers themselves on a
                 synthetic residual stream (no steering), so that layer L's
                 input predicts layers L+1 and L+2 as a real model's does:
                 the router lookahead workload

Residual stream (residual48): residual_{t,l} = MU m + z_{t,l} with a shared
direction m; z_{t,0} = RHO z_{t-1,0} + sqrt(1 - RHO^2) n_t and, per layer,
v_{t,l} = RHO v_{t-1,l} + sqrt(1 - RHO^2) u_{t,l}, z_{t,l} = BETA z_{t,l-1}
+ sqrt(1 - BETA^2) v_{t,l}; the router input is x_{t,l} = rmsnorm(residual)
* g_l with g_l = 1 + 0.1 N(0, 1).  BETA sets how much of layer l+1's input
layer l already holds, RHO the token-to-token reuse, MU the popularity skew.
MU 1.2, RHO 0.7, BETA 0.975 give, at 56 slots, about 20 misses per token and
a one-layer-ahead recall of 72% of the misses at 73% precision -- the
reference's probe on Qwen3-30B-A3B measured 21.4, 75% and 68%
(docs/superpowers/specs/2026-10-04-just-in-time-expert-streaming-design.md,
section 4).

Routing steering: the router still runs W x for every layer; a per-token bias
of +STEER on the 8 target experts of that (token, layer) makes them the top-8
(W x has standard deviation ~0.9, so a margin of 12 is > 10 sigma).  The
targets come from a SplitMix64 stream in this file, so any host reproduces
them without numpy's generators.
"""
import bisect
import math

import numpy as np

from . import _lib

H, E, K, I = 2048, 128, 8, 768
SIGMA_W, SIGMA_R, SIGMA_X = 0.02, 0.02, 1.0
STEER = 12.0
MASK64 = (1 << 64) - 1

# vector kinds of moe_synth_vec
KIND_ROUTER, KIND_X = 0, 1
KIND_RES_MEAN, KIND_RES_TOKEN, KIND_RES_LAYER, KIND_NORM = 3, 4, 5, 6
RESID_MU, RESID_RHO, RESID_BETA, NORM_SIGMA = 1.2, 0.7, 0.975, 0.1


class SplitMix:
    def __init__(self, seed):
        self.s = seed & MASK64

    def next(self):
        self.s = (self.s + 0x9E3779B97F4A7C15) & MASK64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK64
        return z ^ (z >> 31)

    def uniform(self):
        return (self.next() >> 11) * (1.0 / (1 << 53))


def down_types(n_layers, q6k_every_other=True):
    """Q6_K down in odd layers (the 'alternate layers' of the stacked shape)."""
    return [_lib.TYPE_Q6K if (q6k_every_other and l % 2 == 1) else _lib.TYPE_Q4K for l in range(n_layers)]


def zipf_targets(seed, layer, n_tokens, n_experts=E, k=K, s=1.1, reuse=0.6):
    """[n_tokens][k] expert ids: per-layer Zipf(s) popularity over a seeded
    permutation; each of the previous token's experts is kept with p = reuse,
    the rest are drawn from the popularity without replacement."""
    rng = SplitMix(seed * 1000003 + layer * 7919 + 17)
    perm = list(range(n_experts))
    for i in range(n_experts - 1, 0, -1):
        j = rng.next() % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    w = [1.0 / math.pow(r + 1, s) for r in range(n_experts)]
    cdf = []
    acc = 0.0
    for v in w:
        acc += v
        cdf.append(acc)
    total = acc

    def draw():
        return perm[min(bisect.bisect_right(cdf, rng.uniform() * total), n_experts - 1)]

    out = np.empty((n_tokens, k), np.int32)
    prev = []
    for t in range(n_tokens):
        cur = [e for e in prev if rng.uniform() < reuse]
        while len(cur) < k:
            e = draw()
            if e not in cur:
                cur.append(e)
        out[t] = cur
        prev = cur
    return out


def steering_bias(targets_by_layer, n_experts=E):
    """targets [L][T][k] -> bias [T][L][E] float32 (+STEER on the targets)."""
    L = len(targets_by_layer)
    T = targets_by_layer[0].shape[0]
    bias = np.zeros((T, L, n_experts), np.float32)
    for l in range(L):
        tg = targets_by_layer[l]
        for t in range(T):
            bias[t, l, tg[t]] = STEER
    return bias


def residual_stream(seed, n_tokens, n_layers, torch, device, stream_ptr, H=H, mu=RESID_MU, rho=RESID_RHO,
                    beta=RESID_BETA):
    """Router inputs x [T][L][H] f32 and norm weights g [L][H] f32 of the
    residual-stream workload, on the device (innovations from moe_synth_vec,
    recursions in elementwise f32)."""
    T, L = n_tokens, n_layers
    f32 = torch.float32

    def vec(kind, na, nb, sigma=1.0):
        out = torch.empty((na, nb, H), dtype=f32, device=device)
        _lib.check(_lib.lib().moe_synth_vec(seed, kind, 0, na, 0, nb, H, sigma, out.data_ptr(), stream_ptr),
                   "residual stream")
        return out

    m = vec(KIND_RES_MEAN, 1, 1)[0, 0]
    n_tok = vec(KIND_RES_TOKEN, T, 1)[:, 0]                  # [T][H]
    u = vec(KIND_RES_LAYER, T, L)                            # [T][L][H]
    g = 1.0 + vec(KIND_NORM, L, 1, NORM_SIGMA)[:, 0]         # [L][H]
    cr, cb = math.sqrt(1.0 - rho * rho), math.sqrt(1.0 - beta * beta)
    v = torch.empty_like(u)                                  # v[t][l], l >= 1 used
    z0 = torch.empty_like(n_tok)
    for t in range(T):
        if t == 0:
            v[0] = u[0]
            z0[0] = n_tok[0]
        else:
            v[t] = rho * v[t - 1] + cr * u[t]
            z0[t] = rho * z0[t - 1] + cr * n_tok[t]
    z = torch.empty_like(u)
    z[:, 0] = z0
    for l in range(1, L):
        z[:, l] = beta * z[:, l - 1] + cb * v[:, l]
    res = mu * m + z
    x = res * torch.rsqrt((res * res).mean(dim=2, keepdim=True)) * g
    return x.contiguous(), g.contiguous()
