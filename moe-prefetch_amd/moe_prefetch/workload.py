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
