"""MOEP v3 model files written for the cache-hook tests (no reference data)."""
import struct
import numpy as np


def write_moep(path, E, n_layers, present, blocks=(1, 2, 3, 4), seed=5, prior=0.6):
    """A MOEP v3 model for the rigs here: the given blocks (1 prev, 2 cur, 3
    below, 4 self_prev), weights N(0, 0.5), a repeat prior."""
    rng = np.random.default_rng(seed)
    feat = len(blocks) * E
    with open(path, "wb") as f:
        f.write(b"MOEP")
        f.write(struct.pack("<11I", 3, 0, 0, E, n_layers, 8, feat, len(present), len(blocks), 0, 0))
        for i, kind in enumerate(blocks):
            f.write(struct.pack("<3I", kind, i * E, E))
        f.write(np.asarray(present, np.int32).tobytes())
        f.write(np.full(len(present), prior, np.float32).tobytes())
        f.write(rng.normal(0, 0.3, (len(present), E)).astype(np.float32).tobytes())
        f.write(rng.normal(0, 0.5, (len(present), feat, E)).astype(np.float32).tobytes())
