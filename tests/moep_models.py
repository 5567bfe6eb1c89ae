"""MOEP v3 model files written for the cache-hook tests (no reference data)."""
import struct
import numpy as np


def write_moep(path, E, n_layers, present, blocks=(1, 2, 3, 4), seed=5, prior=0.6, pca=None):
    """A MOEP v3 model for the rigs here: the given blocks (1 prev, 2 cur, 3
    below, 4 self_prev), weights N(0, 0.5), a repeat prior.  pca=(d_model,
    n_comp): a PCA block (group 0) first, over a d_model hidden state."""
    rng = np.random.default_rng(seed)
    d_model, n_comp = pca if pca else (0, 0)
    feat = n_comp + len(blocks) * E
    with open(path, "wb") as f:
        f.write(b"MOEP")
        f.write(struct.pack("<11I", 3, d_model, n_comp, E, n_layers, 8, feat, len(present),
                            len(blocks) + (1 if pca else 0), 1 if pca else 0, 0))
        col = 0
        if pca:
            f.write(struct.pack("<3I", 0, 0, n_comp))
            col = n_comp
        for i, kind in enumerate(blocks):
            f.write(struct.pack("<3I", kind, col + i * E, E))
        if pca:
            f.write(rng.normal(0, 1, d_model + d_model * n_comp + n_comp).astype(np.float32).tobytes())
        f.write(np.asarray(present, np.int32).tobytes())
        f.write(np.full(len(present), prior, np.float32).tobytes())
        f.write(rng.normal(0, 0.3, (len(present), E)).astype(np.float32).tobytes())
        f.write(rng.normal(0, 0.5, (len(present), feat, E)).astype(np.float32).tobytes())
