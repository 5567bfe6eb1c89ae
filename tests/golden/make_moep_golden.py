"""Writes tests/golden/moep_small.bin (a small MOEP v3 model: 16 experts, 5
layers of which 4 are present, all four id blocks, a repeat prior) and
tests/golden/moep_small_expected.npz: the scores, top-8 ids, recall values and
the model bytes after a sequence of SGD updates, as the reference's own
moe_predictor (cpp/moe-predictor.cpp, built into oracle/_ref by `make -C oracle
ref`) computes them.  Run from the repository root where the reference tree is
present; the fixtures are committed."""
import os
import struct
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
E, NL, PRESENT = 16, 5, [0, 1, 3, 4]
FEAT = 4 * E


def write_model(path, seed=7):
    rng = np.random.default_rng(seed)
    with open(path, "wb") as f:
        f.write(b"MOEP")
        f.write(struct.pack("<11I", 3, 0, 0, E, NL, 8, FEAT, len(PRESENT), 4, 0, 0))
        for i, kind in enumerate((1, 2, 3, 4)):       # prev, cur, below, self_prev
            f.write(struct.pack("<3I", kind, i * E, E))
        f.write(np.asarray(PRESENT, np.int32).tobytes())
        f.write(np.asarray([0.0, 0.75, 1.5, -0.25], np.float32).tobytes())        # prior per present layer
        f.write(rng.normal(0, 0.3, (len(PRESENT), E)).astype(np.float32).tobytes())   # bias
        f.write(rng.normal(0, 0.5, (len(PRESENT), FEAT, E)).astype(np.float32).tobytes())


def cases(seed=11, n=64):
    rng = np.random.default_rng(seed)
    out = []
    for c in range(n):
        il = int(rng.choice(PRESENT))
        lists = {}
        for name in ("prev", "cur", "below", "self_prev"):
            k = int(rng.integers(0, 9))
            ids = rng.integers(-2, E + 2, k).astype(np.int32)      # out-of-range ids are skipped
            lists[name] = ids
        truth = rng.choice(E, int(rng.integers(1, 9)), replace=False).astype(np.int32)
        out.append((il, lists, truth))
    return out


def main():
    if O.ref_predictor_lib() is None:
        sys.exit("build oracle/_ref first (make -C oracle ref)")
    model = os.path.join(HERE, "moep_small.bin")
    write_model(model)
    cs = cases()
    ref = O.RefPredictor(model)
    scores = np.stack([ref.score(il, E, **l) for il, l, _ in cs])
    top = np.stack([np.pad(ref.top_k(s, 8), (0, 0)) for s in scores])
    recall = np.array([ref.update(il, t, 0.05, **l) for il, l, t in cs], np.float32)
    with tempfile.TemporaryDirectory() as d:
        p = os.path.join(d, "after.bin")
        ref.save(p)
        after = np.frombuffer(open(p, "rb").read(), np.uint8)
    flat = {}
    for i, (il, l, t) in enumerate(cs):
        flat[f"il_{i}"] = np.int32(il)
        flat[f"truth_{i}"] = t
        for name, v in l.items():
            flat[f"{name}_{i}"] = v
    np.savez_compressed(os.path.join(HERE, "moep_small_expected.npz"), scores=scores, top=top, recall=recall, after=after,
             n_cases=np.int32(len(cs)), **flat)
    print("wrote", model, "and moep_small_expected.npz")


if __name__ == "__main__":
    main()
