"""The MOEP expert predictor / evictor (moe_predictor_*; the reference's
cpp/moe-predictor.cpp) against the reference's own implementation:

  * committed fixtures (tests/golden/make_moep_golden.py ran the reference's
    moe_predictor on a small synthetic MOEP file): scores, top-8 ids, the
    recall of each update and the bytes of the model after 64 SGD steps, all
    exactly;
  * where the reference tree is present, its moe_predictor built from source
    into oracle/_ref, on the reference's three shipped models
    (models/predictor-real.bin, predictor-fresh.bin, evictor-real.bin):
    scores and top-k on random id lists, an online-learning sequence (model
    bytes equal after it), and the saved file equal to the shipped one byte for
    byte (the format round-trips);
  * the loader refuses what the reference's refuses (magic, version,
    truncations, block table, trailing bytes, layer range) and never returns a
    half-loaded model.
"""
import os
import struct

import numpy as np
import pytest

from moe_prefetch.moep import MoePredictor
from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MODELS = "/root/reference/models"
REAL = ["predictor-real", "predictor-fresh", "evictor-real"]


def golden():
    z = np.load(os.path.join(GOLD, "moep_small_expected.npz"))
    cases = []
    for i in range(int(z["n_cases"])):
        lists = {n: z[f"{n}_{i}"] for n in ("prev", "cur", "below", "self_prev")}
        cases.append((int(z[f"il_{i}"]), lists, z[f"truth_{i}"]))
    return z, cases


def test_golden_scores_topk_updates_and_bytes(tmp_path):
    z, cases = golden()
    p = MoePredictor(os.path.join(GOLD, "moep_small.bin"))
    assert p.info["n_expert"] == 16 and p.info["n_present"] == 4 and not p.has_layer(2)
    for i, (il, l, _) in enumerate(cases):
        s = p.score(il, **l)
        assert np.array_equal(s.view(np.uint32), z["scores"][i].view(np.uint32)), i
        assert list(p.top_k(s, 8)) == list(z["top"][i]), i
    for i, (il, l, t) in enumerate(cases):
        assert np.float32(p.update(il, t, 0.05, **l)) == z["recall"][i], i
    out = tmp_path / "after.bin"
    p.save(out)
    assert np.array_equal(np.frombuffer(out.read_bytes(), np.uint8), z["after"])


def test_golden_file_round_trips(tmp_path):
    p = MoePredictor(os.path.join(GOLD, "moep_small.bin"))
    p.save(tmp_path / "same.bin")
    assert (tmp_path / "same.bin").read_bytes() == open(os.path.join(GOLD, "moep_small.bin"), "rb").read()


def test_top_k_ties_lower_id_first():
    p = MoePredictor(os.path.join(GOLD, "moep_small.bin"))
    s = np.zeros(16, np.float32)
    s[[3, 9, 12]] = 2.0
    s[[1, 14]] = 1.0
    assert list(p.top_k(s, 6)) == [3, 9, 12, 1, 14, 0]
    assert len(p.top_k(s, 40)) == 16


def corrupt(tmp_path, name, mutate):
    data = bytearray(open(os.path.join(GOLD, "moep_small.bin"), "rb").read())
    data = mutate(data)
    path = tmp_path / name
    path.write_bytes(bytes(data))
    return path


@pytest.mark.parametrize("name,mutate", [
    ("magic", lambda d: b"MOEQ" + d[4:]),
    ("version", lambda d: d[:4] + struct.pack("<I", 2) + d[8:]),
    ("short_header", lambda d: d[:20]),
    ("short_table", lambda d: d[:4 + 44 + 20]),
    ("block_gap", lambda d: d[:4 + 44 + 12 + 4] + struct.pack("<I", 17) + d[4 + 44 + 12 + 8:]),
    ("block_kind", lambda d: d[:4 + 44] + struct.pack("<I", 9) + d[4 + 44 + 4:]),
    ("block_size", lambda d: d[:4 + 44 + 8] + struct.pack("<I", 15) + d[4 + 44 + 12:]),
    ("short_weights", lambda d: d[:-4]),
    ("trailing", lambda d: d + b"\0"),
    ("layer_range", lambda d: d[:4 + 44 + 48] + struct.pack("<i", 9) + d[4 + 44 + 52:]),
])
def test_loader_refuses_like_the_reference(tmp_path, name, mutate):
    path = corrupt(tmp_path, name + ".bin", mutate)
    with pytest.raises(Exception):
        MoePredictor(path)
    if O.ref_predictor_lib() is not None:
        with pytest.raises(ValueError):
            O.RefPredictor(path)


# ---- against the reference's own build, on its shipped models ----------------------------
need_ref = pytest.mark.skipif(O.ref_predictor_lib() is None or not os.path.isdir(MODELS),
                              reason="the reference tree and oracle/_ref are not on this host")


def rand_lists(rng, E):
    out = {}
    for name in ("prev", "cur", "below", "self_prev"):
        out[name] = rng.choice(E, int(rng.integers(0, 9)), replace=False).astype(np.int32)
    return out


@need_ref
@pytest.mark.parametrize("name", REAL)
def test_shipped_models_score_and_round_trip(tmp_path, name):
    path = os.path.join(MODELS, name + ".bin")
    p, r = MoePredictor(path), O.RefPredictor(path)
    E = p.n_expert
    rng = np.random.default_rng(3)
    layers = [l for l in range(p.info["n_layers"]) if p.has_layer(l)]
    assert layers == [l for l in range(p.info["n_layers"]) if r.has_layer(l)]
    for c in range(300):
        il = int(rng.choice(layers))
        l = rand_lists(rng, E)
        a, b = p.score(il, **l), r.score(il, E, **l)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (name, c)
        assert list(p.top_k(a, 8)) == list(r.top_k(b, 8))
    p.save(tmp_path / "rt.bin")
    assert (tmp_path / "rt.bin").read_bytes() == open(path, "rb").read()


@need_ref
def test_shipped_model_online_learning_matches(tmp_path):
    path = os.path.join(MODELS, "predictor-fresh.bin")
    p, r = MoePredictor(path), O.RefPredictor(path)
    rng = np.random.default_rng(9)
    layers = [l for l in range(p.info["n_layers"]) if p.has_layer(l)]
    for c in range(400):
        il = int(rng.choice(layers))
        l = rand_lists(rng, p.n_expert)
        truth = rng.choice(p.n_expert, 8, replace=False).astype(np.int32)
        assert np.float32(p.update(il, truth, 0.01, **l)) == np.float32(r.update(il, truth, 0.01, **l)), c
    p.save(tmp_path / "p.bin")
    r.save(str(tmp_path / "r.bin"))
    assert (tmp_path / "p.bin").read_bytes() == (tmp_path / "r.bin").read_bytes()
