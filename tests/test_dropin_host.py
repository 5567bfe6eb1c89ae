"""Drop-in API of the reference's Python prototypes (CPU parts) and the
synthetic routing generator."""
import numpy as np

from moe_prefetch.predictor import ExpertPredictor
from moe_prefetch.workload import SplitMix, zipf_targets
from predictor import ExpertPredictor as ShimPredictor


def test_predictor_fit_project_topp_save_load(tmp_path):
    rng = np.random.default_rng(0)
    n, d, k = 400, 64, 16
    Hs = rng.standard_normal((n, d)).astype(np.float32)
    src = np.arange(n - 1)
    dst = src + 1
    mean, comp, scale = ExpertPredictor.fit(Hs, None, (src, dst), np.ones(n - 1, bool), n_comp=k)
    assert comp.shape == (d, k) and scale.shape == (k,)
    # leading component has the largest variance
    proj = (Hs - mean) @ comp
    assert proj[:, 0].var() >= proj[:, -1].var()
    X = proj / scale
    Y = np.zeros((n, 128), np.float32)
    Y[np.arange(n), rng.integers(0, 128, n)] = 1
    W = ExpertPredictor.fit_layer(X.astype(np.float32), Y, lam=10.0)
    assert W.shape == (k, 128) and W.dtype == np.float32
    p = ExpertPredictor(mean, comp, scale, {3: W})
    hp = p.project(Hs[0])
    top = p.top_p(3, hp, p=8)
    assert len(top) == 8 and len(set(top.tolist())) == 8
    s = p.scores(3, hp)
    assert set(top.tolist()) == set(np.argsort(-s)[:8].tolist())
    assert p.top_p(5, hp).size == 0 and p.scores(5, hp) is None
    path = str(tmp_path / "pred.npz")
    p.save(path)
    q = ShimPredictor.load(path)
    assert np.array_equal(q.weights[3], W) and q.n_params() == p.n_params()


def test_zipf_targets_properties():
    T = 2000
    tg = zipf_targets(1, 0, T, s=1.1, reuse=0.6)
    assert tg.shape == (T, 8)
    assert all(len(set(r.tolist())) == 8 for r in tg)
    kept = np.mean([len(set(tg[t]) & set(tg[t - 1])) for t in range(1, T)]) / 8
    assert 0.6 <= kept < 0.75                  # p = 0.6 plus Zipf re-draws of the same experts
    counts = np.bincount(tg.reshape(-1), minlength=128)
    top = np.sort(counts)[::-1]
    assert top[0] > 10 * max(top[-1], 1)       # skewed popularity
    assert np.array_equal(tg, zipf_targets(1, 0, T, s=1.1, reuse=0.6))
    assert not np.array_equal(tg, zipf_targets(1, 1, T, s=1.1, reuse=0.6))


def test_splitmix_reference_values():
    # SplitMix64 of seed 0: the published first outputs of the generator
    r = SplitMix(0)
    assert r.next() == 0xE220A8397B1DCDAF
    assert r.next() == 0x6E789E6AA1B965F4
