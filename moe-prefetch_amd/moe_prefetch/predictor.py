"""Drop-in `ExpertPredictor` (the API of the reference's src/predictor.py:26-93).

Per-layer ridge probes over a shared PCA basis: project a hidden state onto
the basis, score experts with a per-layer (k, n_expert) matrix, take the top p.
The predictor is host-side numpy in the reference as well and is off the GPU
decode path (the reference measured it net-negative and ships it disabled);
it is kept so code written against the prototype keeps working.

Method semantics kept from the reference, including that `fit` is a
classmethod returning the (mean, comp, scale) PCA triple rather than an
instance, and that `top_p` returns the top-p set in argpartition order.
"""
import numpy as np

N_EXPERT = 128


class ExpertPredictor:
    def __init__(self, mean, comp, scale, weights):
        self.mean = mean          # (d,)
        self.comp = comp          # (d, k)
        self.scale = scale        # (k,)
        self.weights = weights    # {layer: (k, n_expert)}

    @classmethod
    def fit(cls, H, E, pairs, train_mask, n_comp=256, lam=100.0):
        """PCA basis from the hidden states that appear as training sources.

        H (n, d) hidden states; pairs = (src, dst) index arrays; train_mask over
        pairs.  Returns (mean, comp, scale): comp holds the n_comp leading
        eigenvectors of the sample covariance, scale the per-component std."""
        src, _ = pairs
        rows = np.unique(np.asarray(src)[np.asarray(train_mask)])
        X = H[rows]
        mean = X.mean(axis=0)
        Xc = X - mean
        cov = (Xc.T @ Xc) / max(len(Xc) - 1, 1)
        _, evecs = np.linalg.eigh(cov.astype(np.float64))   # ascending eigenvalues
        comp = evecs[:, ::-1][:, :n_comp].astype(np.float32)
        scale = (Xc @ comp).std(axis=0) + 1e-6
        return mean, comp, scale

    @classmethod
    def fit_layer(cls, X, Y, lam=100.0):
        """Primal ridge: (X^T X + lam I)^-1 X^T Y, as float32 (k, n_expert)."""
        k = X.shape[1]
        G = X.T @ X + lam * np.eye(k, dtype=np.float32)
        return np.linalg.solve(G, X.T @ Y).astype(np.float32)

    def project(self, h):
        return ((h - self.mean) @ self.comp) / self.scale

    def scores(self, layer, h_proj):
        W = self.weights.get(layer)
        return None if W is None else h_proj @ W

    def top_p(self, layer, h_proj, p=8):
        s = self.scores(layer, h_proj)
        if s is None:
            return np.empty(0, dtype=np.int64)
        return np.argpartition(-s, p)[:p]

    def save(self, path):
        layers = sorted(self.weights)
        np.savez_compressed(path, mean=self.mean, comp=self.comp, scale=self.scale,
                            layers=np.array(layers), stack=np.stack([self.weights[l] for l in layers]))

    @classmethod
    def load(cls, path):
        d = np.load(path)
        return cls(d["mean"], d["comp"], d["scale"],
                   {int(l): w for l, w in zip(d["layers"], d["stack"])})

    def n_params(self):
        return self.comp.size + sum(w.size for w in self.weights.values())
