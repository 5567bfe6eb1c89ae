"""The MOEP expert predictor / evictor of the reference's cache (cpp/moe-predictor.h,
cpp/moe-predictor.cpp), over the C ABI (moe_predictor_*).

Scores one layer's experts from id lists the cache already holds on the host:
`prev` (the next layer's experts of the previous token), `cur` (this layer's),
`below` (the layer below's), `self_prev` (this layer's previous ones); a model
uses the blocks its file declares.  `update` takes one logistic SGD step
towards the ids the layer then routed to and returns the recall@8 of the
prediction it learned from; `save` writes MOEP v3 back.
"""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib

BLOCKS = ("prev", "cur", "below", "self_prev")


def _lists(keep, **ids):
    l = _lib.PredictorLists()
    for b, name in enumerate(BLOCKS):
        v = ids.get(name)
        if v is None or len(v) == 0:
            l.ids[b], l.n[b] = None, 0
            continue
        a = np.ascontiguousarray(v, np.int32)
        keep.append(a)
        l.ids[b], l.n[b] = a.ctypes.data, a.size
    return l


class MoePredictor:
    def __init__(self, path):
        h = ctypes.c_void_p()
        check(lib().moe_predictor_load(str(path).encode(), ctypes.byref(h)), "moe_predictor_load")
        self.h = h.value
        i = _lib.PredictorInfo()
        check(lib().moe_predictor_info_get(self.h, ctypes.byref(i)), "moe_predictor_info_get")
        self.info = {n: getattr(i, n) for n, _ in _lib.PredictorInfo._fields_}
        self.n_expert = self.info["n_expert"]

    def close(self):
        if getattr(self, "h", None):
            lib().moe_predictor_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def has_layer(self, layer):
        return bool(lib().moe_predictor_has_layer(self.h, layer))

    def score(self, layer, **ids):
        keep = []
        l = _lists(keep, **ids)
        out = np.empty(self.n_expert, np.float32)
        check(lib().moe_predictor_score(self.h, layer, ctypes.byref(l), out.ctypes.data), "moe_predictor_score")
        return out

    def top_k(self, scores, k=8):
        s = np.ascontiguousarray(scores, np.float32)
        out = np.empty(max(k, 0), np.int32)
        n = lib().moe_predictor_top_k(self.h, s.ctypes.data, k, out.ctypes.data)
        if n < 0:
            check(n, "moe_predictor_top_k")
        return out[:n]

    def update(self, layer, truth, lr, **ids):
        keep = []
        l = _lists(keep, **ids)
        t = np.ascontiguousarray(truth, np.int32)
        r = ctypes.c_float()
        check(lib().moe_predictor_update(self.h, layer, ctypes.byref(l), t.ctypes.data, t.size, lr, ctypes.byref(r)),
              "moe_predictor_update")
        return r.value

    def save(self, path):
        check(lib().moe_predictor_save(self.h, str(path).encode()), "moe_predictor_save")
