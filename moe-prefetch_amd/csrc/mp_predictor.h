// mp_predictor.h -- the MOEP expert predictor / evictor on the host.
//
// Behaviour of moe_predictor (cpp/moe-predictor.h, cpp/moe-predictor.cpp of the
// reference): a per-layer linear scorer over a multi-hot feature vector made
// of expert-id lists (the next layer's ids of the previous token, this layer's
// ids, the layer below's, this layer's previous ones), z-scored per row, plus a
// repeat prior on the `prev` ids; top-k with the lower id first on a tie; one
// logistic SGD step per resolved prediction; the MOEP v3 file format, read
// strictly (every mismatch refused with a message) and written back.
//
// Arithmetic order is fixed so that results are reproducible bit for bit: the
// bias, then the selected rows in block order (prev, cur, below, self_prev)
// and list order, each row added element by element; the mean and variance
// as left-to-right sums; no fused multiply-add.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace mpp {

enum Block { BLOCK_PCA = 0, BLOCK_PREV = 1, BLOCK_CUR = 2, BLOCK_BELOW = 3, BLOCK_SELF_PREV = 4 };

struct Lists {
    const int32_t *ids[4] = {nullptr, nullptr, nullptr, nullptr};   // prev, cur, below, self_prev
    size_t n[4] = {0, 0, 0, 0};
};

class Predictor {
public:
    uint32_t n_expert = 0, n_layers = 0, feat_dim = 0, top_k = 0, d_model = 0, n_comp = 0;
    bool has_pca = false;
    int32_t off[5] = {-1, -1, -1, -1, -1};        // column offset of each block kind, -1 absent
    std::vector<float> pca_mean, pca_comp, pca_scale;
    std::vector<int32_t> layers;                  // present layers, file order
    std::vector<int32_t> slot_of;                 // layer -> index into layers, -1 absent
    std::vector<float> prior, bias, w;            // [present], [present][E], [present][feat][E]

    bool load(const std::string &path, std::string &err);
    bool save(const std::string &path, std::string &err) const;
    bool has_layer(int il) const { return il >= 0 && il < (int)slot_of.size() && slot_of[(size_t)il] >= 0; }
    void score(int il, const Lists &in, float *out) const;
    size_t top(const float *scores, size_t k, int32_t *out) const;
    // one SGD step towards `truth`; returns the recall@8 of the prediction before it
    float update(int il, const Lists &in, const int32_t *truth, size_t n_truth, float lr);
};

}  // namespace mpp
