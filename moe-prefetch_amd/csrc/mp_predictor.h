// mp_predictor.h -- the MOEP expert predictor / evictor on the host.
//
// Behaviour of moe_predictor (cpp/moe-predictor.h, cpp/moe-predictor.cpp of the
// reference): a per-layer linear scorer over a multi-hot feature vector made
// of expert-id lists (the next layer's ids of the previous token, this layer's
// ids, the layer below's, this layer's previous ones), z-scored per row, plus a
// repeat prior on the `prev` ids; top-k with the lower id first on a tie; one
// logistic SGD step per resolved prediction; the MOEP v3 file format, read
// strictly (every file the reference's loader refuses is refused, with a
// message naming the byte offset) and written back byte for byte.
//
// Data layout: one LayerWeights per layer the file holds, each owning its
// bias and its weight rows (row c of a layer = feature column c, n_expert
// floats). A feature vector is multi-hot, so scoring a layer is the bias plus
// the rows the id lists pick; `pick` turns the lists into row numbers once and
// both scoring and the SGD step walk that list.
//
// Arithmetic order is fixed so that results are reproducible bit for bit: per
// output column, the bias, then the picked rows in group order (prev, cur,
// below, self_prev) and list order; the mean and variance as left-to-right
// sums; no fused multiply-add (the library is built with -ffp-contract=off).
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace mpp {

// Column groups of the feature vector, numbered as the file's block table
// numbers them.
enum Group : uint32_t { GROUP_PCA = 0, GROUP_PREV = 1, GROUP_CUR = 2, GROUP_BELOW = 3, GROUP_SELF_PREV = 4, N_GROUPS = 5 };

// The four id lists of one prediction, in group order prev, cur, below, self_prev.
struct Lists {
    const int32_t *ids[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t n[4] = {0, 0, 0, 0};
};

struct Shape {
    uint32_t d_model = 0, n_comp = 0, n_expert = 0, n_layers = 0, top_k = 0, feat_dim = 0;
};

struct LayerWeights {
    int32_t layer = -1;          // the model layer these weights score
    float prior = 0.0f;          // added to the z-scored score of every prev id
    std::vector<float> bias;     // [n_expert]
    std::vector<float> rows;     // [feat_dim][n_expert]
};

class Predictor {
public:
    Shape shape;
    int32_t group_col[N_GROUPS] = {-1, -1, -1, -1, -1};   // first column of each group, -1 absent
    std::vector<float> pca_mean, pca_comp, pca_scale;     // kept only to report them; never scored
    std::vector<LayerWeights> present;                    // file order
    std::vector<int32_t> slot;                            // model layer -> index into present, -1 absent

    bool has_pca() const { return group_col[GROUP_PCA] >= 0; }
    bool has_layer(int il) const { return il >= 0 && (size_t)il < slot.size() && slot[(size_t)il] >= 0; }

    // Replaces *this only when the whole file was accepted.
    bool load(const std::string &path, std::string &err);
    bool save(const std::string &path, std::string &err) const;

    void score(int il, const Lists &in, float *out) const;
    // the k best columns of `scores` (k clamped to n_expert), best first, the
    // lower id first on equal scores; a NaN score ranks with -inf
    size_t top(const float *scores, size_t k, int32_t *out) const;
    // one SGD step towards `truth`; returns the recall@8 of the prediction before it
    float update(int il, const Lists &in, const int32_t *truth, size_t n_truth, float lr);

private:
    void pick(const Lists &in, std::vector<uint32_t> &rows) const;
};

}  // namespace mpp
