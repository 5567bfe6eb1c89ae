// mp_predictor.cpp -- the MOEP expert predictor / evictor (see mp_predictor.h).
//
// File format MOEP v3, as the reference's loader reads it (cpp/moe-predictor.cpp
// load(), 21-151) and its saver writes it (save(), 318-362):
//   "MOEP", u32 version 3, d_model, n_comp, n_expert, n_layers, top_k, feat_dim,
//   n_present, n_blocks, pca_flag, reserved;
//   n_blocks x (u32 kind, offset, size): contiguous from column 0, covering
//   feat_dim; size n_comp for the PCA block, n_expert for the id blocks;
//   [pca_flag] f32 mean[d_model], comp[d_model * n_comp], scale[n_comp];
//   i32 layer[n_present], f32 prior[n_present], f32 bias[n_present][n_expert],
//   f32 w[n_present][feat_dim][n_expert]; nothing after it.
#include "mp_predictor.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <numeric>

namespace mpp {

namespace {

struct File {
    FILE *f;
    explicit File(FILE *p) : f(p) {}
    ~File() {
        if (f) fclose(f);
    }
    bool get(void *p, size_t n) { return fread(p, 1, n, f) == n; }
    bool u32(uint32_t &v) { return get(&v, 4); }
};

}  // namespace

bool Predictor::load(const std::string &path, std::string &err) {
    File in(fopen(path.c_str(), "rb"));
    if (!in.f) {
        err = "cannot open " + path;
        return false;
    }
    Predictor p;                 // filled completely before it replaces *this
    char magic[4];
    if (!in.get(magic, 4) || memcmp(magic, "MOEP", 4) != 0) {
        err = path + ": not a MOEP file";
        return false;
    }
    uint32_t version, n_present, n_blocks, pca_flag, reserved;
    if (!in.u32(version) || !in.u32(p.d_model) || !in.u32(p.n_comp) || !in.u32(p.n_expert) ||
        !in.u32(p.n_layers) || !in.u32(p.top_k) || !in.u32(p.feat_dim) || !in.u32(n_present) ||
        !in.u32(n_blocks) || !in.u32(pca_flag) || !in.u32(reserved)) {
        err = path + ": truncated header";
        return false;
    }
    if (version != 3) {
        err = path + ": version " + std::to_string(version) + ", expected 3";
        return false;
    }
    p.has_pca = pca_flag != 0;
    // the block table says which columns mean what: it must tile [0, feat_dim)
    uint32_t next = 0;
    for (uint32_t i = 0; i < n_blocks; ++i) {
        uint32_t kind, offset, size;
        if (!in.u32(kind) || !in.u32(offset) || !in.u32(size)) {
            err = path + ": truncated block table";
            return false;
        }
        if (offset != next) {
            err = path + ": block " + std::to_string(i) + " starts at " + std::to_string(offset) + ", expected " +
                  std::to_string(next);
            return false;
        }
        if (kind > BLOCK_SELF_PREV) {
            err = path + ": unknown feature block kind " + std::to_string(kind);
            return false;
        }
        const uint32_t want = kind == BLOCK_PCA ? p.n_comp : p.n_expert;
        if (size != want) {
            static const char *names[] = {"PCA", "prev", "cur", "below", "self_prev"};
            err = path + ": " + names[kind] + " block size " + std::to_string(size) + " != " + std::to_string(want);
            return false;
        }
        p.off[kind] = (int32_t)offset;
        next += size;
    }
    if (next != p.feat_dim) {
        err = path + ": blocks cover " + std::to_string(next) + " columns, feat_dim is " + std::to_string(p.feat_dim);
        return false;
    }
    if (p.has_pca != (p.off[BLOCK_PCA] >= 0)) {
        err = path + ": the PCA flag disagrees with the block table";
        return false;
    }
    if (p.has_pca) {
        p.pca_mean.resize(p.d_model);
        p.pca_comp.resize((size_t)p.d_model * p.n_comp);
        p.pca_scale.resize(p.n_comp);
        if (!in.get(p.pca_mean.data(), p.pca_mean.size() * 4) || !in.get(p.pca_comp.data(), p.pca_comp.size() * 4) ||
            !in.get(p.pca_scale.data(), p.pca_scale.size() * 4)) {
            err = path + ": truncated PCA block";
            return false;
        }
    }
    p.layers.resize(n_present);
    p.prior.resize(n_present);
    p.bias.resize((size_t)n_present * p.n_expert);
    if (!in.get(p.layers.data(), (size_t)n_present * 4) || !in.get(p.prior.data(), (size_t)n_present * 4) ||
        !in.get(p.bias.data(), p.bias.size() * 4)) {
        err = path + ": truncated layer table";
        return false;
    }
    p.w.resize((size_t)n_present * p.feat_dim * p.n_expert);
    if (!in.get(p.w.data(), p.w.size() * 4)) {
        err = path + ": truncated weights (wanted " + std::to_string(p.w.size() * 4) + " bytes)";
        return false;
    }
    char extra;
    if (fread(&extra, 1, 1, in.f) != 0) {
        err = path + ": trailing bytes after the weights";
        return false;
    }
    p.slot_of.assign(p.n_layers, -1);
    for (uint32_t i = 0; i < n_present; ++i) {
        const int32_t il = p.layers[i];
        if (il < 0 || il >= (int32_t)p.n_layers) {
            err = path + ": layer index " + std::to_string(il) + " out of range";
            return false;
        }
        p.slot_of[(size_t)il] = (int32_t)i;
    }
    *this = std::move(p);
    return true;
}

void Predictor::score(int il, const Lists &in, float *out) const {
    const int32_t slot = slot_of[(size_t)il];
    const uint32_t E = n_expert;
    const float *W = w.data() + (size_t)slot * feat_dim * E;
    memcpy(out, bias.data() + (size_t)slot * E, (size_t)E * sizeof(float));
    // x is multi-hot: x . W adds the rows its ids select, block by block
    static const int kinds[4] = {BLOCK_PREV, BLOCK_CUR, BLOCK_BELOW, BLOCK_SELF_PREV};
    for (int b = 0; b < 4; ++b) {
        const int32_t o = off[kinds[b]];
        if (o < 0) continue;
        for (size_t i = 0; i < in.n[b]; ++i) {
            const int32_t e = in.ids[b][i];
            if (e < 0 || e >= (int32_t)E) continue;
            const float *row = W + (size_t)(o + e) * E;
            for (uint32_t j = 0; j < E; ++j) out[j] += row[j];
        }
    }
    // z-score the row, then the repeat prior on the prev ids (the order the
    // prior's weight was fitted in)
    float sum = 0.0f;
    for (uint32_t j = 0; j < E; ++j) sum += out[j];
    const float mean = sum / (float)E;
    float ss = 0.0f;
    for (uint32_t j = 0; j < E; ++j) {
        const float dv = out[j] - mean;
        const float sq = dv * dv;
        ss += sq;
    }
    const float sd = std::sqrt(ss / (float)E) + 1e-9f;
    for (uint32_t j = 0; j < E; ++j) out[j] = (out[j] - mean) / sd;
    const float pw = prior[(size_t)slot];
    if (pw != 0.0f)
        for (size_t i = 0; i < in.n[0]; ++i) {
            const int32_t e = in.ids[0][i];
            if (e >= 0 && e < (int32_t)E) out[e] += pw;
        }
}

size_t Predictor::top(const float *scores, size_t k, int32_t *out) const {
    const size_t E = n_expert;
    if (k > E) k = E;
    std::vector<int32_t> order(E);
    std::iota(order.begin(), order.end(), 0);
    std::partial_sort(order.begin(), order.begin() + (ptrdiff_t)k, order.end(), [scores](int32_t a, int32_t b) {
        return scores[a] != scores[b] ? scores[a] > scores[b] : a < b;
    });
    std::copy(order.begin(), order.begin() + (ptrdiff_t)k, out);
    return k;
}

float Predictor::update(int il, const Lists &in, const int32_t *truth, size_t n_truth, float lr) {
    if (!has_layer(il) || n_truth == 0) return 0.0f;
    const int32_t slot = slot_of[(size_t)il];
    const uint32_t E = n_expert;
    std::vector<float> s(E), g(E);
    score(il, in, s.data());
    std::vector<uint8_t> y(E, 0);
    for (size_t i = 0; i < n_truth; ++i)
        if (truth[i] >= 0 && truth[i] < (int32_t)E) y[(size_t)truth[i]] = 1;
    int32_t best[8];
    const size_t nt = top(s.data(), 8, best);
    float hits = 0.0f;
    for (size_t i = 0; i < nt; ++i) hits += y[(size_t)best[i]] ? 1.0f : 0.0f;
    const float recall = hits / (float)n_truth;
    // logistic loss on the z-scored scores: d/ds = sigmoid(s) - y
    for (uint32_t j = 0; j < E; ++j) {
        const float p = 1.0f / (1.0f + std::exp(-s[j]));
        g[j] = (p - (y[j] ? 1.0f : 0.0f)) * lr;
    }
    float *W = w.data() + (size_t)slot * feat_dim * E;
    static const int kinds[4] = {BLOCK_PREV, BLOCK_CUR, BLOCK_BELOW, BLOCK_SELF_PREV};
    for (int b = 0; b < 4; ++b) {
        const int32_t o = off[kinds[b]];
        if (o < 0) continue;
        for (size_t i = 0; i < in.n[b]; ++i) {
            const int32_t e = in.ids[b][i];
            if (e < 0 || e >= (int32_t)E) continue;
            float *row = W + (size_t)(o + e) * E;
            for (uint32_t j = 0; j < E; ++j) row[j] -= g[j];
        }
    }
    float *bb = bias.data() + (size_t)slot * E;
    for (uint32_t j = 0; j < E; ++j) bb[j] -= g[j];
    return recall;
}

bool Predictor::save(const std::string &path, std::string &err) const {
    if (has_pca) {
        err = "a predictor with a PCA block is not saved (the cache never uses one)";
        return false;
    }
    FILE *f = fopen(path.c_str(), "wb");
    if (!f) {
        err = "cannot open " + path + " for writing";
        return false;
    }
    bool ok = true;
    auto put = [&](const void *p, size_t n) { ok = ok && fwrite(p, 1, n, f) == n; };
    auto u32 = [&](uint32_t v) { put(&v, 4); };
    std::vector<std::pair<int32_t, uint32_t>> blocks;      // (offset, kind), in column order
    for (uint32_t kind = BLOCK_PREV; kind <= BLOCK_SELF_PREV; ++kind)
        if (off[kind] >= 0) blocks.push_back({off[kind], kind});
    std::sort(blocks.begin(), blocks.end());
    put("MOEP", 4);
    for (uint32_t v : {3u, d_model, n_comp, n_expert, n_layers, top_k, feat_dim, (uint32_t)layers.size(),
                       (uint32_t)blocks.size(), 0u, 0u})
        u32(v);
    for (const auto &b : blocks) {
        u32(b.second);
        u32((uint32_t)b.first);
        u32(n_expert);
    }
    put(layers.data(), layers.size() * 4);
    put(prior.data(), prior.size() * 4);
    put(bias.data(), bias.size() * 4);
    put(w.data(), w.size() * 4);
    if (fclose(f) != 0) ok = false;
    if (!ok) err = "short write to " + path;
    return ok;
}

}  // namespace mpp
