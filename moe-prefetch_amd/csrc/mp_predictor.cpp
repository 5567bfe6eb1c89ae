// mp_predictor.cpp -- the MOEP expert predictor / evictor (behaviour of the
// reference's cpp/moe-predictor.cpp: load() 21-155, score() 165-222,
// top_k_ids() 224-238, update() 241-309, save() 318-362).
//
// MOEP v3, little-endian, as the reference's loader and saver define it:
//   "MOEP", then eleven u32: version (3), d_model, n_comp, n_expert, n_layers,
//   top_k, feat_dim, n_present, n_blocks, pca_flag, reserved;
//   n_blocks x (u32 group, first column, width), the groups laid end to end
//   from column 0 up to feat_dim, width n_comp for the PCA group and n_expert
//   for the id groups (a group named twice keeps its last entry);
//   when pca_flag is set: f32 mean[d_model], comp[d_model][n_comp], scale[n_comp];
//   i32 layer[n_present], f32 prior[n_present], f32 bias[n_present][n_expert],
//   f32 w[n_present][feat_dim][n_expert], and nothing after it.
//
// The loader reads the file whole, checks the header and the block table,
// derives from them the size the file must have and compares it with the size
// it has (a short or an over-long file is refused by that one test), then
// splits the sections. Every refusal names the byte offset it concerns.
#include "mp_predictor.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

namespace mpp {

namespace {

const char *const kGroupName[N_GROUPS] = {"PCA", "prev", "cur", "below", "self_prev"};
constexpr uint32_t kVersion = 3;

struct Refused {
    std::string why;
};

std::string at_byte(size_t off) { return "byte " + std::to_string(off) + ": "; }

// The file's bytes and a read position; a read past the end is a refusal
// that names what was being read.
class Image {
public:
    bool open(const std::string &path) {
        FILE *f = fopen(path.c_str(), "rb");
        if (!f) return false;
        uint8_t chunk[1 << 16];
        size_t got;
        while ((got = fread(chunk, 1, sizeof chunk, f)) > 0) bytes_.insert(bytes_.end(), chunk, chunk + got);
        const bool ok = !ferror(f);
        fclose(f);
        return ok;
    }
    size_t size() const { return bytes_.size(); }
    size_t at() const { return at_; }
    const uint8_t *take(size_t n, const char *what) {
        if (bytes_.size() - at_ < n)
            throw Refused{at_byte(bytes_.size()) + "the file ends inside the " + what};
        const uint8_t *p = bytes_.data() + at_;
        at_ += n;
        return p;
    }
    uint32_t u32(const char *what) {
        uint32_t v;
        memcpy(&v, take(4, what), 4);
        return v;
    }
    template <class T>
    void fill(std::vector<T> &dst, size_t n, const char *what) {
        dst.resize(n);
        if (n) memcpy(dst.data(), take(n * sizeof(T), what), n * sizeof(T));
    }

private:
    std::vector<uint8_t> bytes_;
    size_t at_ = 0;
};

// Byte counts the header implies, refused when they do not fit a size_t.
size_t mul(size_t a, size_t b) {
    if (a != 0 && b > SIZE_MAX / a) throw Refused{"the header describes more data than can be addressed"};
    return a * b;
}
size_t add(size_t a, size_t b) {
    if (b > SIZE_MAX - a) throw Refused{"the header describes more data than can be addressed"};
    return a + b;
}

// Order-preserving 32-bit image of a score: a larger score has a larger key,
// -0 and +0 are equal, and a NaN is equal to -inf.
uint32_t order_bits(float s) {
    if (s != s) s = -INFINITY;
    if (s == 0.0f) s = 0.0f;
    uint32_t b;
    memcpy(&b, &s, 4);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

}  // namespace

bool Predictor::load(const std::string &path, std::string &err) {
    Image im;
    if (!im.open(path)) {
        err = "cannot read " + path;
        return false;
    }
    Predictor p;
    try {
        if (memcmp(im.take(4, "magic"), "MOEP", 4) != 0) throw Refused{at_byte(0) + "the magic is not MOEP"};
        uint32_t h[11];
        for (uint32_t &v : h) v = im.u32("header");
        const uint32_t version = h[0], n_present = h[7], n_blocks = h[8], pca_flag = h[9];
        if (version != kVersion)
            throw Refused{at_byte(4) + "format version " + std::to_string(version) + ", this loader reads " +
                          std::to_string(kVersion)};
        p.shape = Shape{h[1], h[2], h[3], h[4], h[5], h[6]};

        // the block table: which feature columns hold which group
        uint64_t column = 0;
        for (uint32_t i = 0; i < n_blocks; ++i) {
            const size_t entry = im.at();
            const uint32_t group = im.u32("block table"), first = im.u32("block table"),
                           width = im.u32("block table");
            if (first != column)
                throw Refused{at_byte(entry) + "block " + std::to_string(i) + " begins at column " +
                              std::to_string(first) + " where the previous blocks end at " + std::to_string(column)};
            if (group >= N_GROUPS)
                throw Refused{at_byte(entry) + "block " + std::to_string(i) + " names group " +
                              std::to_string(group) + ", known groups are 0.." + std::to_string(N_GROUPS - 1)};
            const uint32_t want = group == GROUP_PCA ? p.shape.n_comp : p.shape.n_expert;
            if (width != want)
                throw Refused{at_byte(entry) + "the " + kGroupName[group] + " block is " + std::to_string(width) +
                              " columns wide, the header implies " + std::to_string(want)};
            p.group_col[group] = (int32_t)first;
            column = (uint32_t)(column + width);     // the 32-bit sum the format's own offsets use
        }
        if (column != p.shape.feat_dim)
            throw Refused{at_byte(im.at()) + "the blocks cover " + std::to_string(column) +
                          " columns, the header's feat_dim is " + std::to_string(p.shape.feat_dim)};
        if ((pca_flag != 0) != p.has_pca())
            throw Refused{at_byte(40) + "pca_flag " + std::to_string(pca_flag) +
                          (p.has_pca() ? " but the block table has a PCA block"
                                       : " but the block table has no PCA block")};

        // the size every later section fixes, checked before any is split off
        const size_t E = p.shape.n_expert;
        const size_t pca_floats =
            pca_flag ? add(add(p.shape.d_model, mul(p.shape.d_model, p.shape.n_comp)), p.shape.n_comp) : 0;
        const size_t per_layer = add(add(2, E), mul(p.shape.feat_dim, E));    // layer id, prior, bias, rows
        const size_t want = add(im.at(), mul(4, add(pca_floats, mul(n_present, per_layer))));
        if (im.size() != want)
            throw Refused{at_byte(std::min(im.size(), want)) + "the file is " + std::to_string(im.size()) +
                          " bytes, its header and block table describe " + std::to_string(want)};

        if (pca_flag) {
            im.fill(p.pca_mean, p.shape.d_model, "PCA mean");
            im.fill(p.pca_comp, (size_t)p.shape.d_model * p.shape.n_comp, "PCA components");
            im.fill(p.pca_scale, p.shape.n_comp, "PCA scale");
        }
        const size_t tables = im.at();
        std::vector<int32_t> layer;
        std::vector<float> prior;
        im.fill(layer, n_present, "layer list");
        im.fill(prior, n_present, "prior list");
        p.present.resize(n_present);
        p.slot.assign(p.shape.n_layers, -1);
        for (uint32_t i = 0; i < n_present; ++i) {
            LayerWeights &lw = p.present[i];
            lw.layer = layer[i];
            lw.prior = prior[i];
            if (lw.layer < 0 || lw.layer >= (int64_t)p.shape.n_layers)
                throw Refused{at_byte(tables + 4 * (size_t)i) + "layer " + std::to_string(lw.layer) +
                              " is outside the model's " + std::to_string(p.shape.n_layers) + " layers"};
            p.slot[(size_t)lw.layer] = (int32_t)i;     // a layer listed twice scores with its last entry
        }
        for (LayerWeights &lw : p.present) im.fill(lw.bias, E, "biases");
        for (LayerWeights &lw : p.present) im.fill(lw.rows, (size_t)p.shape.feat_dim * E, "weights");
    } catch (const Refused &r) {
        err = "MOEP " + path + ", " + r.why;
        return false;
    }
    *this = std::move(p);
    return true;
}

void Predictor::pick(const Lists &in, std::vector<uint32_t> &rows) const {
    static const Group kOrder[4] = {GROUP_PREV, GROUP_CUR, GROUP_BELOW, GROUP_SELF_PREV};
    const int32_t E = (int32_t)shape.n_expert;
    rows.clear();
    for (int b = 0; b < 4; ++b) {
        const int32_t col = group_col[kOrder[b]];
        if (col < 0) continue;
        for (size_t i = 0; i < in.n[b]; ++i) {
            const int32_t e = in.ids[b][i];
            if (e >= 0 && e < E) rows.push_back((uint32_t)(col + e));
        }
    }
}

void Predictor::score(int il, const Lists &in, float *out) const {
    const LayerWeights &lw = present[(size_t)slot[(size_t)il]];
    const size_t E = shape.n_expert;
    std::vector<uint32_t> rows;
    pick(in, rows);
    // x . W for a multi-hot x: per column, the bias plus the picked rows
    for (size_t j = 0; j < E; ++j) {
        float acc = lw.bias[j];
        for (uint32_t r : rows) acc += lw.rows[(size_t)r * E + j];
        out[j] = acc;
    }
    // z-score over the row, then the repeat prior (the prior's weight was
    // fitted on z-scored scores)
    float total = 0.0f;
    for (size_t j = 0; j < E; ++j) total += out[j];
    const float mean = total / (float)E;
    float ss = 0.0f;
    for (size_t j = 0; j < E; ++j) ss += (out[j] - mean) * (out[j] - mean);
    const float sd = std::sqrt(ss / (float)E) + 1e-9f;
    for (size_t j = 0; j < E; ++j) out[j] = (out[j] - mean) / sd;
    if (lw.prior == 0.0f) return;          // adding +0 would turn a -0 score into +0
    const int32_t *prev = in.ids[0];
    for (size_t i = 0; i < in.n[0]; ++i)
        if (prev[i] >= 0 && prev[i] < (int32_t)E) out[prev[i]] += lw.prior;
}

size_t Predictor::top(const float *scores, size_t k, int32_t *out) const {
    const size_t E = shape.n_expert;
    k = std::min(k, E);
    // one 64-bit key per column, score bits above the complemented id, so that
    // a descending sort puts the larger score first and, on equal scores, the
    // lower id first
    std::vector<uint64_t> key(E);
    for (size_t e = 0; e < E; ++e) key[e] = (uint64_t)order_bits(scores[e]) << 32 | (0xffffffffu - (uint32_t)e);
    std::partial_sort(key.begin(), key.begin() + (ptrdiff_t)k, key.end(), [](uint64_t a, uint64_t b) { return a > b; });
    for (size_t i = 0; i < k; ++i) out[i] = (int32_t)(0xffffffffu - (uint32_t)key[i]);
    return k;
}

float Predictor::update(int il, const Lists &in, const int32_t *truth, size_t n_truth, float lr) {
    if (!has_layer(il) || n_truth == 0) return 0.0f;
    LayerWeights &lw = present[(size_t)slot[(size_t)il]];
    const size_t E = shape.n_expert;
    std::vector<float> s(E);
    score(il, in, s.data());
    std::vector<char> hit(E, 0);
    for (size_t i = 0; i < n_truth; ++i)
        if (truth[i] >= 0 && (size_t)truth[i] < E) hit[(size_t)truth[i]] = 1;
    // recall@8 of the prediction the step corrects, over every truth entry given
    int32_t best[8];
    float found = 0.0f;
    for (size_t i = 0, n = top(s.data(), 8, best); i < n; ++i) found += hit[(size_t)best[i]] ? 1.0f : 0.0f;
    // logistic loss on the z-scored scores: the step is lr * (sigmoid(s) - y)
    std::vector<float> step(E);
    for (size_t j = 0; j < E; ++j) step[j] = (1.0f / (1.0f + std::exp(-s[j])) - (hit[j] ? 1.0f : 0.0f)) * lr;
    std::vector<uint32_t> rows;
    pick(in, rows);
    for (uint32_t r : rows) {
        float *row = lw.rows.data() + (size_t)r * E;
        for (size_t j = 0; j < E; ++j) row[j] -= step[j];
    }
    for (size_t j = 0; j < E; ++j) lw.bias[j] -= step[j];
    return found / (float)n_truth;
}

bool Predictor::save(const std::string &path, std::string &err) const {
    if (has_pca()) {
        err = "MOEP " + path + ": not written, the model has a PCA block (scoring never uses it, so a "
              "written copy could not be checked against the model that wrote it)";
        return false;
    }
    // the id groups in column order
    std::vector<uint32_t> groups;
    for (uint32_t g = GROUP_PREV; g < N_GROUPS; ++g)
        if (group_col[g] >= 0) groups.push_back(g);
    std::sort(groups.begin(), groups.end(), [this](uint32_t a, uint32_t b) { return group_col[a] < group_col[b]; });

    std::vector<uint8_t> buf;
    auto put = [&buf](const void *p, size_t n) {
        const uint8_t *b = (const uint8_t *)p;
        buf.insert(buf.end(), b, b + n);
    };
    auto word = [&put](uint32_t v) { put(&v, 4); };
    put("MOEP", 4);
    for (uint32_t v : {kVersion, shape.d_model, shape.n_comp, shape.n_expert, shape.n_layers, shape.top_k,
                       shape.feat_dim, (uint32_t)present.size(), (uint32_t)groups.size(), 0u, 0u})
        word(v);
    for (uint32_t g : groups) {
        word(g);
        word((uint32_t)group_col[g]);
        word(shape.n_expert);
    }
    for (const LayerWeights &lw : present) put(&lw.layer, 4);
    for (const LayerWeights &lw : present) put(&lw.prior, 4);
    for (const LayerWeights &lw : present) put(lw.bias.data(), lw.bias.size() * 4);
    for (const LayerWeights &lw : present) put(lw.rows.data(), lw.rows.size() * 4);

    FILE *f = fopen(path.c_str(), "wb");
    if (!f) {
        err = "MOEP " + path + ": cannot open for writing";
        return false;
    }
    const bool wrote = fwrite(buf.data(), 1, buf.size(), f) == buf.size();
    if (fclose(f) != 0 || !wrote) {
        err = "MOEP " + path + ": short write";
        return false;
    }
    return true;
}

}  // namespace mpp
