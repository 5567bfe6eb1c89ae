// ref_predictor_shim.cpp -- a C entry point onto the reference's own MOEP
// predictor (cpp/moe-predictor.cpp, compiled from where it lies by the Makefile
// in this directory into _ref/, only where the reference tree is present).
// TEST INFRASTRUCTURE ONLY: what the tests compare moe_predictor_* in the product with.
#include "moe-predictor.h"

#include <cstdint>
#include <cstring>
#include <string>

namespace {
void copy_err(const std::string &e, char *buf, int n) {
    if (buf && n > 0) {
        strncpy(buf, e.c_str(), (size_t)n - 1);
        buf[n - 1] = 0;
    }
}
moe_predictor::inputs lists(const int32_t *p, int np, const int32_t *c, int nc, const int32_t *b, int nb,
                            const int32_t *s, int ns) {
    moe_predictor::inputs in;
    in.prev = p; in.n_prev = (size_t)np;
    in.cur = c; in.n_cur = (size_t)nc;
    in.below = b; in.n_below = (size_t)nb;
    in.self_prev = s; in.n_self_prev = (size_t)ns;
    return in;
}
}  // namespace

extern "C" {
void *rp_load(const char *path, char *err, int errlen) {
    auto *p = new moe_predictor();
    std::string e;
    if (!p->load(path, e)) {
        copy_err(e, err, errlen);
        delete p;
        return nullptr;
    }
    return p;
}
void rp_free(void *h) { delete (moe_predictor *)h; }
int rp_has_layer(void *h, int il) { return ((moe_predictor *)h)->has_layer(il) ? 1 : 0; }
void rp_score(void *h, int il, const int32_t *p, int np, const int32_t *c, int nc, const int32_t *b, int nb,
              const int32_t *s, int ns, float *out) {
    ((moe_predictor *)h)->score(il, lists(p, np, c, nc, b, nb, s, ns), out);
}
int rp_top_k(void *h, const float *scores, int k, int32_t *out) {
    return (int)((moe_predictor *)h)->top_k_ids(scores, (size_t)k, out);
}
float rp_update(void *h, int il, const int32_t *p, int np, const int32_t *c, int nc, const int32_t *b, int nb,
                const int32_t *s, int ns, const int32_t *truth, int nt, float lr) {
    return ((moe_predictor *)h)->update(il, lists(p, np, c, nc, b, nb, s, ns), truth, (size_t)nt, lr);
}
int rp_save(void *h, const char *path, char *err, int errlen) {
    std::string e;
    if (!((moe_predictor *)h)->save(path, e)) {
        copy_err(e, err, errlen);
        return -1;
    }
    return 0;
}
}
