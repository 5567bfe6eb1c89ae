// mp_cpu.h -- the routed-expert chain on the host CPU (internal interface).
//
// Used to serve experts that are absent from the HBM slots from the pinned
// store by the CPU instead of streaming their bytes over PCIe.  Arithmetic is
// the device kernels' and the CPU reference chain's: Q8_K activations, exact
// integer dots, fp32 per super-block in row order (scale term, then min term),
// SiLU with the canonical exp, Q8_K of h, then the down rows.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace mpc {

// One expert of a batch of host work: its bytes ([up][gate][down], host
// memory), the Q8_K of its input ([H/256][292]) and its output rows [H].
struct CpuExpert {
    const uint8_t *w;
    const uint8_t *q8x;
    float *y;
};

// A persistent team of worker threads.  Between `hot(true)` and `hot(false)`
// idle workers poll for work (microsecond hand-off); otherwise they sleep.
class Team;
Team *team_create(int n_threads);     // n_threads includes the caller
void team_destroy(Team *t);
int team_size(const Team *t);
void team_hot(Team *t, bool on);

// y_k = W_down,k . Q8_K(silu(W_gate,k . x) * (W_up,k . x)) for every expert,
// rows split over the team (the caller works too).  h_scratch holds n * I
// floats and q8h_scratch n * (I/256) * 292 bytes.
void experts(Team *t, const CpuExpert *e, int n, int H, int I, int down_type, float *h_scratch,
             uint8_t *q8h_scratch);

// The same chain for groups of tokens that share an expert: group g applies
// expert g.w to tokens first .. first + n - 1 (q8x[j], y[j]), reading each
// block of the expert's rows from memory once for all of them.  h_scratch
// holds (total tokens) * I floats and q8h_scratch (total tokens) * (I/256) *
// 292 bytes.  Results equal experts() token by token.
struct CpuGroup {
    const uint8_t *w;
    int first, n;
};
void experts_grouped(Team *t, const CpuGroup *g, int n_groups, const uint8_t *const *q8x, float *const *y, int H,
                     int I, int down_type, float *h_scratch, uint8_t *q8h_scratch);

// Map every page of [p, p + n) into this process's page tables for reading
// (memory another device filled has never been touched by the CPU: its first
// reads would fault page by page, ~1 ms per expert, in the middle of a decode)
void prefault(Team *t, const void *p, size_t n);

// The token's K routed experts from its logits (bias added), as the batch-1
// decode kernels select them: the softmax in their canonical order (the
// maximum; canonical exp; per 64-expert chunk a balanced pairwise sum in
// expert order, the chunks added in order; IEEE division), plus the cache
// prior (on the probabilities, or on the logits), then the K best by the
// selection value with the lower id first on a tie (a NaN as -inf, -0 as +0).
// ids in rank order.  E a multiple of 64, at most 256; K <= E.
void route_topk(const float *logits, int E, const float *prior, bool prior_on_logits, int K, int32_t *ids);

// building blocks (exposed for the tests of this file's arithmetic)
void quant_q8k(const float *x, int n, uint8_t *out);
float dot_q4k(const uint8_t *row, const uint8_t *q8, int nb);
float dot_q6k(const uint8_t *row, const uint8_t *q8, int nb);
// nrows rows (stride bytes apart) of type Q4_K or Q6_K against one Q8_K vector
void dot_rows(int type, const uint8_t *row0, size_t stride, int nrows, const uint8_t *q8, int nb, float *out);
// bring nrows rows of nb super-blocks into the cache (a hint: never faults)
void prefetch_rows(int type, const uint8_t *row0, size_t stride, int nrows, int nb);
bool has_vnni();
void set_portable(bool on);     // force the portable dots (tests)

}  // namespace mpc
