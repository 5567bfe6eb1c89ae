/*
 * stream.c -- router lookahead and the just-in-time copy planner, restated.
 * TEST INFRASTRUCTURE ONLY (nothing in the product links or calls this code).
 *
 * or_ahead follows k_moe_ahead_scores / k_moe_ahead_post
 * (patches/0010-team-and-streaming.patch:382-474): scores s[e] = W_T[e] . (x * r)
 * for a target layer T, the k best experts (best first, the lower id on a
 * tie), and of those the ones whose table entry is the dummy, in that order.
 * The dot product here is the canonical router order (oracle.h) applied to the
 * f32 products x[i] * r[i]; the reference's warp-strided sum is not pinned and
 * the GPU kernel follows this order instead.
 *
 * or_planner_* follows moe_planner (patches/0010-team-and-streaming.patch:777-909):
 * one job per (target layer, expert); earliest deadline first in chunks of at
 * most chunk_bytes; a job that can no longer land before its deadline is
 * dropped (DROP_LATE); the unfinished jobs of a layer that has read its table
 * are dropped (DROP_POSTED) and that layer takes no new job; a repeat offer
 * with an earlier deadline tightens the job; hold_after >= 0 holds back jobs
 * whose target is beyond that layer (not dropped for it).
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

float or_row_logit(int H, const float *w, const float *x);

int or_ahead(int E, int H, int k, const float *W, const float *x, const float *r,
             const int32_t *table, int32_t dummy, float *scores_out, int32_t *ids) {
    float xr[8192];
    float s[1024];
    if (H > 8192 || E > 1024 || k > E) return -1;
    for (int i = 0; i < H; ++i) xr[i] = x[i] * r[i];
    for (int e = 0; e < E; ++e) s[e] = or_row_logit(H, W + (size_t)e * H, xr);
    if (scores_out) memcpy(scores_out, s, (size_t)E * sizeof(float));
    for (int e = 0; e < E; ++e)
        if (s[e] != s[e]) s[e] = -INFINITY;            /* a NaN ranks with -inf */
    unsigned char taken[1024] = {0};
    int n = 0;
    for (int round = 0; round < k; ++round) {
        int best = -1;
        for (int e = 0; e < E; ++e) {
            if (taken[e]) continue;
            if (best < 0 || s[e] > s[best]) best = e;   /* strict: the lower id keeps a tie */
        }
        taken[best] = 1;
        if (table[best] == dummy) ids[n++] = best;
    }
    return n;
}

/* ---- planner ----------------------------------------------------------- */
typedef struct {
    int target;
    int32_t expert;
    size_t bytes, sent;
    uint64_t deadline_ns;
    int dropped, drop;
} or_pjob;

struct or_planner {
    size_t chunk_bytes;
    or_pjob *jobs;
    int n, cap;
    int *posted;
    int n_posted, cap_posted;
    uint64_t n_offered, n_dup, n_drop_late, n_drop_posted;
};

or_planner *or_planner_create(size_t chunk_bytes) {
    or_planner *p = (or_planner *)calloc(1, sizeof(or_planner));
    p->chunk_bytes = chunk_bytes;
    return p;
}

void or_planner_destroy(or_planner *p) {
    if (!p) return;
    free(p->jobs);
    free(p->posted);
    free(p);
}

void or_planner_reset(or_planner *p) {
    p->n = 0;
    p->n_posted = 0;
}

int or_planner_offer(or_planner *p, int target, int32_t expert, size_t bytes, uint64_t deadline_ns) {
    for (int i = 0; i < p->n_posted; ++i)
        if (p->posted[i] == target) return -1;
    for (int i = 0; i < p->n; ++i) {
        or_pjob *j = &p->jobs[i];
        if (j->target == target && j->expert == expert) {
            if (!j->dropped && deadline_ns < j->deadline_ns) j->deadline_ns = deadline_ns;
            p->n_dup++;
            return -1;
        }
    }
    if (p->n == p->cap) {
        p->cap = p->cap ? 2 * p->cap : 16;
        p->jobs = (or_pjob *)realloc(p->jobs, (size_t)p->cap * sizeof(or_pjob));
    }
    or_pjob *j = &p->jobs[p->n];
    j->target = target;
    j->expert = expert;
    j->bytes = bytes;
    j->sent = 0;
    j->deadline_ns = deadline_ns;
    j->dropped = 0;
    j->drop = OR_DROP_NONE;
    p->n_offered++;
    return p->n++;
}

void or_planner_posted(or_planner *p, int target) {
    if (p->n_posted == p->cap_posted) {
        p->cap_posted = p->cap_posted ? 2 * p->cap_posted : 16;
        p->posted = (int *)realloc(p->posted, (size_t)p->cap_posted * sizeof(int));
    }
    p->posted[p->n_posted++] = target;
    for (int i = 0; i < p->n; ++i) {
        or_pjob *j = &p->jobs[i];
        if (j->target == target && !j->dropped && j->sent < j->bytes) {
            j->dropped = 1;
            j->drop = OR_DROP_POSTED;
            p->n_drop_posted++;
        }
    }
}

int or_planner_next(or_planner *p, uint64_t free_at_ns, double bytes_per_ns, int hold_after, or_chunk *out) {
    int best = -1;
    for (int i = 0; i < p->n; ++i) {
        or_pjob *j = &p->jobs[i];
        if (j->dropped || j->sent >= j->bytes) continue;
        const uint64_t finish = free_at_ns + (uint64_t)((double)(j->bytes - j->sent) / bytes_per_ns);
        if (finish > j->deadline_ns) {
            j->dropped = 1;
            j->drop = OR_DROP_LATE;
            p->n_drop_late++;
            continue;
        }
        if (hold_after >= 0 && j->target > hold_after) continue;
        if (best < 0 || j->deadline_ns < p->jobs[best].deadline_ns) best = i;
    }
    if (best < 0) return 0;
    or_pjob *j = &p->jobs[best];
    const size_t remaining = j->bytes - j->sent;
    out->job = best;
    out->offset = j->sent;
    out->len = remaining < p->chunk_bytes ? remaining : p->chunk_bytes;
    out->last = out->len == remaining;
    j->sent += out->len;
    return 1;
}

int or_planner_size(const or_planner *p) { return p->n; }

void or_planner_get(const or_planner *p, int id, or_planner_job *out) {
    const or_pjob *j = &p->jobs[id];
    out->target = j->target;
    out->expert = j->expert;
    out->bytes = j->bytes;
    out->sent = j->sent;
    out->deadline_ns = j->deadline_ns;
    out->dropped = j->dropped;
    out->drop = j->drop;
}

void or_planner_counters(const or_planner *p, uint64_t out[4]) {
    out[0] = p->n_offered;
    out[1] = p->n_dup;
    out[2] = p->n_drop_late;
    out[3] = p->n_drop_posted;
}
