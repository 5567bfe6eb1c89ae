/*
 * cache.c -- the per-layer expert-id -> slot state machine, restated.
 * TEST INFRASTRUCTURE ONLY (see oracle.h).
 *
 * Follows llama-moecache.cpp as patched by 0006, 0007 and 0008 (file:line are
 * inside those .patch files):
 *   observe   0006:295-400, 0007:247-321 (heat, miss window), 0008:504-518 (route trace)
 *   issue     0006:241-293, 0007:230-246 (early path)
 *   step      0006:765-953, 0007:655-771, 0008:607-660 (deterministic publication)
 *   admission 0007:398-429 (lru_resident, admit_ok)
 *   tables    0007:327-396 (set_table_entry, flush_tables)
 *   map trace 0008:417-489 (record and replay)
 *   heat file 0007:431-485 (load/save), 0007:568-621 (warm start), 0007:745-752
 *   freeze    0008:496-500, 825-832
 *   streaming 0010:1096-1129 (map frame one step late), 0010:1183-1210 (account),
 *             0010:1466-1530 (take), 0010:1722-1760 (adopt), 0010:1138-1175 (pool target,
 *             issue skip, observe skip)
 *   predictor 0006:295-400 (online resolution, next-layer prediction), 0007:330-355
 *             (admission guard on speculative uploads, spec jobs), 0006:501-560 (knobs)
 *   evictor   0006:404-427 (scores), 0006:790-900 and 0007:676-724 (victims), 0006:918-922
 *   probation 0007:149-153, 0007:655-668 (speculative jobs published oldest and protected)
 * The hooks are pinned only where they reduce to the recorded traces (a flat
 * evictor is LRU); beyond that they are parity unpinned: no reference trace
 * ran with a predictor.
 *
 * Upload completion: every job is published at the step after the one that
 * scheduled (or, early path, issued) it.  With `deterministic` the order is
 * (layer, slot), as LLAMA_MOE_DETERMINISTIC=1 sorts the done list
 * (0008:613-627); without it the order is scheduling order, which is the order
 * the single upload worker of a live run finishes them in (0006:654-723).  A
 * live run differs from this only when a copy is still running at the next
 * boundary; or_cache_hold_job() models that by holding one job back a step.
 */
#include "oracle.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define U64MAX 0xffffffffffffffffull

typedef struct {
    int il, S, E;
    int32_t *slot_expert, *expert_slot;
    uint64_t *slot_last_use, *slot_protect;
    uint8_t *slot_in_flight;
    int32_t *free_slots;
    int n_free;
    int32_t *pending;
    int n_pending;
    float *heat;
    uint32_t *use_count;            /* heat-file counts, or NULL */
    uint64_t *miss_last, *miss_prev;
    int32_t *tbl_mirror;
    float *prior_mirror;
    int tbl_dirty;
    uint64_t n_hit, n_miss;
    /* predictor / evictor: this token's ids, the previous token's, and the
     * features of the last prediction made for this layer */
    int32_t *cur_ids, *prev_ids, *pend_prev, *pend_cur;
    int n_cur, n_prev_ids, n_pend_prev, n_pend_cur, cap_ids;
    int pend_valid;
} layer_t;

typedef struct {
    int li, expert, slot;
    uint64_t sched_step;
    int hold, spec;
} job_t;

typedef struct {
    int li, slot, d;
    int landed, in_time, late;
} sjob_t;

enum { ST_RECORDS, ST_OFFERED, ST_LANDED, ST_IN_TIME, ST_LATE, ST_UNUSED, ST_DROP_LATE, ST_DROP_POSTED,
       ST_NOT_SENT, ST_GPU_MISS, ST_BYTES };

struct or_cache {
    int n_layers, E;
    or_knobs k;
    layer_t *L;
    uint64_t clock, n_steps, n_uploads, n_scheduled, n_published;
    uint64_t n_admit_ok, n_admit_denied, n_table_flushes;
    job_t *jobs;
    int n_jobs, cap_jobs;
    job_t *holds;
    int n_holds;
    FILE *route, *map, *replay;
    char *heat_path;
    int freeze, replay_err;
    /* just-in-time streaming (0010): jobs of this token, one per planner job */
    int st_on, st_per_layer, st_reserve;
    double st_bytes_per_ns, st_tau_ns;
    uint64_t st_margin_ns;
    or_planner *st_planner;
    sjob_t *sjobs;
    int n_sjobs, cap_sjobs;
    int32_t *st_mark;               /* [layer][E]: job + 1 while streamed this token */
    int *st_n_this_token;
    uint32_t st_last_layer;
    uint64_t st_last_t_ns;
    uint64_t st_n[11];              /* records, offered, landed, in time, late, unused, dropped late,
                                       dropped posted, not sent, GPU misses, bytes */
    int32_t *rec_frame;             /* [layer][S] frame held back one step (map record) */
    uint64_t rec_step;
    int rec_have;
    int32_t *rec_used;              /* (layer, slot, expert) triples used in time this step */
    int n_rec_used;
    /* MOEP predictor (borrowed; updated in place when online_lr > 0) and evictor */
    or_moep *pred, *evict;
    int predict_top, spec_probation;
    float online_lr;
    uint64_t online_n, n_spec;
    double online_recall;
};

/* room for n ids in each of a layer's id lists */
static void ids_room(layer_t *ls, int n) {
    if (n <= ls->cap_ids) return;
    ls->cap_ids = n;
    ls->cur_ids = (int32_t *)realloc(ls->cur_ids, sizeof(int32_t) * (size_t)n);
    ls->prev_ids = (int32_t *)realloc(ls->prev_ids, sizeof(int32_t) * (size_t)n);
    ls->pend_prev = (int32_t *)realloc(ls->pend_prev, sizeof(int32_t) * (size_t)n);
    ls->pend_cur = (int32_t *)realloc(ls->pend_cur, sizeof(int32_t) * (size_t)n);
}

static void push_job(or_cache *c, int li, int e, int slot, int spec) {
    if (c->n_jobs == c->cap_jobs) {
        c->cap_jobs = c->cap_jobs ? 2 * c->cap_jobs : 256;
        c->jobs = (job_t *)realloc(c->jobs, sizeof(job_t) * (size_t)c->cap_jobs);
    }
    job_t j = {li, e, slot, c->n_steps, 0, spec};
    for (int h = 0; h < c->n_holds; ++h) {
        const job_t *q = &c->holds[h];
        if (q->li == li && q->expert == e && q->slot == slot && q->sched_step == c->n_steps) j.hold = 1;
    }
    c->jobs[c->n_jobs++] = j;
}

static void set_table_entry(or_cache *c, layer_t *ls, int expert, int v) {
    ls->tbl_mirror[expert] = v;
    if (ls->prior_mirror) ls->prior_mirror[expert] = v == ls->S ? 0.0f : c->k.cache_prior;
    ls->tbl_dirty = 1;
}

static int32_t lru_resident(const layer_t *ls) {
    int32_t victim = -1;
    uint64_t best = U64MAX;
    for (int s = 0; s < ls->S; ++s) {
        if (ls->slot_in_flight[s] || ls->slot_expert[s] < 0) continue;
        if (ls->slot_last_use[s] < best) {
            best = ls->slot_last_use[s];
            victim = ls->slot_expert[s];
        }
    }
    return victim;
}

static int admit_ok(or_cache *c, const layer_t *ls, int id, int victim) {
    if (c->k.admit_mode == 0 || victim < 0) return 1;
    int ok = 1;
    if (c->k.admit_mode == 1) {
        ok = ls->heat[id] > ls->heat[victim] * 1.25f + c->k.admit_floor;
    } else if (c->k.admit_mode == 2) {
        ok = ls->miss_prev[id] != U64MAX &&
             ls->miss_last[id] - ls->miss_prev[id] < (uint64_t)c->k.admit_window;
    }
    if (ok) c->n_admit_ok++; else c->n_admit_denied++;
    return ok;
}

or_cache *or_cache_create(int n_layers, int n_experts, const int32_t *slots, const or_knobs *k) {
    or_cache *c = (or_cache *)calloc(1, sizeof(or_cache));
    c->n_layers = n_layers;
    c->E = n_experts;
    c->k = *k;
    if (c->k.max_inserts <= 0) c->k.max_inserts = 2;
    if (c->k.admit_window <= 0) c->k.admit_window = 8;
    if (c->k.admit_half <= 0) c->k.admit_half = 64;
    c->L = (layer_t *)calloc((size_t)n_layers, sizeof(layer_t));
    for (int l = 0; l < n_layers; ++l) {
        layer_t *ls = &c->L[l];
        const int S = slots[l], E = n_experts;
        ls->il = l;
        ls->S = S;
        ls->E = E;
        ls->slot_expert = (int32_t *)malloc(sizeof(int32_t) * (size_t)S);
        ls->expert_slot = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
        ls->slot_last_use = (uint64_t *)calloc((size_t)S, sizeof(uint64_t));
        ls->slot_protect = (uint64_t *)calloc((size_t)S, sizeof(uint64_t));
        ls->slot_in_flight = (uint8_t *)calloc((size_t)S, 1);
        ls->free_slots = (int32_t *)malloc(sizeof(int32_t) * (size_t)S);
        ls->pending = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
        ls->tbl_mirror = (int32_t *)malloc(sizeof(int32_t) * (size_t)E);
        for (int s = 0; s < S; ++s) ls->slot_expert[s] = -1;
        for (int e = 0; e < E; ++e) { ls->expert_slot[e] = -1; ls->tbl_mirror[e] = S; }
        for (int s = 0; s < S; ++s) ls->free_slots[s] = S - 1 - s;   /* lowest slot on top */
        ls->n_free = S;
        if (c->k.cache_prior > 0.0f) ls->prior_mirror = (float *)calloc((size_t)E, sizeof(float));
        if (c->k.admit_mode == 1) ls->heat = (float *)calloc((size_t)E, sizeof(float));
        if (c->k.admit_mode == 2) {
            ls->miss_last = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)E);
            ls->miss_prev = (uint64_t *)malloc(sizeof(uint64_t) * (size_t)E);
            for (int e = 0; e < E; ++e) ls->miss_last[e] = ls->miss_prev[e] = U64MAX;
        }
    }
    return c;
}

static int layer_off(const or_cache *c, int li) {
    int o = 0;
    for (int l = 0; l < li; ++l) o += c->L[l].S;
    return o;
}

static void write_frame(or_cache *c, uint64_t step, const int32_t *frame) {
    fprintf(c->map, "step %llu\n", (unsigned long long)step);
    for (int l = 0; l < c->n_layers; ++l) {
        const layer_t *ls = &c->L[l];
        const int32_t *f = frame + layer_off(c, l);
        fprintf(c->map, "map %d", ls->il);
        for (int s = 0; s < ls->S; ++s) fprintf(c->map, " %d", f[s]);
        fputc('\n', c->map);
    }
    fflush(c->map);
}

void or_cache_destroy(or_cache *c) {
    if (!c) return;
    for (int l = 0; l < c->n_layers; ++l) {
        layer_t *ls = &c->L[l];
        free(ls->slot_expert); free(ls->expert_slot); free(ls->slot_last_use);
        free(ls->slot_protect); free(ls->slot_in_flight); free(ls->free_slots);
        free(ls->pending); free(ls->tbl_mirror); free(ls->prior_mirror);
        free(ls->heat); free(ls->miss_last); free(ls->miss_prev); free(ls->use_count);
        free(ls->cur_ids); free(ls->prev_ids); free(ls->pend_prev); free(ls->pend_cur);
    }
    if (c->map && c->rec_have) write_frame(c, c->rec_step, c->rec_frame);   /* the last boundary */
    if (c->route) fclose(c->route);
    if (c->map) fclose(c->map);
    if (c->replay) fclose(c->replay);
    free(c->heat_path);
    or_planner_destroy(c->st_planner);
    free(c->sjobs); free(c->st_mark); free(c->st_n_this_token); free(c->rec_frame); free(c->rec_used);
    free(c->L);
    free(c->jobs);
    free(c->holds);
    free(c);
}

static void flush_tables(or_cache *c);
static int save_heat(or_cache *c);

/* 0008:436-474: read this step's frame and make it the placement */
static void replay_frame(or_cache *c) {
    unsigned long long step = 0;
    if (fscanf(c->replay, " step %llu", &step) != 1 || step != c->n_steps) { c->replay_err = 1; return; }
    int32_t *want = (int32_t *)malloc(sizeof(int32_t) * 4096);
    uint8_t *seen = (uint8_t *)malloc((size_t)c->E);
    for (int l = 0; l < c->n_layers && !c->replay_err; ++l) {
        layer_t *ls = &c->L[l];
        int il = -1;
        if (fscanf(c->replay, " map %d", &il) != 1 || il != ls->il) { c->replay_err = 1; break; }
        memset(seen, 0, (size_t)c->E);
        for (int s = 0; s < ls->S; ++s) {
            if (fscanf(c->replay, "%d", &want[s]) != 1 || want[s] < -1 || want[s] >= ls->E ||
                (want[s] >= 0 && seen[want[s]])) { c->replay_err = 1; break; }
            if (want[s] >= 0) seen[want[s]] = 1;
        }
        if (c->replay_err) break;
        for (int e = 0; e < ls->E; ++e) { ls->expert_slot[e] = -1; set_table_entry(c, ls, e, ls->S); }
        for (int s = 0; s < ls->S; ++s) {
            ls->slot_expert[s] = want[s];
            ls->slot_in_flight[s] = 0;
            if (want[s] >= 0) { ls->expert_slot[want[s]] = s; set_table_entry(c, ls, want[s], s); }
        }
    }
    free(want);
    free(seen);
    if (!c->replay_err) flush_tables(c);
}

static void map_frame(or_cache *c) {
    if (c->replay && !c->replay_err) replay_frame(c);
    if (!c->map) return;
    const int total = layer_off(c, c->n_layers);
    int32_t *frame = (int32_t *)malloc(sizeof(int32_t) * (size_t)(total + 1));
    for (int l = 0; l < c->n_layers; ++l) or_cache_frame(c, l, frame + layer_off(c, l));
    if (!c->st_on) {
        write_frame(c, c->n_steps, frame);
        free(frame);
        return;
    }
    /* 0010:1096-1129: the token after a boundary also used the experts that
     * streamed in before their layer read its table; the boundary's frame is
     * written one step late with those experts in the slots they used */
    if (c->rec_have) {
        for (int u = 0; u < c->n_rec_used; ++u) {
            const int li = c->rec_used[3 * u], slot = c->rec_used[3 * u + 1], e = c->rec_used[3 * u + 2];
            c->rec_frame[layer_off(c, li) + slot] = e;
        }
        write_frame(c, c->rec_step, c->rec_frame);
    }
    c->n_rec_used = 0;
    free(c->rec_frame);
    c->rec_frame = frame;
    c->rec_step = c->n_steps;
    c->rec_have = 1;
}

int or_cache_trace_open(or_cache *c, const char *route_path, const char *map_path) {
    if (route_path) {
        c->route = fopen(route_path, "w");
        if (!c->route) return -1;
    }
    if (map_path) {
        c->map = fopen(map_path, "w");
        if (!c->map) return -1;
        fprintf(c->map, "moe-map 1 %d\n", c->n_layers);
        for (int l = 0; l < c->n_layers; ++l)
            fprintf(c->map, "layer %d %d %d\n", c->L[l].il, c->L[l].S, c->L[l].E);
        map_frame(c);
    }
    return 0;
}

/* 0006:241-293: early issue out of pre-freed slots; caller-side admission;
 * spec: issued from a prediction (0007:232-242) */
static int issue_uploads(or_cache *c, int li, const int32_t *ids, int n, int budget, int min_keep, int spec) {
    layer_t *ls = &c->L[li];
    int issued = 0;
    if (c->freeze) return 0;
    for (int i = 0; i < n && issued < budget; ++i) {
        const int id = ids[i];
        if (id < 0 || id >= ls->E) continue;
        if (ls->expert_slot[id] >= 0) continue;
        if (c->st_on && c->st_mark[li * c->E + id]) continue;      /* being streamed this token */
        if (ls->n_free <= min_keep) break;
        int dup = 0;
        for (int j = 0; j < c->n_jobs; ++j)
            if (c->jobs[j].li == li && c->jobs[j].expert == id) { dup = 1; break; }
        if (dup) continue;
        const int slot = ls->free_slots[--ls->n_free];
        ls->slot_in_flight[slot] = 1;
        push_job(c, li, id, slot, spec);
        c->n_uploads++;
        c->n_scheduled++;
        c->n_spec += spec != 0;
        issued++;
    }
    return issued;
}

static int pool_target_of(const or_cache *c) {
    if (c->freeze) return 0;
    return c->k.max_inserts + (c->pred ? c->predict_top : 0) + (c->st_on ? c->st_reserve : 0);
}

/* gslots (batch 1 with streaming): the slots the GPU used, n_slots = absent */
static void observe_body(or_cache *c, int li, const int32_t *ids, int n_ids, int n_tok, const int32_t *gslots) {
    layer_t *ls = &c->L[li];
    if (c->route) {
        fprintf(c->route, "route %llu %d %d %d", (unsigned long long)c->n_steps, ls->il, n_ids, n_tok);
        for (int i = 0; i < n_ids * n_tok; ++i) {
            int slot = (ids[i] >= 0 && ids[i] < ls->E) ? ls->expert_slot[ids[i]] : -1;
            if (gslots) slot = gslots[i] >= ls->S ? -1 : gslots[i];   /* 0010:1147-1154 */
            fprintf(c->route, " %d:%d", ids[i], slot);
        }
        fputc('\n', c->route);
    }
    ids_room(ls, n_ids * n_tok);
    int32_t *observed = (int32_t *)malloc(sizeof(int32_t) * (size_t)(n_ids * n_tok + 1));
    int n_obs = 0;
    for (int t = 0; t < n_tok; ++t) {
        for (int i = 0; i < n_ids; ++i) {
            const int id = ids[t * n_ids + i];
            if (id < 0 || id >= ls->E) continue;
            observed[n_obs++] = id;
            if (ls->heat) ls->heat[id] += 1.0f;
            if (ls->use_count) ls->use_count[id]++;
            const int slot = ls->expert_slot[id];
            if (slot < 0 && c->st_on && c->st_mark[li * c->E + id]) continue;  /* the GPU's table decides */
            if (slot >= 0) {
                ls->n_hit++;
                ls->slot_last_use[slot] = ++c->clock;
            } else {
                ls->n_miss++;
                if (ls->miss_last && ls->miss_last[id] != c->n_steps) {
                    ls->miss_prev[id] = ls->miss_last[id];
                    ls->miss_last[id] = c->n_steps;
                }
                int dup = 0;
                for (int p = 0; p < ls->n_pending; ++p) if (ls->pending[p] == id) { dup = 1; break; }
                if (!dup) ls->pending[ls->n_pending++] = id;
            }
        }
    }
    /* 0006:323-363: the prediction made for this layer resolves against what it routed */
    if (c->pred && c->online_lr > 0.0f && ls->pend_valid && or_moep_has_layer(c->pred, ls->il)) {
        or_moep_lists in = {{ls->pend_prev, ls->pend_cur, NULL, NULL}, {ls->n_pend_prev, ls->n_pend_cur, 0, 0}};
        const float hit = or_moep_update(c->pred, ls->il, &in, observed, n_obs, c->online_lr);
        ls->pend_valid = 0;
        c->online_recall += hit;
        c->online_n++;
    }
    if (c->k.early_issue) {
        const int pool_target = pool_target_of(c);
        const int next_victim = c->k.admit_mode == 0 ? -1 :
            (ls->n_free > pool_target ? -1 : lru_resident(ls));
        if (c->k.admit_mode == 0) {
            issue_uploads(c, li, ls->pending, ls->n_pending, c->k.max_inserts, 0, 0);
        } else {
            int32_t adm[1024];
            int n = 0;
            for (int p = 0; p < ls->n_pending; ++p) {
                const int id = ls->pending[p];
                if (ls->expert_slot[id] < 0 && admit_ok(c, ls, id, next_victim)) adm[n++] = id;
            }
            issue_uploads(c, li, adm, n, c->k.max_inserts, 0, 0);
        }
        /* 0006:367-396, 0007:424-452: the next layer's experts, predicted from
         * its previous ids and this layer's, copied into its spare slots */
        if (c->pred && or_moep_has_layer(c->pred, ls->il) && li + 1 < c->n_layers) {
            layer_t *nls = &c->L[li + 1];
            const int E = or_moep_n_expert(c->pred);
            float *sc = (float *)malloc(sizeof(float) * (size_t)E);
            int32_t *top = (int32_t *)malloc(sizeof(int32_t) * (size_t)(c->predict_top + 1));
            or_moep_lists in = {{nls->cur_ids, observed, NULL, NULL}, {nls->n_cur, n_obs, 0, 0}};
            or_moep_score(c->pred, ls->il, &in, sc);
            const int n_top = or_moep_top(c->pred, sc, c->predict_top, top);
            if (c->online_lr > 0.0f) {
                ids_room(nls, n_obs > nls->n_cur ? n_obs : nls->n_cur);
                memcpy(nls->pend_prev, nls->cur_ids, sizeof(int32_t) * (size_t)nls->n_cur);
                nls->n_pend_prev = nls->n_cur;
                memcpy(nls->pend_cur, observed, sizeof(int32_t) * (size_t)n_obs);
                nls->n_pend_cur = n_obs;
                nls->pend_valid = 1;
            }
            int n_issue = n_top;
            if (c->k.admit_mode == 1) {
                /* a guess may only displace something colder than itself */
                const int nv = nls->n_free > pool_target ? -1 : lru_resident(nls);
                n_issue = 0;
                for (int k = 0; k < n_top; ++k) {
                    const int id = top[k];
                    if (id >= 0 && id < nls->E && nls->expert_slot[id] < 0 && admit_ok(c, nls, id, nv))
                        top[n_issue++] = id;
                }
            }
            issue_uploads(c, li + 1, top, n_issue, c->predict_top, c->k.max_inserts, 1);
            free(sc);
            free(top);
        }
    }
    memcpy(ls->cur_ids, observed, sizeof(int32_t) * (size_t)n_obs);
    ls->n_cur = n_obs;
    free(observed);
}

/* 0006:404-427: the evictor's scores of a layer's experts, once per step
 * (0 when there is no model for the layer) */
static int evict_scores(const or_cache *c, int li, float *out) {
    const layer_t *ls = &c->L[li];
    if (!c->evict || !or_moep_has_layer(c->evict, ls->il)) return 0;
    or_moep_lists in = {{NULL, ls->cur_ids, NULL, ls->prev_ids}, {0, ls->n_cur, 0, ls->n_prev_ids}};
    if (li + 1 < c->n_layers) {
        in.ids[0] = c->L[li + 1].prev_ids;
        in.n[0] = c->L[li + 1].n_prev_ids;
    }
    if (li > 0) {
        in.ids[2] = c->L[li - 1].cur_ids;
        in.n[2] = c->L[li - 1].n_cur;
    }
    or_moep_score(c->evict, ls->il, &in, out);
    return 1;
}

void or_cache_set_predictor(or_cache *c, or_moep *m, int predict_top, float online_lr) {
    c->pred = m && predict_top > 0 ? m : NULL;
    c->predict_top = predict_top;
    c->online_lr = online_lr;
    if (c->pred) c->k.early_issue = 1;      /* 0006:558-562: a predictor needs early issue */
}

void or_cache_set_evictor(or_cache *c, or_moep *m) { c->evict = m; }

void or_cache_set_spec_probation(or_cache *c, int on) { c->spec_probation = on != 0; }

void or_cache_predictor_stats(const or_cache *c, uint64_t *n_updates, double *recall_sum, uint64_t *n_spec) {
    if (n_updates) *n_updates = c->online_n;
    if (recall_sum) *recall_sum = c->online_recall;
    if (n_spec) *n_spec = c->n_spec;
}

void or_cache_observe(or_cache *c, int li, const int32_t *ids, int n_ids, int n_tok) {
    observe_body(c, li, ids, n_ids, n_tok, NULL);
}

/* 0010:1183-1210: the GPU's slots say whether each streamed expert made it */
static void stream_account(or_cache *c, int li, const int32_t *ids, const int32_t *gslots, int n_ids) {
    for (int i = 0; i < n_ids; ++i) {
        const int id = ids[i];
        layer_t *ls0 = &c->L[li];
        if (id < 0 || id >= ls0->E) continue;
        const int miss = gslots[i] >= ls0->S;
        const int m = c->st_mark[li * c->E + id];
        if (!m) { c->st_n[ST_GPU_MISS] += miss; continue; }
        sjob_t *j = &c->sjobs[m - 1];
        layer_t *ls = &c->L[j->li];
        if (!miss && !j->in_time) {
            j->in_time = 1;
            c->st_n[ST_IN_TIME]++;
            ls->n_hit++;
        } else if (miss && !j->in_time && !j->late) {
            j->late = 1;
            c->st_n[ST_LATE]++;
            c->st_n[ST_GPU_MISS]++;
            ls->n_miss++;
        }
    }
}

void or_cache_observe_gpu(or_cache *c, int li, const int32_t *ids, const int32_t *gslots, int n_ids) {
    observe_body(c, li, ids, n_ids, 1, c->st_on ? gslots : NULL);
    if (c->st_on) stream_account(c, li, ids, gslots, n_ids);
}

int or_cache_stream_enable(or_cache *c, int per_layer, int reserve, double gbps, size_t chunk_bytes) {
    if (!c->k.early_issue || !c->k.batch_tables || c->k.deterministic || c->replay || c->freeze || c->map)
        return -1;
    if (c->st_on) return 0;
    c->st_on = 1;
    c->st_per_layer = per_layer < 1 ? 1 : per_layer;
    c->st_reserve = reserve < 0 ? 0 : reserve;
    c->st_bytes_per_ns = gbps < 1.0 ? 1.0 : gbps;
    c->st_tau_ns = 103000.0;
    c->st_margin_ns = 5000;
    c->st_planner = or_planner_create(chunk_bytes ? chunk_bytes : 512 * 1024);
    c->st_mark = (int32_t *)calloc((size_t)c->n_layers * (size_t)c->E, sizeof(int32_t));
    c->st_n_this_token = (int *)calloc((size_t)c->n_layers, sizeof(int));
    c->st_last_layer = 0xffffffffu;
    return 0;
}

/* 0010:1466-1530: one lookahead record (source layer `layer`, GPU time t_ns)
 * becomes planner jobs, each with a free slot */
int or_cache_stream_take(or_cache *c, int layer, const int32_t *targets, const int32_t *n, const int32_t *ids,
                         uint64_t now_ns, uint64_t t_ns, size_t expert_bytes) {
    if (!c->st_on) return -1;
    if (c->st_last_layer != 0xffffffffu && (uint32_t)layer == c->st_last_layer + 1 && t_ns > c->st_last_t_ns) {
        const double dt = (double)(t_ns - c->st_last_t_ns);
        if (dt > 10000.0 && dt < 1000000.0) c->st_tau_ns = 0.9 * c->st_tau_ns + 0.1 * dt;
    }
    c->st_last_layer = (uint32_t)layer;
    c->st_last_t_ns = t_ns;
    c->st_n[ST_RECORDS]++;
    int taken = 0;
    for (int t = 0; t < 2; ++t) {
        const int T = targets[t];
        if (T < 0 || T >= c->n_layers) continue;
        layer_t *ls = &c->L[T];
        const int d = T - layer;
        const uint64_t lead = (uint64_t)(d * c->st_tau_ns);
        const uint64_t deadline = now_ns + (lead > c->st_margin_ns ? lead - c->st_margin_ns : 0);
        for (int j = 0; j < n[t] && j < 8; ++j) {
            const int e = ids[8 * t + j];
            if (e < 0 || e >= ls->E || ls->expert_slot[e] >= 0) continue;
            if (c->st_mark[T * c->E + e]) {
                or_planner_offer(c->st_planner, T, e, expert_bytes, deadline);     /* may tighten */
                continue;
            }
            if (c->st_n_this_token[T] >= c->st_per_layer) continue;
            if (ls->n_free <= c->k.max_inserts) { c->st_n[ST_NOT_SENT]++; continue; }
            int dup = 0;
            for (int q = 0; q < c->n_jobs; ++q)
                if (c->jobs[q].li == T && c->jobs[q].expert == e) { dup = 1; break; }
            if (dup) continue;
            const int id = or_planner_offer(c->st_planner, T, e, expert_bytes, deadline);
            if (id < 0) continue;
            if (c->n_sjobs == c->cap_sjobs) {
                c->cap_sjobs = c->cap_sjobs ? 2 * c->cap_sjobs : 64;
                c->sjobs = (sjob_t *)realloc(c->sjobs, sizeof(sjob_t) * (size_t)c->cap_sjobs);
            }
            sjob_t sj = {T, ls->free_slots[--ls->n_free], d, 0, 0, 0};
            ls->slot_in_flight[sj.slot] = 1;
            c->sjobs[c->n_sjobs++] = sj;
            c->st_mark[T * c->E + e] = id + 1;
            c->st_n_this_token[T]++;
            c->st_n[ST_OFFERED]++;
            taken++;
        }
    }
    return taken;
}

void or_cache_stream_posted(or_cache *c, int layer) {
    if (c->st_on) or_planner_posted(c->st_planner, layer);
}

int or_cache_stream_next(or_cache *c, uint64_t free_at_ns, int hold_after, or_chunk *out) {
    if (!c->st_on) return 0;
    const int r = or_planner_next(c->st_planner, free_at_ns, c->st_bytes_per_ns, hold_after, out);
    if (r) c->st_n[ST_BYTES] += out->len;
    return r;
}

void or_cache_stream_land(or_cache *c, int job) {
    if (!c->st_on || job < 0 || job >= c->n_sjobs || c->sjobs[job].landed) return;
    c->sjobs[job].landed = 1;
    c->st_n[ST_LANDED]++;
}

/* slot and target layer of a job (-1 when there is none) */
int or_cache_stream_job(const or_cache *c, int job, int32_t *layer, int32_t *expert) {
    if (!c->st_on || job < 0 || job >= c->n_sjobs) return -1;
    or_planner_job pj;
    or_planner_get(c->st_planner, job, &pj);
    if (layer) *layer = c->sjobs[job].li;
    if (expert) *expert = pj.expert;
    return c->sjobs[job].slot;
}

void or_cache_stream_stats(const or_cache *c, uint64_t out[11]) {
    for (int i = 0; i < 11; ++i) out[i] = c->st_n[i];
}

/* 0010:1722-1760 (mover idle): landed experts join the cache, the slots of the
 * others go back to the pool */
static void stream_adopt(or_cache *c) {
    c->n_rec_used = 0;
    if (c->n_sjobs) c->rec_used = (int32_t *)realloc(c->rec_used, sizeof(int32_t) * 3 * (size_t)c->n_sjobs);
    for (int k = 0; k < c->n_sjobs; ++k) {
        const sjob_t *sj = &c->sjobs[k];
        or_planner_job pj;
        or_planner_get(c->st_planner, k, &pj);
        layer_t *ls = &c->L[sj->li];
        const int e = pj.expert;
        ls->slot_in_flight[sj->slot] = 0;
        if (sj->in_time) {
            c->rec_used[3 * c->n_rec_used] = sj->li;
            c->rec_used[3 * c->n_rec_used + 1] = sj->slot;
            c->rec_used[3 * c->n_rec_used + 2] = e;
            c->n_rec_used++;
        }
        if (sj->landed && ls->expert_slot[e] >= 0) {
            ls->free_slots[ls->n_free++] = sj->slot;
            c->st_n[ST_UNUSED] += !sj->in_time && !sj->late;
            ls->tbl_dirty = 1;
        } else if (sj->landed) {
            ls->slot_expert[sj->slot] = e;
            ls->expert_slot[e] = sj->slot;
            ls->slot_last_use[sj->slot] = sj->in_time || sj->late ? ++c->clock : 1;
            set_table_entry(c, ls, e, sj->slot);
            c->n_published++;
            if (!sj->in_time && !sj->late) c->st_n[ST_UNUSED]++;
        } else {
            ls->free_slots[ls->n_free++] = sj->slot;
        }
        c->st_mark[sj->li * c->E + e] = 0;
    }
    uint64_t pc[4];
    or_planner_counters(c->st_planner, pc);
    c->st_n[ST_DROP_LATE] = pc[2];
    c->st_n[ST_DROP_POSTED] = pc[3];
    c->n_sjobs = 0;
    or_planner_reset(c->st_planner);
    for (int l = 0; l < c->n_layers; ++l) c->st_n_this_token[l] = 0;
    c->st_last_layer = 0xffffffffu;
}

static int job_cmp(const void *a, const void *b) {
    const job_t *x = (const job_t *)a, *y = (const job_t *)b;
    if (x->li != y->li) return x->li < y->li ? -1 : 1;
    return x->slot < y->slot ? -1 : x->slot > y->slot;
}

void or_cache_step(or_cache *c) {
    /* 1) publish every job not held back (sorted when deterministic) */
    job_t *done = (job_t *)malloc(sizeof(job_t) * (size_t)(c->n_jobs + 1));
    int n_done = 0, n_keep = 0;
    for (int j = 0; j < c->n_jobs; ++j) {
        job_t jb = c->jobs[j];
        if (jb.hold) { jb.hold = 0; c->jobs[n_keep++] = jb; }
        else done[n_done++] = jb;
    }
    c->n_jobs = n_keep;
    if (c->k.deterministic) qsort(done, (size_t)n_done, sizeof(job_t), job_cmp);
    for (int j = 0; j < n_done; ++j) {
        layer_t *ls = &c->L[done[j].li];
        ls->slot_expert[done[j].slot] = done[j].expert;
        ls->expert_slot[done[j].expert] = done[j].slot;
        if (done[j].spec && c->spec_probation) {
            /* oldest recency, protected through this step's top-up and the next token */
            ls->slot_last_use[done[j].slot] = 1;
            ls->slot_protect[done[j].slot] = c->n_steps + 1;
        } else {
            ls->slot_last_use[done[j].slot] = ++c->clock;
        }
        ls->slot_in_flight[done[j].slot] = 0;
        set_table_entry(c, ls, done[j].expert, done[j].slot);
        c->n_published++;
    }
    free(done);
    if (c->st_on) stream_adopt(c);      /* after the uploads: an expert both copied is kept once */

    c->n_steps++;

    /* 2) per layer: schedule (non-early) or top the free pool up (early);
     * victims by the evictor's score where it has a model, else LRU */
    float *esc = (float *)malloc(sizeof(float) * (size_t)c->E);
    for (int li = 0; li < c->n_layers; ++li) {
        layer_t *ls = &c->L[li];
        if (!c->k.early_issue) {
            if (ls->n_pending == 0) continue;
            int budget = c->k.max_inserts;
            const int use_model = evict_scores(c, li, esc);
            for (int p = ls->n_pending - 1; p >= 0 && budget > 0; --p) {
                const int id = ls->pending[p];
                if (ls->expert_slot[id] >= 0) { --budget; continue; }
                int slot = -1;
                uint64_t best = U64MAX;
                float best_score = 3.4e38f;
                for (int s = 0; s < ls->S; ++s) {
                    if (ls->slot_in_flight[s]) continue;
                    if (ls->slot_expert[s] < 0) { slot = s; break; }
                    if (ls->slot_protect[s] >= c->n_steps) continue;
                    if (use_model) {
                        const float sc = esc[ls->slot_expert[s]];
                        if (sc < best_score || (sc == best_score && ls->slot_last_use[s] < best)) {
                            best_score = sc;
                            best = ls->slot_last_use[s];
                            slot = s;
                        }
                    } else if (ls->slot_last_use[s] < best) {
                        best = ls->slot_last_use[s];
                        slot = s;
                    }
                }
                if (slot < 0) break;
                const int victim = ls->slot_expert[slot];
                if (!admit_ok(c, ls, id, victim)) continue;
                --budget;
                if (victim >= 0) {
                    ls->expert_slot[victim] = -1;
                    ls->slot_expert[slot] = -1;
                    set_table_entry(c, ls, victim, ls->S);
                }
                ls->slot_in_flight[slot] = 1;
                push_job(c, li, id, slot, 0);
                c->n_scheduled++;
            }
            ls->n_pending = 0;
            continue;
        }
        ls->n_pending = 0;
        const int pool_target = pool_target_of(c);
        const int use_model = evict_scores(c, li, esc);
        while (ls->n_free < pool_target) {
            int slot = -1;
            uint64_t best = U64MAX;
            float best_score = 3.4e38f;
            for (int s = 0; s < ls->S; ++s) {
                if (ls->slot_in_flight[s] || ls->slot_expert[s] < 0) continue;
                if (ls->slot_protect[s] >= c->n_steps) continue;
                if (use_model) {
                    const float sc = esc[ls->slot_expert[s]];
                    if (sc < best_score || (sc == best_score && ls->slot_last_use[s] < best)) {
                        best_score = sc;
                        best = ls->slot_last_use[s];
                        slot = s;
                    }
                } else if (ls->slot_last_use[s] < best) {
                    best = ls->slot_last_use[s];
                    slot = s;
                }
            }
            if (slot < 0) break;
            const int victim = ls->slot_expert[slot];
            ls->expert_slot[victim] = -1;
            ls->slot_expert[slot] = -1;
            set_table_entry(c, ls, victim, ls->S);
            ls->free_slots[ls->n_free++] = slot;
        }
    }
    free(esc);
    /* 0006:915-922: after every eviction decision, this token's ids become the previous ones */
    if (c->evict)
        for (int li = 0; li < c->n_layers; ++li) {
            layer_t *ls = &c->L[li];
            memcpy(ls->prev_ids, ls->cur_ids, sizeof(int32_t) * (size_t)ls->n_cur);
            ls->n_prev_ids = ls->n_cur;
        }

    /* 3) heat decay on a clock */
    if (c->k.admit_mode == 1 && c->k.admit_half > 0 && c->n_steps % (uint64_t)c->k.admit_half == 0) {
        for (int li = 0; li < c->n_layers; ++li)
            for (int e = 0; e < c->E; ++e) c->L[li].heat[e] *= 0.5f;
    }

    /* 4) flush_tables: one batched write of every dirty layer */
    flush_tables(c);

    /* 5) heat file every 512 steps (not while frozen), then the map frame */
    if (!c->freeze && c->heat_path && c->n_steps % 512 == 0) save_heat(c);
    map_frame(c);
    if (c->route) fflush(c->route);
}

static void flush_tables(or_cache *c) {
    if (c->k.batch_tables) {
        int any = 0;
        for (int li = 0; li < c->n_layers; ++li) {
            if (c->L[li].tbl_dirty) { any = 1; c->L[li].tbl_dirty = 0; }
        }
        if (any) c->n_table_flushes++;
    } else {
        for (int li = 0; li < c->n_layers; ++li) c->L[li].tbl_dirty = 0;
    }
}

/* 0007:468-485: "moe-heat 1 <layers> <experts>", then "<il> <expert> <count>"
 * for every non-zero count, written to <path>.tmp and renamed */
static int save_heat(or_cache *c) {
    const size_t n = strlen(c->heat_path);
    char *tmp = (char *)malloc(n + 5);
    memcpy(tmp, c->heat_path, n);
    memcpy(tmp + n, ".tmp", 5);
    FILE *f = fopen(tmp, "w");
    int ok = f != NULL;
    if (f) {
        fprintf(f, "moe-heat 1 %d %d\n", c->n_layers, c->E);
        for (int l = 0; l < c->n_layers; ++l)
            for (int e = 0; e < c->E; ++e)
                if (c->L[l].use_count[e]) fprintf(f, "%d %d %u\n", c->L[l].il, e, c->L[l].use_count[e]);
        ok = fclose(f) == 0 && rename(tmp, c->heat_path) == 0;
    }
    free(tmp);
    return ok ? 0 : -1;
}

int or_cache_heat_file(or_cache *c, const char *path, long long *n_records, long long *n_placed) {
    long long n_rec = 0, placed = 0;
    free(c->heat_path);
    c->heat_path = (char *)malloc(strlen(path) + 1);
    memcpy(c->heat_path, path, strlen(path) + 1);
    for (int l = 0; l < c->n_layers; ++l) {
        free(c->L[l].use_count);
        c->L[l].use_count = (uint32_t *)calloc((size_t)c->E, sizeof(uint32_t));
    }
    /* 0007:434-466: load, refusing another model's dimensions; counts halved */
    FILE *f = fopen(path, "r");
    if (f) {
        int ver = 0, nl = 0, ne = 0;
        if (fscanf(f, "moe-heat %d %d %d", &ver, &nl, &ne) == 3 && ver == 1 && nl == c->n_layers && ne == c->E) {
            int il = 0, e = 0;
            unsigned cnt = 0;
            while (fscanf(f, "%d %d %u", &il, &e, &cnt) == 3) {
                if (il < 0 || il >= c->n_layers || e < 0 || e >= c->E) continue;
                c->L[il].use_count[e] = cnt / 2;
                n_rec++;
            }
        }
        fclose(f);
    }
    /* 0007:576-611: hottest first into slots 0.., a reserve left for early issue */
    if (n_rec > 0) {
        const int reserve = c->k.early_issue ? (c->freeze ? 0 : c->k.max_inserts + (c->pred ? c->predict_top : 0)) : 0;
        int32_t *order = (int32_t *)malloc(sizeof(int32_t) * (size_t)c->E);
        for (int l = 0; l < c->n_layers; ++l) {
            layer_t *ls = &c->L[l];
            for (int e = 0; e < ls->E; ++e) order[e] = e;
            for (int i = 1; i < ls->E; ++i) {             /* stable insertion sort, count descending */
                const int32_t v = order[i];
                int j = i - 1;
                while (j >= 0 && ls->use_count[order[j]] < ls->use_count[v]) { order[j + 1] = order[j]; --j; }
                order[j + 1] = v;
            }
            const int fill = ls->S - reserve > 0 ? ls->S - reserve : 0;
            int slot = 0;
            for (int k = 0; k < ls->E && slot < fill; ++k) {
                const int e = order[k];
                if (ls->use_count[e] == 0) break;
                ls->slot_expert[slot] = e;
                ls->expert_slot[e] = slot;
                ls->slot_last_use[slot] = (uint64_t)(fill - slot);
                set_table_entry(c, ls, e, slot);
                ++slot;
                ++placed;
            }
            if ((uint64_t)fill > c->clock) c->clock = (uint64_t)fill;
            ls->n_free = 0;
            for (int s = ls->S - 1; s >= slot; --s) ls->free_slots[ls->n_free++] = s;
        }
        free(order);
        flush_tables(c);
    }
    if (n_records) *n_records = n_rec;
    if (n_placed) *n_placed = placed;
    return 0;
}

void or_cache_freeze(or_cache *c) {
    c->freeze = 1;
    c->k.max_inserts = 0;
}

int or_cache_map_replay(or_cache *c, const char *path) {
    FILE *f = fopen(path, "r");
    if (!f) return -1;
    int ver = 0, nl = 0;
    int ok = fscanf(f, "moe-map %d %d", &ver, &nl) == 2 && ver == 1 && nl == c->n_layers;
    for (int l = 0; ok && l < c->n_layers; ++l) {
        int il = -1, s = 0, e = 0;
        ok = fscanf(f, " layer %d %d %d", &il, &s, &e) == 3 && il == c->L[l].il && s == c->L[l].S && e == c->L[l].E;
    }
    if (!ok) { fclose(f); return -1; }
    c->replay = f;
    or_cache_freeze(c);
    map_frame(c);                   /* the frame of step 0, as at init (0008:571) */
    return c->replay_err ? -1 : 0;
}

int or_cache_replay_error(const or_cache *c) { return c->replay_err; }

void or_cache_hold_job(or_cache *c, int layer, int expert, int slot, uint64_t sched_step) {
    c->holds = (job_t *)realloc(c->holds, sizeof(job_t) * (size_t)(c->n_holds + 1));
    job_t j = {layer, expert, slot, sched_step, 1, 0};
    c->holds[c->n_holds++] = j;
}

void or_cache_frame(const or_cache *c, int layer, int32_t *out) {
    const layer_t *ls = &c->L[layer];
    for (int s = 0; s < ls->S; ++s) out[s] = -1;
    for (int e = 0; e < ls->E; ++e)
        if (ls->expert_slot[e] >= 0) out[ls->expert_slot[e]] = e;
}

void or_cache_table(const or_cache *c, int layer, int32_t *tbl, float *prior) {
    const layer_t *ls = &c->L[layer];
    if (tbl) memcpy(tbl, ls->tbl_mirror, sizeof(int32_t) * (size_t)ls->E);
    if (prior) {
        if (ls->prior_mirror) memcpy(prior, ls->prior_mirror, sizeof(float) * (size_t)ls->E);
        else memset(prior, 0, sizeof(float) * (size_t)ls->E);
    }
}

void or_cache_stats(const or_cache *c, or_stats *s) {
    memset(s, 0, sizeof *s);
    s->n_steps = c->n_steps;
    s->clock = c->clock;
    for (int l = 0; l < c->n_layers; ++l) { s->n_hit += c->L[l].n_hit; s->n_miss += c->L[l].n_miss; }
    s->n_uploads = c->n_uploads;
    s->n_scheduled = c->n_scheduled;
    s->n_published = c->n_published;
    s->n_admit_ok = c->n_admit_ok;
    s->n_admit_denied = c->n_admit_denied;
    s->n_table_flushes = c->n_table_flushes;
}
