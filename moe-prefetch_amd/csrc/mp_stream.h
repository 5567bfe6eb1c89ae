// mp_stream.h -- the copy planner of just-in-time expert streaming.
//
// Behaviour follows moe_planner (patches/0010-team-and-streaming.patch:777-909):
// a job is one expert wanted by a target layer before a deadline; jobs go to
// the copy engine earliest deadline first, in chunks of at most chunk_bytes,
// so an urgent job waits at most one chunk behind a less urgent one.  A job
// that can no longer land before its deadline is dropped, not sent late, and
// so are the unfinished jobs of a layer that has already read its table (that
// layer takes no new job until reset()).  A repeat offer with an earlier
// deadline tightens the job (a one-layer-ahead refresh of a two-layer guess).
// hold_after >= 0 holds back, without dropping, jobs whose target lies beyond
// that layer (the host is computing an absent expert of it and a copy would
// slow that).  Pure bookkeeping, one thread.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace mps {

enum Drop { DROP_NONE = 0, DROP_LATE = 1, DROP_POSTED = 2 };

struct PlanJob {
    int target;
    int32_t expert;
    size_t bytes, sent;
    uint64_t deadline_ns;
    int dropped, drop;
};

struct Chunk {
    int job;
    size_t offset, len;
    int last;          // the job's final chunk: its table word goes right after it
};

class Planner {
public:
    explicit Planner(size_t chunk_bytes = 512 * 1024) : chunk_(chunk_bytes) {}

    void reset() {
        jobs_.clear();
        read_.clear();
    }

    // the new job's id, or -1 (the pair has a job already, or the target has read its table)
    int offer(int target, int32_t expert, size_t bytes, uint64_t deadline_ns) {
        if (has_read(target)) return -1;
        for (PlanJob &j : jobs_) {
            if (j.target != target || j.expert != expert) continue;
            if (!j.dropped && deadline_ns < j.deadline_ns) j.deadline_ns = deadline_ns;
            n_dup++;
            return -1;
        }
        jobs_.push_back(PlanJob{target, expert, bytes, 0, deadline_ns, 0, DROP_NONE});
        n_offered++;
        return (int)jobs_.size() - 1;
    }

    // `target` has read its table: what it still waits for can no longer help
    void posted(int target) {
        if (target >= 0) {
            if ((size_t)target >= read_.size()) read_.resize((size_t)target + 1, 0);
            read_[(size_t)target] = 1;
        }
        for (PlanJob &j : jobs_) {
            if (j.target == target && !j.dropped && j.sent < j.bytes) {
                j.dropped = 1;
                j.drop = DROP_POSTED;
                n_drop_posted++;
            }
        }
    }

    // free_at_ns: when the copy engine finishes what is queued on it already
    bool next(uint64_t free_at_ns, double bytes_per_ns, int hold_after, Chunk &out) {
        int pick = -1;
        for (int i = 0; i < (int)jobs_.size(); ++i) {
            PlanJob &j = jobs_[(size_t)i];
            if (j.dropped || j.sent >= j.bytes) continue;
            const uint64_t lands = free_at_ns + (uint64_t)((double)(j.bytes - j.sent) / bytes_per_ns);
            if (lands > j.deadline_ns) {
                j.dropped = 1;
                j.drop = DROP_LATE;
                n_drop_late++;
                continue;
            }
            if (hold_after >= 0 && j.target > hold_after) continue;
            if (pick < 0 || j.deadline_ns < jobs_[(size_t)pick].deadline_ns) pick = i;
        }
        if (pick < 0) return false;
        PlanJob &j = jobs_[(size_t)pick];
        const size_t left = j.bytes - j.sent;
        out.job = pick;
        out.offset = j.sent;
        out.len = left < chunk_ ? left : chunk_;
        out.last = out.len == left;
        j.sent += out.len;
        return true;
    }

    const PlanJob &get(int id) const { return jobs_[(size_t)id]; }
    int size() const { return (int)jobs_.size(); }

    uint64_t n_offered = 0, n_dup = 0, n_drop_late = 0, n_drop_posted = 0;

private:
    bool has_read(int target) const {
        return target >= 0 && (size_t)target < read_.size() && read_[(size_t)target];
    }
    size_t chunk_;
    std::vector<PlanJob> jobs_;
    std::vector<uint8_t> read_;
};

}  // namespace mps
