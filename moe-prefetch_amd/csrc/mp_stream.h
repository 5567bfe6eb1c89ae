// mp_stream.h -- the copy planner of just-in-time expert streaming.
//
// Behaviour of moe_planner (patches/0010-team-and-streaming.patch:777-909): a
// job is one expert wanted by a target layer before a deadline; the copy
// engine is fed earliest deadline first (the lower job id on equal deadlines),
// in chunks of at most chunk_bytes, so an urgent job waits at most one chunk
// behind a less urgent one. A job whose remaining bytes can no longer land by
// its deadline is dropped, not sent late; so are the unfinished jobs of a
// layer that has read its table, and that layer takes no new job until
// reset(). A repeat offer with an earlier deadline tightens the job (a
// one-layer-ahead refresh of a two-layer guess). hold_after >= 0 holds back,
// without dropping, jobs whose target lies beyond that layer (the host is
// computing an absent expert of it and a copy would slow that).
//
// Layout: the jobs in offer order (a job's id is its index); an index from
// (target, expert) to the job, so a repeat offer costs one lookup; each
// target's job ids, so posting a layer touches only its own jobs; and the
// `open` list -- ids of the jobs with bytes left to send that are not
// dropped, kept in id order -- which is all next() scans. Pure bookkeeping,
// one thread.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <unordered_map>
#include <unordered_set>
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
    int last;          // 1 on the chunk that completes the expert: the mover writes the table word after it
};

class Planner {
public:
    explicit Planner(size_t chunk_bytes = 512 * 1024) : chunk_(chunk_bytes) {}

    // token boundary: forget every job and every layer that has read its table
    void reset() {
        jobs_.clear();
        by_pair_.clear();
        by_target_.clear();
        open_.clear();
        posted_.clear();
    }

    // The new job's id, or -1: the target has read its table, or the pair has
    // a job already (whose deadline an earlier one tightens unless it was dropped).
    int offer(int target, int32_t expert, size_t bytes, uint64_t deadline_ns) {
        if (posted_.count(target)) return -1;
        const auto found = by_pair_.find(pair_key(target, expert));
        if (found != by_pair_.end()) {
            PlanJob &j = jobs_[(size_t)found->second];
            if (!j.dropped && deadline_ns < j.deadline_ns) j.deadline_ns = deadline_ns;
            n_dup++;
            return -1;
        }
        const int id = (int)jobs_.size();
        jobs_.push_back(PlanJob{target, expert, bytes, 0, deadline_ns, 0, DROP_NONE});
        by_pair_.emplace(pair_key(target, expert), id);
        by_target_[target].push_back(id);
        if (bytes > 0) open_.push_back(id);         // an empty job never has a chunk to send
        n_offered++;
        return id;
    }

    // `target` has read its table: what it still waits for can no longer help
    void posted(int target) {
        posted_.insert(target);
        const auto mine = by_target_.find(target);
        if (mine == by_target_.end()) return;
        for (int id : mine->second) {
            PlanJob &j = jobs_[(size_t)id];
            if (!j.dropped && j.sent < j.bytes) retire(j, DROP_POSTED);
        }
        close_dropped();
    }

    // The next chunk for the copy engine, false when nothing can go now.
    // free_at_ns: when the engine finishes what is queued on it already.
    bool next(uint64_t free_at_ns, double bytes_per_ns, int hold_after, Chunk &out) {
        drop_late(free_at_ns, bytes_per_ns);
        const int id = earliest(hold_after);
        if (id < 0) return false;
        PlanJob &j = jobs_[(size_t)id];
        const size_t left = j.bytes - j.sent;
        out.job = id;
        out.offset = j.sent;
        out.len = left < chunk_ ? left : chunk_;
        out.last = out.len == left;
        j.sent += out.len;
        if (out.last) close_finished(id);
        return true;
    }

    const PlanJob &get(int id) const { return jobs_[(size_t)id]; }
    int size() const { return (int)jobs_.size(); }

    uint64_t n_offered = 0, n_dup = 0, n_drop_late = 0, n_drop_posted = 0;

private:
    static uint64_t pair_key(int target, int32_t expert) {
        return (uint64_t)(uint32_t)target << 32 | (uint32_t)expert;
    }

    void retire(PlanJob &j, Drop why) {
        j.dropped = 1;
        j.drop = why;
        (why == DROP_LATE ? n_drop_late : n_drop_posted)++;
    }

    // Every open job whose remaining bytes, started at free_at_ns at
    // bytes_per_ns, would land after its deadline is dropped, held or not.
    void drop_late(uint64_t free_at_ns, double bytes_per_ns) {
        bool any = false;
        for (int id : open_) {
            PlanJob &j = jobs_[(size_t)id];
            const uint64_t lands = free_at_ns + (uint64_t)((double)(j.bytes - j.sent) / bytes_per_ns);
            if (lands > j.deadline_ns) {
                retire(j, DROP_LATE);
                any = true;
            }
        }
        if (any) close_dropped();
    }

    // the open, unheld job with the earliest deadline; the lower id on a tie
    int earliest(int hold_after) const {
        int best = -1;
        for (int id : open_) {
            const PlanJob &j = jobs_[(size_t)id];
            if (hold_after >= 0 && j.target > hold_after) continue;
            if (best < 0 || j.deadline_ns < jobs_[(size_t)best].deadline_ns) best = id;
        }
        return best;
    }

    void close_dropped() {
        size_t keep = 0;
        for (int id : open_)
            if (!jobs_[(size_t)id].dropped) open_[keep++] = id;
        open_.resize(keep);
    }

    void close_finished(int id) {
        for (size_t i = 0; i < open_.size(); ++i)
            if (open_[i] == id) {
                open_.erase(open_.begin() + (ptrdiff_t)i);
                return;
            }
    }

    size_t chunk_;
    std::vector<PlanJob> jobs_;
    std::unordered_map<uint64_t, int> by_pair_;
    std::unordered_map<int, std::vector<int>> by_target_;
    std::vector<int> open_;
    std::unordered_set<int> posted_;
};

}  // namespace mps
