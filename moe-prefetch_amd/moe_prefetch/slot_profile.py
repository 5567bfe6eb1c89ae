"""Per-layer slot counts under a fixed VRAM budget (LLAMA_MOE_SLOT_PROFILE).

Restates the reference's allocation (experiments/p7_slot_allocation.py:128-230,
greedy_allocate and greedy_allocate_bytes): start every layer at the smallest
capacity of a measured grid, then repeatedly give the next grid step to the
layer whose step avoids the most misses per unit of cost (slots, or bytes when
expert sizes are given), until the budget of the uniform allocation is spent.
Layers with no measurement are frozen at the uniform capacity.  Equal values go
to the lower layer index.  A layer whose next step no longer fits the remaining
budget leaves the contest for good (the budget only shrinks).

Output feeds MoeCache(slot_profile=...) directly, or as the reference's
"il:slots,..." string (patches/0006-...:447-480).
"""
import heapq


def _greedy(miss_by_cap, grid, n_layers, cost, budget, frozen, uniform_cap, stop_when_empty):
    pos = [0] * n_layers
    cap = [grid[0]] * n_layers
    for l in frozen:
        cap[l] = uniform_cap
    remaining = budget - sum(cap[l] * cost[l] for l in range(n_layers))
    if remaining < 0:
        raise ValueError("the starting allocation already exceeds the budget")

    def next_step(l):
        if l in frozen or pos[l] + 1 >= len(grid):
            return 0.0, 0.0
        a, b = grid[pos[l]], grid[pos[l] + 1]
        gain = miss_by_cap[a][l] - miss_by_cap[b][l]
        price = (b - a) * cost[l]
        return gain / price, price

    heap = []
    for l in range(n_layers):
        v, price = next_step(l)
        if v > 0 and (stop_when_empty is False or price <= remaining):
            heapq.heappush(heap, (-v, l))
    while heap and (remaining > 0 or not stop_when_empty):
        _, l = heapq.heappop(heap)
        v, price = next_step(l)
        if v <= 0 or price > remaining:
            continue
        pos[l] += 1
        cap[l] = grid[pos[l]]
        remaining -= price
        v, price = next_step(l)
        if v > 0 and (stop_when_empty is False or price <= remaining):
            heapq.heappush(heap, (-v, l))
    return cap, remaining


def allocate_slots(miss_by_cap, grid, uniform_cap, frozen=None):
    """Slot-priced greedy: total slots = n_layers * uniform_cap.
    miss_by_cap[c][l] = misses-of-k of layer l at capacity c (c in grid)."""
    miss_by_cap = {int(c): v for c, v in miss_by_cap.items()}
    n_layers = len(miss_by_cap[grid[0]])
    frozen = set(_unmeasured(miss_by_cap, grid, n_layers) if frozen is None else frozen)
    cap, left = _greedy(miss_by_cap, grid, n_layers, [1] * n_layers, n_layers * uniform_cap, frozen,
                        uniform_cap, stop_when_empty=True)
    return cap, int(left)


def allocate_bytes(miss_by_cap, grid, uniform_cap, expert_bytes, frozen=None):
    """Byte-priced greedy: budget = bytes of the uniform allocation; a step's
    value is misses avoided per byte.  expert_bytes[l] (None -> mean)."""
    miss_by_cap = {int(c): v for c, v in miss_by_cap.items()}
    n_layers = len(miss_by_cap[grid[0]])
    frozen = set(_unmeasured(miss_by_cap, grid, n_layers) if frozen is None else frozen)
    known = [b for b in expert_bytes if b]
    mean = sum(known) / len(known)
    cost = [b if b else mean for b in expert_bytes]
    budget = sum(uniform_cap * cost[l] for l in range(n_layers))
    cap, left = _greedy(miss_by_cap, grid, n_layers, cost, budget, frozen, uniform_cap, stop_when_empty=False)
    return cap, budget - left, budget


def _unmeasured(miss_by_cap, grid, n_layers):
    """A layer with zero misses at every capacity has no rows in the corpus."""
    return [l for l in range(n_layers) if all(miss_by_cap[c][l] == 0 for c in grid)]


def profile_string(cap, uniform_cap):
    """'il:slots' for every layer off the uniform capacity, in layer order."""
    return ",".join(f"{l}:{c}" for l, c in enumerate(cap) if c != uniform_cap)
