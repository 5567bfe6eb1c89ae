"""The byte-priced slot-profile allocator against the reference's own run
(artifacts/p7_slot_allocation.json: inputs and both greedy outputs), and the
profile string against the one the reference's engine traces were recorded
with (experiments/x3_fused_bench.py:29-33)."""
import json
import os

import pytest

from moe_prefetch.slot_profile import allocate_bytes, allocate_slots, profile_string
import x3t

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "p7_slot_allocation.json")


@pytest.fixture(scope="module")
def golden():
    with open(FIX) as f:
        return json.load(f)


def test_slot_priced_greedy_reproduces_reference(golden):
    cap, left = allocate_slots(golden["per_layer_miss8_by_cap"], golden["grid"], golden["baseline_cap"])
    assert cap == golden["new_cap"]
    assert left == golden["leftover"]
    assert sum(cap) == golden["total_budget"]
    assert profile_string(cap, golden["baseline_cap"]) == golden["slot_profile_env"]


def test_byte_priced_greedy_reproduces_reference(golden):
    eb = [golden["expert_bytes"][str(l)] for l in range(48)]
    cap, used, budget = allocate_bytes(golden["per_layer_miss8_by_cap"], golden["grid"], golden["baseline_cap"], eb)
    assert cap == golden["byte_priced_new_cap"]
    assert profile_string(cap, golden["baseline_cap"]) == golden["byte_priced_slot_profile_env"]
    assert abs(budget / 2**20 - golden["byte_priced_vram"]["budget_mib"]) < 1e-6
    assert abs(used / 2**20 - golden["byte_priced_vram"]["used_mib"]) < 1e-6
    assert used <= budget


def test_profile_is_the_one_the_x3t_traces_ran_with(golden):
    slots, _, _, _ = x3t.load(0)
    eb = [golden["expert_bytes"][str(l)] for l in range(48)]
    cap, _, _ = allocate_bytes(golden["per_layer_miss8_by_cap"], golden["grid"], golden["baseline_cap"], eb)
    assert cap == [slots[l] for l in range(48)]


def test_concave_toy_case_is_optimal():
    # two layers, layer 0 gains more per slot: it takes every step first
    grid = [1, 2, 3]
    miss = {1: [8.0, 4.0], 2: [4.0, 3.0], 3: [2.0, 2.5]}
    cap, left = allocate_slots(miss, grid, uniform_cap=2, frozen=[])
    assert cap == [3, 1] and left == 0
