"""Copy the inputs and outputs of the reference's slot-allocation run into a fixture.

Source (data files only, nothing executed):
  artifacts/p7_slot_allocation.json           grid, per-layer misses-of-8 by capacity,
                                              the slot-count greedy's caps and the
                                              byte-priced greedy's caps / env strings
  artifacts/expert_bytes_qwen3-30b-a3b-q4km.json   bytes of one expert per layer
Run: python tests/golden/make_slot_allocation_fixture.py /root/reference
"""
import json
import os
import sys


def main(ref):
    a = json.load(open(os.path.join(ref, "artifacts", "p7_slot_allocation.json")))
    b = json.load(open(os.path.join(ref, "artifacts", "expert_bytes_qwen3-30b-a3b-q4km.json")))
    out = {
        "grid": a["grid"], "baseline_cap": a["baseline_cap"], "total_budget": a["total_budget"],
        "per_layer_miss8_by_cap": a["per_layer_miss8_by_cap"],
        "new_cap": a["new_cap"], "leftover": a["leftover"], "slot_profile_env": a["slot_profile_env"],
        "byte_priced_new_cap": a["byte_priced"]["new_cap"],
        "byte_priced_slot_profile_env": a["byte_priced"]["slot_profile_env"],
        "byte_priced_vram": a["byte_priced"]["vram"],
        "expert_bytes": b,
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "p7_slot_allocation.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
    print(path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
