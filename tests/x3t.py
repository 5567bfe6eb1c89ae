"""Readers for the reference's engine trace formats (fixtures in tests/golden/x3t).

route trace (patches/0008-fused-cpu-moe-rows.patch:508-518):
    route <step> <il> <n_ids> <n_tok> <id>:<slot> ...
placement map (patches/0008-fused-cpu-moe-rows.patch:417-489):
    moe-map 1 <n_layers>
    layer <il> <slots> <experts>          (one per layer)
    step <s>                              (one frame per step, frame 0 at init)
    map <il> <expert of slot 0> ... <expert of slot S-1>   (-1 = empty)
"""
import gzip
import os

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "x3t")


def read_text(path):
    if path.endswith(".gz"):
        with gzip.open(path, "rt") as f:
            return f.read()
    with open(path) as f:
        return f.read()


def parse_map(text):
    lines = text.split("\n")
    head = lines[0].split()
    assert head[0] == "moe-map" and head[1] == "1", head
    n_layers = int(head[2])
    slots, experts = {}, {}
    for k in range(n_layers):
        t = lines[1 + k].split()
        assert t[0] == "layer"
        slots[int(t[1])] = int(t[2])
        experts[int(t[1])] = int(t[3])
    frames, cur = {}, None
    for line in lines[1 + n_layers:]:
        if not line:
            continue
        t = line.split()
        if t[0] == "step":
            cur = int(t[1])
            frames[cur] = {}
        else:
            assert t[0] == "map"
            frames[cur][int(t[1])] = [int(v) for v in t[2:]]
    return slots, experts, frames


def parse_routes(text):
    out = []
    for line in text.split("\n"):
        if not line:
            continue
        t = line.split()
        assert t[0] == "route"
        step, il, n_ids, n_tok = int(t[1]), int(t[2]), int(t[3]), int(t[4])
        pairs = [tuple(int(v) for v in p.split(":")) for p in t[5:]]
        assert len(pairs) == n_ids * n_tok
        out.append((step, il, n_ids, n_tok, pairs))
    return out


def load(i):
    slots, experts, frames = parse_map(read_text(os.path.join(GOLDEN, f"{i}.map.txt.gz")))
    routes = parse_routes(read_text(os.path.join(GOLDEN, f"{i}.routes-record.txt.gz")))
    return slots, experts, frames, routes


# Recording settings of the fixtures: window admission (W = 8), batched tables,
# no cache prior, max_inserts 2 (llama.cpp default for --moe-expert-cache-inserts),
# non-early path, deterministic publication DISABLED (0.log-record.txt), so the
# single upload worker publishes in the order it was handed the jobs.
X3T_KNOBS = dict(max_inserts=2, admit="window", admit_window=8, batch_tables=True,
                 early_issue=False, cache_prior=0.0, deterministic=False)
