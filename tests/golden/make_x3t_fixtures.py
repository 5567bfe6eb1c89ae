"""Copy the reference's engine-recorded cache traces into gzipped fixtures.

Source (data files only, nothing executed):
  artifacts/x3_logits_1791160431756057451/{0..3}.routes-record.txt
  artifacts/x3_logits_1791160431756057451/{0..3}.map.txt
Recorded by the patched llama.cpp engine on Qwen3-30B-A3B Q4_K_M with
LLAMA_MOE_ADMIT=window, LLAMA_MOE_BATCH_TABLES=1, LLAMA_MOE_CACHE_PRIOR=0, the
byte-priced slot profile and --moe-expert-cache 56 (experiments/x3_fused_bench.py:24-34,
experiments/x3_logits_replay.py:26-65, experiments/r3_real_bench.py:137).

Run from the repository root in a container that has the reference mounted:
  python tests/golden/make_x3t_fixtures.py /root/reference
"""
import gzip
import pathlib
import sys

SRC = "artifacts/x3_logits_1791160431756057451"


def main(ref_root):
    out = pathlib.Path(__file__).resolve().parent / "x3t"
    out.mkdir(exist_ok=True)
    for i in range(4):
        for kind in ("routes-record", "map"):
            src = pathlib.Path(ref_root) / SRC / f"{i}.{kind}.txt"
            data = src.read_bytes()
            with open(out / f"{i}.{kind}.txt.gz", "wb") as raw:
                with gzip.GzipFile(fileobj=raw, mode="wb", compresslevel=9, mtime=0) as f:
                    f.write(data)
            print(src, len(data))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
