"""Writes results_schema.json: the key structure of the reference's dashboard
data file (site/data/results.json, written by bench/run_bench.py:200-266),
for tests that check nkilab.results emits the same schema.  Run here, where
the reference is mounted; the output is a committed fixture."""
import json
import os
import sys

SRC = "/root/reference/site/data/results.json"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "results_schema.json")


def keys(d):
    return sorted(d.keys())


def common(items):
    """Keys every item of a list (or every value of a dict) carries."""
    items = list(items.values()) if isinstance(items, dict) else list(items)
    out = set(items[0])
    for it in items[1:]:
        out &= set(it)
    return sorted(out)


def main():
    r = json.load(open(SRC))
    schema = {
        "source": "reference site/data/results.json (bench/run_bench.py:200-266, nkilab/profiler.py:210-244)",
        "top": keys(r),
        "versions": keys(r["versions"]),
        "matmul": keys(r["matmul"]),
        "matmul.variants[]": common(r["matmul"]["variants"]),
        "matmul.sweep[]": common(r["matmul"]["sweep"]),
        "norm": keys(r["norm"]),
        "norm.variants[]": common(r["norm"]["variants"]),
        "attention": keys(r["attention"]),
        "attention.ladder[]": common(r["attention"]["ladder"]),
        "attention.scaling[]": common(r["attention"]["scaling"]),
        "decoder_block": keys(r["decoder_block"]),
        "decoder_block.parts[]": common(r["decoder_block"]["parts"]),
        "correctness[]": common(r["correctness"]),
        "traces{}": common(r["traces"]),
        "traces{}.events[]": common(e for t in r["traces"].values() for e in t["events"]),
        "trace_names": sorted(r["traces"].keys()),
        "hardware_model.read_by_dashboard": ["peak_flops.bfloat16", "hbm_bytes_per_s"],
    }
    with open(OUT, "w") as f:
        json.dump(schema, f, indent=1)
    print("wrote", OUT)


if __name__ == "__main__":
    sys.exit(main())
