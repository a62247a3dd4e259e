"""Extract the reference's recorded continuous-batching run with every
request arriving at t = 0 (bench/serving.json, runs["rate=0"], written by
crates/cli/src/metal_serve.rs:373-469) into serving_rate0.json.

With rate 0 the scheduler's decisions do not depend on measured step times,
so the iteration count, the rows, the KV page peak and the block-table
snapshot statistics are functions of the request stream, the scheduling
policy and the page allocator alone -- golden values for ni_serve on a
host-only handle.  The time-weighted kv_pages_avg_used is left out (it
weighs each iteration by its measured GPU time).

    python tests/golden/make_serving_golden.py /root/reference/bench/serving.json
"""
import json
import os
import sys


def main(src):
    run = json.load(open(src))["runs"]["rate=0"]
    w, c = run["workload"], run["continuous"]
    out = {
        "source": "bench/serving.json runs['rate=0'] (crates/cli/src/metal_serve.rs defaults: seed 7)",
        "workload": {"seed": 7, "requests": w["requests"], "rate": w["rate_req_s"], "prompt": w["prompt"],
                     "output": w["output"], "max_batch": w["max_batch"], "prefill_budget": w["prefill_budget"],
                     "kv_pages": w["kv_pages"], "max_rows": 512, "prompt_tokens": w["prompt_tokens"],
                     "output_tokens": w["output_tokens"]},
        "continuous": {k: c[k] for k in ("iterations", "kv_pages_peak", "rows_computed", "generated_tokens")},
        "kv_stats": c["kv_stats"],
    }
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "serving_rate0.json")
    with open(dst, "w") as f:
        json.dump(out, f, indent=1, sort_keys=True)
        f.write("\n")
    print(dst)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/bench/serving.json")
