"""Extract known answers for the split heuristic and the byte model from the reference's
own results files (data only; nothing from the reference is imported or run).

    python tests/golden/make_known_answers.py /root/reference

Writes tests/golden/reference_known_answers.json: for every auto-split row of
results/triton_fp16_splitkv_{A100,T4}.json (reference bench/bench_triton_fp16.py:59-66)
the inputs of choose_num_splits (batch, ctx, block_size, SM count) with the split count
the reference's heuristic picked, and the kv_MB byte count of every row.
"""
import json
import os
import sys


def main(ref):
    out = {"source": "pawaryd/kvq-decode results/*.json (bench/bench_triton_fp16.py output)",
           "kv_heads": 8, "head_dim": 128, "auto_splits": [], "kv_bytes": []}
    for name in ("triton_fp16_splitkv_A100.json", "triton_fp16_splitkv_T4.json"):
        with open(os.path.join(ref, "results", name)) as f:
            d = json.load(f)
        bs, sms = d["block_size"], d["sms"]
        for r in d["rows"]:
            if r["num_splits"] is None:
                out["auto_splits"].append({"file": name, "batch": r["B"], "ctx": r["ctx"],
                                           "block_size": bs, "sms": sms,
                                           "auto_splits": r["auto_splits"]})
                out["kv_bytes"].append({"file": name, "batch": r["B"], "ctx": r["ctx"],
                                        "kv_MB": r["kv_MB"]})
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)),
                        "reference_known_answers.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
    print("wrote", path)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
