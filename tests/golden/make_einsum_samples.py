"""Writes tests/golden/einsum_samples.json: the shape fixtures of the
reference's sample workloads (data only: einsum strings, dimension sizes,
contraction paths and contraction trees), read from the reference checkout.

  tccg              samples/tccg/settings_full.cfg and settings_batch.cfg
                    (binary contractions of the TCCG suite, run by the
                    reference through bench_expression with path (0,1))
  einsum_benchmark  samples/einsum_benchmark/{synthetic, str_nw_mera_open_26,
                    lm_first_last_brackets_4_16d,
                    lm_batch_likelihood_sentence_5_16d_batch128}.cfg
                    (expression, sizes, path) and the *_et.cfg trees
                    (bench_tree format) of the first three

Run in a checkout that has the reference at REF (default /root/reference):
    python tests/golden/make_einsum_samples.py [REF]
"""
import json
import os
import re
import sys

HERE = os.path.dirname(os.path.abspath(__file__))


def quoted(line):
    return re.findall(r'"([^"]*)"', line)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    out = {"source": "reference samples/tccg and samples/einsum_benchmark (shape data only)",
           "tccg": [], "einsum_benchmark": {}}
    seen = set()
    for name in ("settings_full.cfg", "settings_batch.cfg"):
        with open(os.path.join(ref, "samples", "tccg", name)) as f:
            for line in f:
                q = quoted(line)
                if len(q) != 3 or (q[0], q[1]) in seen:
                    continue
                seen.add((q[0], q[1]))
                out["tccg"].append({"expr": q[0], "sizes": q[1], "path": q[2], "file": name})
    eb = os.path.join(ref, "samples", "einsum_benchmark")
    for name in ("synthetic", "str_nw_mera_open_26", "lm_first_last_brackets_4_16d",
                 "lm_batch_likelihood_sentence_5_16d_batch128"):
        with open(os.path.join(eb, name + ".cfg")) as f:
            q = quoted(f.read())
        entry = {"expr": q[0], "sizes": q[1], "path": q[2]}
        et = os.path.join(eb, name + "_et.cfg")
        if os.path.exists(et):
            with open(et) as f:
                t = quoted(f.read())
            entry["tree"], entry["tree_sizes"] = t[0], t[1]
        out["einsum_benchmark"][name] = entry
    with open(os.path.join(HERE, "einsum_samples.json"), "w") as f:
        json.dump(out, f, indent=1)
    print(f"tccg: {len(out['tccg'])} contractions; einsum_benchmark: {list(out['einsum_benchmark'])}")


if __name__ == "__main__":
    main()
