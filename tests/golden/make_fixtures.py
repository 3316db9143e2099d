"""Extract the reference's recorded window-table values into a small JSON fixture.

Run once in the build container (it reads data files under /root/reference; it
imports and runs none of the reference's code):

    python tests/golden/make_fixtures.py [/root/reference]

Sources (all recorded outputs of the reference's own runs):
  window_tables/c1_window_tables.txt               FA4 16-snap zhi and FI vec8 zhi, base 1e7
  window_tables/w_meta_*.json                      inv_freq and fp64 widths from real models
  results_raw/summaries/*.e2e_summary.json         wvec head/tail, fa_zhi, fi_zhi8, fi_s_bar
  e2e_pipeline/n6_1m/*/meta_start.json             wvec head/tail (4 entries each)
  microbench/7b_prefill_mb.json                    qk_slice_ratio_s per N (base 1e7)
  microbench/ports_fig/b1_bench_A*.json            qk_slice_ratio_theory / kload ratio
  evaluations/partial_rope_qk_closed_form/results.csv  closed-form pruned shares
The output, tests/golden/window_golden.json, holds only values (inputs and
expected outputs), no reference source text.
"""
import ast
import csv
import glob
import json
import os
import re
import sys

REF = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "window_golden.json")


def c1_tables():
    txt = open(os.path.join(REF, "window_tables/c1_window_tables.txt"), encoding="utf-8").read()
    rows = []
    k = None
    for line in txt.splitlines():
        m = re.match(r"k=([\d.]+): FA4 16snap len=(\d+) sha=([0-9a-f]+) (\[.*\])", line)
        if m:
            k = float(m.group(1))
            rows.append({"k": k, "fa_sha16": m.group(3), "fa_zhi": ast.literal_eval(m.group(4))})
            continue
        m = re.match(r"\s+FI\s+8snap\s+len=(\d+) sha=([0-9a-f]+) (\[.*\])", line)
        if m:
            rows[-1]["fi_sha16"] = m.group(2)
            rows[-1]["fi_zhi8"] = ast.literal_eval(m.group(3))
    m = re.search(r"wavelengths_sorted head/tail: (\[.*?\]) \.\.\. (\[.*?\])", txt)
    return {"base": 1e7, "head_dim": 128, "cap": 1_100_000, "tables": rows,
            "wvec_head_round1": ast.literal_eval(m.group(1)),
            "wvec_tail_round1": ast.literal_eval(m.group(2))}


def w_meta():
    out = []
    for f in sorted(glob.glob(os.path.join(REF, "window_tables/w_meta_*.json"))):
        d = json.load(open(f))
        out.append({"file": os.path.basename(f), "model": d["model"], "k": d["k_convex"],
                    "head_dim": d.get("head_dim", 2 * len(d["inv_freq"])),
                    "rope_theta": d.get("rope_theta"),
                    "inv_freq": d["inv_freq"], "lam": d["lam"], "w": d["w"]})
    return out


def summaries():
    seen = {}
    files = sorted(glob.glob(os.path.join(REF, "results_raw/summaries/*.e2e_summary.json")))
    files += sorted(glob.glob(os.path.join(REF, "e2e_pipeline/n6_1m/*/e2e_summary.json")))
    for f in files:
        d = json.load(open(f))
        me, ms = d["meta"], d["mma_slices"]
        rec = {"raw_base": me["raw_base"], "head_dim": me["head_dim"],
               "k_prefill": me["k_ret_prefill"], "k_decode": me["k_ret_decode"],
               "wvec_head": me["wvec_head"], "wvec_tail": me["wvec_tail"],
               "fa_zhi": ms["fa_zhi"], "fi_zhi8": ms["fi_zhi8"],
               "fi_s_bar": ms["fi_s_bar"], "at_len": ms["at_len"],
               "fi_ceiling": ms["fi_ceiling_2_over_1ps"]}
        key = json.dumps({k: rec[k] for k in ("raw_base", "k_prefill", "k_decode", "at_len")})
        seen[key] = rec
    for f in sorted(glob.glob(os.path.join(REF, "e2e_pipeline/n6_1m/*/meta_start.json"))):
        d = json.load(open(f))
        rec = {"raw_base": 1e7, "head_dim": 128, "k_prefill": 2.0, "wvec_head": d["wvec_head"],
               "wvec_tail": d["wvec_tail"]}
        seen["meta_start:" + json.dumps(rec["wvec_head"])] = rec
    return list(seen.values())


def prefill_slice_ratios():
    out = []
    d = json.load(open(os.path.join(REF, "microbench/7b_prefill_mb.json")))
    for r in d["results"]:
        out.append({"src": "7b_prefill_mb", "base": 1e7, "head_dim": 128, "k": 2.0, "N": r["N"],
                    "block_m": 128, "block_n": 64, "qk_slice_ratio": r["qk_slice_ratio_s"],
                    "kload_dim_ratio": None})
    bases = {"llama": (5e5, 128, 128, 64), "qwen": (1e6, 64, 128, 128)}
    for f in ("b1_bench_A.json", "b1_bench_A_n128k.json"):
        d = json.load(open(os.path.join(REF, "microbench/ports_fig", f)))
        seen = set()
        for r in d["results"]:
            if "qk_slice_ratio_theory" not in r:
                continue
            key = (r["model"], r["N"])
            if key in seen:
                continue
            seen.add(key)
            base, hd, bm, bn = bases[r["model"]]
            assert hd == r["d"]
            out.append({"src": f, "base": base, "head_dim": hd, "k": 2.0, "N": r["N"],
                        "block_m": bm, "block_n": bn,
                        "qk_slice_ratio": r["qk_slice_ratio_theory"],
                        "kload_dim_ratio": r["kload_dim_ratio_theory"]})
    return out


def closed_form():
    path = os.path.join(REF, "evaluations/partial_rope_qk_closed_form/results.csv")
    with open(path, newline="") as f:
        rows = list(csv.reader(f))
    return {"header": rows[0], "rows": [[int(r[0])] + [float(x) for x in r[1:]] for r in rows[1:]],
            "k": 2.0}


def main():
    fx = {"c1": c1_tables(), "w_meta": w_meta(), "summaries": summaries(),
          "prefill_slice_ratios": prefill_slice_ratios(), "closed_form": closed_form()}
    with open(OUT, "w") as f:
        json.dump(fx, f, indent=1)
    print("wrote", OUT, os.path.getsize(OUT), "bytes")


if __name__ == "__main__":
    main()
