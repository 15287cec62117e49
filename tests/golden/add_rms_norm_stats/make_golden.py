"""Extract the element dumps of the reference's add_rms_norm_stats golden self-check
(ascend-kernel/csrc/ops/add_rms_norm_stats/test/f2_golden_selfcheck.json, produced by
run_golden_selfcheck.py:65-103) into a small fixture: for each dumped element of
mode 1's y, the case, its (row, col), the fp64-model value `ref`, the gamma
element and CANN's rstd of that row. The inputs are re-created from the case's
seed by the reference's generator (add_rms_norm_stats_cases.py:33-43), so the
fixture pins the oracle against values the reference recorded.

usage: python tests/golden/add_rms_norm_stats/make_golden.py /root/reference
"""
import json
import os
import sys
import zlib

ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
src = os.path.join(ref_root, "ascend-kernel/csrc/ops/add_rms_norm_stats/test/f2_golden_selfcheck.json")
data = json.load(open(src))
out = {"source": "ascend-kernel/csrc/ops/add_rms_norm_stats/test/f2_golden_selfcheck.json",
       "eps": 1e-6, "mode": 1, "cases": []}
for dump in data["violating_element_dumps"]:
    dtype = dump["dtype"]
    m, k = (int(v) for v in dump["shape"].split("x"))
    torch_name = "torch." + dtype
    seed = zlib.crc32(f"golden/{torch_name}/{dump['case']}".encode()) % 2 ** 31
    out["cases"].append({
        "dtype": dtype, "case": dump["case"], "m": m, "k": k, "seed": seed,
        "elements": [{"row": e["row"], "col": e["col"], "ref": e["ref"], "gamma": e["gamma"],
                      "rstd_cann": e["rstd_cann"]} for e in dump["elements"]],
    })
here = os.path.dirname(os.path.abspath(__file__))
json.dump(out, open(os.path.join(here, "golden_selfcheck_points.json"), "w"), indent=1)
print("wrote", sum(len(c["elements"]) for c in out["cases"]), "points from", len(out["cases"]), "cases")
