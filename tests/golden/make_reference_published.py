"""Extract the reference's published ozaki_matmul timings (reference/test_results.csv
of WhFanatic/Ozaki_triton: do_bench times in ms on its own, unnamed NVIDIA GPU)
into reference_published.json, for `bench.py --reference-shapes`.

Kept: the Ozaki rows (splits 1-4; splits 0 is the naive fp16 matmul), with
their CSV line numbers.  Columns: scenario, input/slice dtype, shape
(B, M, N, K), splits, ozaki_time (ms), rel_error (against a @ b in the input
dtype, test.py:112-128).  Run in a container that has /root/reference:
    python tests/golden/make_reference_published.py
"""
import csv
import json
import os
import sys

SRC = sys.argv[1] if len(sys.argv) > 1 else "/root/reference/reference/test_results.csv"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_published.json")

rows = []
with open(SRC, newline="") as f:
    for line_no, r in enumerate(csv.DictReader(f), start=2):
        s = int(r["splits"])
        if s < 1:
            continue
        rows.append({
            "csv_line": line_no,
            "scenario": r["scenario"],
            "input_dtype": r["input_dtype"],
            "slice_dtype": r["slice_dtype"],
            "shape_bmnk": [int(x) for x in r["shape"].strip("()").split(",")],
            "splits": s,
            "ozaki_ms": float(r["ozaki_time"]),
            "rel_error": float(r["rel_error"]),
        })
with open(OUT, "w") as f:
    f.write('{"source": "reference/test_results.csv (WhFanatic/Ozaki_triton)",\n "rows": [\n')
    f.write(",\n".join("  " + json.dumps(r) for r in rows))
    f.write("\n]}\n")
print(f"wrote {len(rows)} rows to {OUT}")
