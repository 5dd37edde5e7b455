"""Writes tests/golden/pareto_qt_kat.json: the reference's published (bits,
rel_err) known answers for its allocators, copied as data from the reference's
results/pareto.json: the quadtree families (QT, QT-P) and the three uniform-block
families (16x16 blocks: fixed width, RD without importance, RD with importance)
of every scenario.

Run in the build container, where the reference checkout is mounted:
    python tests/golden/make_pareto_kat.py /root/reference/results/pareto.json
"""

import json
import os
import sys

FAMILIES = ("MTC-QT quadtree 32-4 (ours)", "MTC-QT-P permuted quadtree (ours)",
            "MTC scales, fixed width (ablation)", "MTC-RD, no importance (ablation)", "MTC-RD fixed 16x16 (v1)")


def main(src):
    with open(src) as f:
        data = json.load(f)
    out = {}
    for scenario, fams in data.items():
        keep = {fam: [{"label": p["label"], "bits": p["bits"], "rel_err": p["rel_err"]} for p in pts]
                for fam, pts in fams.items() if fam in FAMILIES}
        if keep:
            out[scenario] = keep
    dst = os.path.join(os.path.dirname(os.path.abspath(__file__)), "pareto_qt_kat.json")
    with open(dst, "w") as f:
        json.dump({"source": "results/pareto.json (Sharexi/TensorPack)", "scenarios": out}, f, indent=1)
    print("wrote", dst)


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/results/pareto.json")
