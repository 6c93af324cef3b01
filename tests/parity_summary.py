"""Turn the end-to-end parity records of a GPU test run into a markdown table.

The GPU tests append one JSON line per compared output to the file named by
QMOE_PARITY_LOG (tests/parity.py). Records of one check that differ only in
the token index ("token 0", "token 1", ...) are merged into one row: the
worst rel-L2, max-abs and bf16-step error, and the element-weighted
bit-exact fraction. The step error of an element is |got - ref| in bf16
steps of max(|ref|, max|ref| / 256) over the compared output.

    QMOE_PARITY_LOG=gpurun_out/parity.jsonl python -m pytest tests -m gpu
    python tests/parity_summary.py gpurun_out/parity.jsonl > summary.md
"""
import json
import re
import sys
from collections import OrderedDict


def _key(rec):
    what = re.sub(r"\btoken \d+ ", "", rec["what"])
    test = rec.get("test", "").split("::")
    name = "::".join(test[-1:]) if test else ""
    return rec["kind"], name, what


def merge(records):
    rows = OrderedDict()
    for rec in records:
        k = _key(rec)
        n = rec.get("n", 0)
        row = rows.setdefault(k, {"count": 0, "n": 0, "rel_l2": 0.0, "max_abs": 0.0, "max_steps": None,
                                  "max_ref": 0.0, "exact_w": 0.0, "beyond": 0, "outside": None,
                                  "file": rec.get("test", "").split("::")[0]})
        row["count"] += 1
        row["n"] += n
        row["rel_l2"] = max(row["rel_l2"], rec["rel_l2"])
        row["max_abs"] = max(row["max_abs"], rec["max_abs"])
        if "max_steps" in rec:
            row["max_steps"] = max(row["max_steps"] or 0.0, rec["max_steps"])
            row["max_ref"] = max(row["max_ref"], rec["max_ref"])
        row["exact_w"] += rec["bitexact"] * n
        row["beyond"] += rec["beyond"]
        if rec.get("outside_bounds") is not None:
            row["outside"] = (row["outside"] or 0) + rec["outside_bounds"]
    return rows


def table(rows):
    out = ["| test | check | outputs | elements | max rel-L2 | max abs | max bf16 steps | max \\|ref\\| "
           "| bit-exact | beyond 1e-2 + 1 step | outside bounds |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for (kind, test, what), r in rows.items():
        exact = f"{r['exact_w'] / r['n']:.4f}" if r["n"] else "-"
        steps = "-" if r["max_steps"] is None else f"{r['max_steps']:.2f}"
        maxref = "-" if r["max_steps"] is None else f"{r['max_ref']:.3g}"
        outside = "-" if r["outside"] is None else str(r["outside"])
        out.append(f"| {test} | {what} | {r['count']} | {r['n']} | {r['rel_l2']:.2e} | {r['max_abs']:.3g} | {steps} "
                   f"| {maxref} | {exact} | {r['beyond']} | {outside} |")
    return "\n".join(out)


def main(path):
    with open(path) as fh:
        records = [json.loads(line) for line in fh if line.strip()]
    rows = merge(records)
    n = sum(r["n"] for r in rows.values())
    worst = max((r["rel_l2"] for r in rows.values()), default=0.0)
    outside = sum(r["outside"] or 0 for r in rows.values())
    print(f"{len(records)} compared outputs in {len(rows)} checks, {n} elements; worst rel-L2 {worst:.2e} "
          f"(bar 2e-3); elements outside their propagated bounds: {outside}.\n")
    print(table(rows))


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "parity.jsonl")
