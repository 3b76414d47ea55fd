"""Summarise an ``LTV_ERR_REPORT`` file (written by tests/conftest.py at the end
of a pytest session) as a markdown table: one row per (check label,
tolerance), with the number of checks and the worst max |a - e|, normwise
relative error max|a - e| / max|e| and element-wise relative error
max |a - e| / |e| (over |e| >= 1e-2 max|e|) among them.

    python tests/summarize_err_report.py <err.json> [--command "<how it was made>"]
"""

from __future__ import annotations

import argparse
import json
import re
from collections import defaultdict


def check_name(label: str) -> str:
    """A label without its case parameters ("q T=33 r=4 bft" -> "q"; numbers,
    name=value pairs and bracketed lists dropped), so parametrised cases of
    one check share a row."""
    s = re.sub(r"\[[^\]]*\]|\([^)]*\)", " ", label)
    s = re.sub(r"\b[\w.]+=\S*", " ", s)
    s = re.sub(r"(?<![A-Za-z_])[-+]?\d[\d.e+-]*\b", " ", s)
    return " ".join(s.replace(",", " ").split()) or label


def summarize(records):
    groups = defaultdict(list)
    for r in records:
        groups[(check_name(r["label"]), r["tol"])].append(r)
    rows = []
    for (label, tol), rs in groups.items():
        def worst(key):
            vals = [r[key] for r in rs if r.get(key) is not None]
            return max(vals) if vals else None
        rows.append({"label": label, "tol": tol, "checks": len(rs),
                     "elements": sum(int(r.get("size", 0)) for r in rs),
                     "max_abs": worst("max_abs"), "norm_rel": worst("norm_rel"),
                     "elem_rel": worst("elem_rel")})
    rows.sort(key=lambda r: (r["tol"] != 0, -r["checks"], r["label"]))
    return rows


def fmt(v):
    if v is None:
        return "-"
    return "0" if v == 0 else f"{v:.2e}"


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("report")
    ap.add_argument("--command", default="")
    args = ap.parse_args()
    records = json.load(open(args.report))
    rows = summarize(records)
    exact = [r for r in rows if r["tol"] == 0]
    print(f"{len(records)} checks in {len(rows)} groups; "
          f"{sum(r['checks'] for r in exact)} exact (tol 0) checks, worst max|a-e| among them "
          f"{fmt(max((r['max_abs'] or 0) for r in exact) if exact else None)}.\n")
    if args.command:
        print(f"Command: `{args.command}`\n")
    print("| check | tol | checks | elements | worst max abs | worst normwise rel | "
          "worst element-wise rel |")
    print("|---|---:|---:|---:|---:|---:|---:|")
    for r in rows:
        print(f"| {r['label']} | {r['tol']:g} | {r['checks']} | {r['elements']} | "
              f"{fmt(r['max_abs'])} | {fmt(r['norm_rel'])} | {fmt(r['elem_rel'])} |")


if __name__ == "__main__":
    main()
