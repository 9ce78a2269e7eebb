"""Summarise a rocprofv3 CSV output directory (``--kernel-trace`` and/or
``--pmc`` with ``--output-format csv``) as a Markdown table per kernel.

    python3 -m yuuka_amd.profsum DIR [--steps N] [--by-grid] [--templates] [--counters]

``--steps N`` keeps the dispatches of the last N verify steps: those after
the (N+1)-th-from-last ``accept_finalize_kernel`` up to the last one (every
verify step ends with exactly one). Kernel names are shown without namespace
or template arguments; ``--by-grid`` splits a kernel's rows by grid size and
``--templates`` by template arguments.
With ``--counters`` the per-dispatch average of every collected counter is
appended. Reads the CSV files only; writes to stdout."""
from __future__ import annotations

import argparse
import collections
import csv
import glob
import os
import re


def base_name(name: str, templates: bool = False) -> str:
    """`void yk::(anonymous namespace)::foo<1, 2>(...)` -> `foo` (or `foo<1, 2>`)."""
    n = name.replace("(anonymous namespace)", "anon")
    m = re.search(r"(\w+)\s*(<[^()]*>)?\s*\(", n) or re.search(r"(\w+)\s*[<(]", n)
    if not m:
        return n.strip()
    args = m.group(2) if m.re.groups >= 2 else None
    return m.group(1) + (args if templates and args else "")


def load(directory: str) -> dict:
    files = sorted(glob.glob(os.path.join(directory, "**", "*kernel_trace.csv"), recursive=True)
                   + glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True))
    if not files:
        raise SystemExit(f"no rocprofv3 CSV files under {directory}")
    disp: dict[int, dict] = {}
    for f in files:
        with open(f, newline="") as fh:
            for r in csv.DictReader(fh):
                d = int(r.get("Dispatch_Id") or r.get("Correlation_Id"))
                grid = r.get("Grid_Size") or "x".join(r.get(k, "") for k in ("Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"))
                e = disp.setdefault(d, {"name": r["Kernel_Name"], "grid": grid, "start": int(r["Start_Timestamp"]),
                                        "end": int(r["End_Timestamp"]), "c": {}})
                if "Counter_Name" in r:
                    e["c"][r["Counter_Name"]] = e["c"].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return disp


def summarise(disp: dict, steps: int = 0, by_grid: bool = False, counters: bool = False,
              templates: bool = False) -> str:
    ids = sorted(disp)
    if steps:
        acc = [i for i in ids if base_name(disp[i]["name"]) == "accept_finalize_kernel"]
        if len(acc) < steps + 1:
            raise SystemExit(f"only {len(acc)} verify steps in the trace, {steps + 1} needed")
        first = acc[-(steps + 1)]
        ids = [i for i in ids if first < i <= acc[-1]]
    agg: dict[str, dict] = collections.OrderedDict()
    for i in ids:
        e = disp[i]
        k = base_name(e["name"], templates) + (f" grid={e['grid']}" if by_grid else "")
        g = agg.setdefault(k, {"n": 0, "dur": 0.0, "c": collections.Counter()})
        g["n"] += 1
        g["dur"] += (e["end"] - e["start"]) / 1e3
        for cn, v in e["c"].items():
            g["c"][cn] += v
    total = sum(g["dur"] for g in agg.values())
    div = steps or 1
    names = sorted({cn for g in agg.values() for cn in g["c"]}) if counters else []
    head = "| kernel | launches/step | avg us | us/step | share |" + "".join(f" {c} |" for c in names)
    lines = [head, "|---" * (5 + len(names)) + "|"]
    for k, g in sorted(agg.items(), key=lambda kv: -kv[1]["dur"]):
        n = g["n"]
        row = (f"| `{k}` | {n / div:g} | {g['dur'] / n:.2f} | {g['dur'] / div:.1f} | "
               f"{100 * g['dur'] / total if total else 0:.1f}% |")
        row += "".join(f" {g['c'][c] / n:.6g} |" for c in names)
        lines.append(row)
    lines.append(f"| total | {len(ids) / div:g} | | {total / div:.1f} | 100% |" + " |" * len(names))
    return "\n".join(lines)


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("dir")
    ap.add_argument("--steps", type=int, default=0)
    ap.add_argument("--by-grid", action="store_true")
    ap.add_argument("--templates", action="store_true")
    ap.add_argument("--counters", action="store_true")
    a = ap.parse_args(argv)
    print(summarise(load(a.dir), a.steps, a.by_grid, a.counters, a.templates))


if __name__ == "__main__":
    main()
