"""Summarise a rocprofv3 kernel trace (the SQLite database `--kernel-trace`
writes) as the markdown tables kept under profiles/.

    python -m chunkedgreedy_amd.profsum RESULTS.db [--phase-gap S] [--match RE]
        [--pmc]

Rows are kernels grouped by name (template arguments kept, function
arguments dropped): calls, average / minimum / maximum duration in
microseconds, total milliseconds, and the dispatch's VGPRs, LDS bytes and
grid.  --phase-gap splits the trace where the GPU was idle longer than S
seconds (separate configurations of one sweep run, whose host-side input
generation leaves such gaps) and prints one table per phase.  --match keeps
only kernels whose name matches the regular expression.  --pmc also lists,
per kernel, the mean of every counter the database holds (a `--pmc` run).
"""

from __future__ import annotations

import argparse
import re
import sqlite3
import statistics
import sys


def short_name(name: str) -> str:
    """`ns::(anonymous namespace)::kern<4, 2>(int, ...)` -> `kern<4, 2>`."""
    depth = 0
    cut = len(name)
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not name.startswith("(anonymous", i):
            cut = i
            break
    base = name[:cut]
    base = re.sub(r"^.*::(?=[A-Za-z_][\w]*(<|$))", "", base) if "::" in base else base
    return base.strip() or name


def load(db: str):
    con = sqlite3.connect(db)
    cur = con.cursor()
    rows = cur.execute(
        "select name, start, end, vgpr_count, lds_size, grid_x, workgroup_x, dispatch_id "
        "from kernels order by start").fetchall()
    return con, rows


def phases(rows, gap_s: float):
    if not rows:
        return []
    out, cur = [], [rows[0]]
    for r in rows[1:]:
        if gap_s > 0 and r[1] - cur[-1][2] > gap_s * 1e9:
            out.append(cur)
            cur = []
        cur.append(r)
    out.append(cur)
    return out


def table(rows, pattern: str | None) -> str:
    groups: dict[str, list] = {}
    for name, start, end, vgpr, lds, gx, wx, _ in rows:
        s = short_name(name)
        if pattern and not re.search(pattern, s):
            continue
        groups.setdefault(s, []).append((end - start, vgpr, lds, gx, wx))
    lines = ["| kernel | calls | avg us | min us | max us | total ms | vgpr | lds B | grid x | wg x |",
             "|---|---|---|---|---|---|---|---|---|---|"]
    order = sorted(groups.items(), key=lambda kv: -sum(d[0] for d in kv[1]))
    for s, ds in order:
        dur = [d[0] / 1e3 for d in ds]
        _, vgpr, lds, gx, wx = ds[0]
        lines.append(f"| `{s}` | {len(ds)} | {statistics.mean(dur):.1f} | {min(dur):.1f} | "
                     f"{max(dur):.1f} | {sum(dur) / 1e3:.3f} | {vgpr} | {lds} | {gx} | {wx} |")
    return "\n".join(lines)


def pmc_table(con, pattern: str | None) -> str:
    cur = con.cursor()
    views = {r[0] for r in cur.execute("select name from sqlite_master")}
    if "counters_collection" not in views:
        return "(no counter collection in this database)"
    cols = [r[1] for r in cur.execute("pragma table_info(counters_collection)")]
    kcol = "kernel_name" if "kernel_name" in cols else "name"
    rows = cur.execute(f"select {kcol}, counter_name, value from counters_collection").fetchall()
    acc: dict[tuple, list] = {}
    for kname, cname, value in rows:
        s = short_name(kname)
        if pattern and not re.search(pattern, s):
            continue
        acc.setdefault((s, cname), []).append(value)
    lines = ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---|---|"]
    for (s, cname), vs in sorted(acc.items()):
        lines.append(f"| `{s}` | {cname} | {len(vs)} | {statistics.mean(vs):.1f} |")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("db")
    ap.add_argument("--phase-gap", type=float, default=0.0)
    ap.add_argument("--match", default=None)
    ap.add_argument("--pmc", action="store_true")
    a = ap.parse_args(argv)
    con, rows = load(a.db)
    for i, ph in enumerate(phases(rows, a.phase_gap)):
        if a.phase_gap > 0:
            span = (ph[-1][2] - ph[0][1]) / 1e9
            print(f"\n### phase {i + 1}: {len(ph)} dispatches over {span:.2f} s\n")
        print(table(ph, a.match))
    if a.pmc:
        print()
        print(pmc_table(con, a.match))
    return 0


if __name__ == "__main__":
    sys.exit(main())
