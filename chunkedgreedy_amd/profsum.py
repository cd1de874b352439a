"""Summarise a rocprofv3 kernel trace (the SQLite database `--kernel-trace`
writes) as the markdown tables kept under profiles/.

    python -m chunkedgreedy_amd.profsum RESULTS.db [--phase-gap S] [--match RE]
        [--pmc] [--dispatches A:B]
    python -m chunkedgreedy_amd.profsum --traffic FETCH.db WRITE.db
        --calib RE --calib-bytes B [--match RE] [--json] [--dispatches A:B]

Rows are kernels grouped by name (template arguments kept, function
arguments dropped): calls, average / minimum / maximum duration in
microseconds, total milliseconds, and the dispatch's VGPRs, LDS bytes and
grid.  --phase-gap splits the trace where the GPU was idle longer than S
seconds (separate configurations of one sweep run, whose host-side input
generation leaves such gaps) and prints one table per phase.  --match keeps
only kernels whose name matches the regular expression.  --pmc also lists,
per kernel, the mean of every counter the database holds (a `--pmc` run).

--traffic turns two `--pmc` runs of one command (FETCH_SIZE in the first,
WRITE_SIZE in the second, both in KiB per dispatch) into HBM bytes per
dispatch: each counter is scaled by B / (what it reads, per dispatch, for the
calibration kernel matching --calib, which reads B bytes and writes B bytes:
a copy of known size), because the raw counts need not be bytes.  With --json
one JSON object per kernel (fetch_bytes, write_bytes, bytes_per_launch and
the scales, the form bench.py reads from profiles/pmc_traffic.json).
"""

from __future__ import annotations

import argparse
import json
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


def table(rows, pattern: str | None, part: slice | None = None) -> str:
    groups: dict[str, list] = {}
    for name, start, end, vgpr, lds, gx, wx, _ in rows:
        s = short_name(name)
        if pattern and not re.search(pattern, s):
            continue
        groups.setdefault(s, []).append((end - start, vgpr, lds, gx, wx))
    if part is not None:
        groups = {k: v[part] for k, v in groups.items() if v[part]}
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


def counter_means(db: str, counter: str, part: slice | None = None) -> dict:
    """Mean value per dispatch of `counter`, by short kernel name; `part`
    keeps a slice of each kernel's dispatches in launch order."""
    con = sqlite3.connect(db)
    cur = con.cursor()
    acc: dict[str, list] = {}
    for kname, value in cur.execute(
            "select kernel_name, value from counters_collection where counter_name = ? "
            "order by dispatch_id", (counter,)):
        acc.setdefault(short_name(kname), []).append(value)
    out = {}
    for k, v in acc.items():
        if part is not None and not re.search("stream_copy", k):
            v = v[part]
        if v:
            out[k] = (statistics.mean(v), len(v))
    return out


def traffic(fetch_db: str, write_db: str, calib: str, calib_bytes: int,
            pattern: str | None, part: slice | None = None) -> tuple[dict, list]:
    fetch = counter_means(fetch_db, "FETCH_SIZE", part)
    write = counter_means(write_db, "WRITE_SIZE", part)
    cal = [k for k in fetch if re.search(calib, k)]
    if not cal or not any(re.search(calib, k) for k in write):
        raise SystemExit(f"calibration kernel /{calib}/ not in both databases")
    fscale = calib_bytes / (fetch[cal[0]][0] * 1024.0)
    wkey = [k for k in write if re.search(calib, k)][0]
    wscale = calib_bytes / (write[wkey][0] * 1024.0)
    scales = {"fetch_scale": round(fscale, 4), "write_scale": round(wscale, 4),
              "calibration_kernel": cal[0], "calibration_bytes": calib_bytes,
              "calibration_fetch_kib": round(fetch[cal[0]][0], 1),
              "calibration_write_kib": round(write[wkey][0], 1)}
    rows = []
    for k in sorted(set(fetch) | set(write)):
        if pattern and not re.search(pattern, k):
            continue
        f_kib, nf = fetch.get(k, (0.0, 0))
        w_kib, nw = write.get(k, (0.0, 0))
        fb, wb = f_kib * 1024.0 * fscale, w_kib * 1024.0 * wscale
        rows.append({"kernel": k, "dispatches": max(nf, nw), "fetch_kib": round(f_kib, 1),
                     "write_kib": round(w_kib, 1), "fetch_bytes": int(round(fb)),
                     "write_bytes": int(round(wb)), "bytes_per_launch": int(round(fb + wb))})
    return scales, rows


def main(argv=None) -> int:
    if argv is None:
        argv = sys.argv[1:]
    if argv and argv[0] == "--traffic":
        tp = argparse.ArgumentParser(description="HBM bytes per dispatch from two --pmc runs")
        tp.add_argument("--traffic", nargs=2, metavar=("FETCH_DB", "WRITE_DB"), required=True)
        tp.add_argument("--calib", required=True)
        tp.add_argument("--calib-bytes", type=int, required=True)
        tp.add_argument("--match", default=None)
        tp.add_argument("--json", action="store_true")
        tp.add_argument("--dispatches", default=None, metavar="A:B",
                        help="only dispatches A..B-1 of each kernel, in launch order (the "
                        "calibration kernel's are all kept)")
        t = tp.parse_args(argv)
        part = None
        if t.dispatches:
            a, b = t.dispatches.split(":")
            part = slice(int(a) if a else None, int(b) if b else None)
        scales, rows = traffic(t.traffic[0], t.traffic[1], t.calib, t.calib_bytes, t.match,
                               part)
        if t.json:
            for r in rows:
                print(json.dumps({**r, **scales}))
            return 0
        print(f"calibration `{scales['calibration_kernel']}` over {t.calib_bytes} bytes: "
              f"FETCH_SIZE {scales['calibration_fetch_kib']} KiB, WRITE_SIZE "
              f"{scales['calibration_write_kib']} KiB per dispatch; scales "
              f"{scales['fetch_scale']} (fetch) and {scales['write_scale']} (write)\n")
        print("| kernel | dispatches | FETCH_SIZE KiB | fetched MB | WRITE_SIZE KiB | written MB "
              "| total MB |")
        print("|---|---|---|---|---|---|---|")
        for r in rows:
            print(f"| `{r['kernel']}` | {r['dispatches']} | {r['fetch_kib']} | "
                  f"{r['fetch_bytes'] / 1e6:.1f} | {r['write_kib']} | {r['write_bytes'] / 1e6:.1f} "
                  f"| {r['bytes_per_launch'] / 1e6:.1f} |")
        return 0
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("db")
    ap.add_argument("--phase-gap", type=float, default=0.0)
    ap.add_argument("--match", default=None)
    ap.add_argument("--pmc", action="store_true")
    ap.add_argument("--dispatches", default=None, metavar="A:B",
                    help="only dispatches A..B-1 of each kernel, in launch order")
    a = ap.parse_args(argv)
    part = None
    if a.dispatches:
        lo, hi = a.dispatches.split(":")
        part = slice(int(lo) if lo else None, int(hi) if hi else None)
    con, rows = load(a.db)
    for i, ph in enumerate(phases(rows, a.phase_gap)):
        if a.phase_gap > 0:
            span = (ph[-1][2] - ph[0][1]) / 1e9
            print(f"\n### phase {i + 1}: {len(ph)} dispatches over {span:.2f} s\n")
        print(table(ph, a.match, part))
    if a.pmc:
        print()
        print(pmc_table(con, a.match))
    return 0


if __name__ == "__main__":
    sys.exit(main())
