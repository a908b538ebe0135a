"""Summaries of rocprofv3 result databases for the committed profiles.

    python -m bybylang_amd.profile_summary trace DB [--between-marks]
        per-kernel dispatch count and average / min / max duration (kernel-trace runs); with
        --between-marks only the dispatches that start between the two dispatches of each pair of
        timing marks (the library's timing_mark kernel: bench.py's timed steps)

    python -m bybylang_amd.profile_summary regions DB
        one table per timed region (the dispatches between the two dispatches of each pair of
        timing marks, in order: bench.py's configurations in the order it runs them): the region's
        span from the end of its first mark to the start of its second, and per kernel the dispatch
        count and average / min / max duration

    python -m bybylang_amd.profile_summary regions DB --timed
        the same for every second region only, in one table with short kernel names: bench.py's
        recordings run once when they are made and once timed, so these are the timed replays

    python -m bybylang_amd.profile_summary traffic --fetch DB --write DB --copy-bytes N
                                                   --kernel SUBSTRING [--json OUT]
        HBM bytes per dispatch of the kernel whose name contains SUBSTRING, from a FETCH_SIZE run
        and a WRITE_SIZE run (KiB per dispatch). Each counter is scaled by what it reads for the
        library's copy kernel (copy_words) moving N bytes in the same run, so the figure is in the
        units of a known transfer: factor = N / (counter KiB * 1024) for reads and for writes.

    python -m bybylang_amd.profile_summary counters DB [DB ...] --kernel SUBSTRING
        for each kernel whose name contains SUBSTRING: the average per dispatch of every counter
        in the databases (summed over the counter's instances: XCDs, SEs, CUs), and the average
        dispatch duration

The databases are the *_results.db files rocprofv3 writes with -d/-o.
"""
from __future__ import annotations

import argparse
import collections
import json
import sqlite3
import sys


def kernel_durations(db: str):
    con = sqlite3.connect(db)
    rows = con.execute("select name, count(*), avg(end-start), min(end-start), max(end-start) "
                       "from kernels group by name order by sum(end-start) desc").fetchall()
    con.close()
    return rows


def kernel_durations_between_marks(db: str):
    """kernel_durations over the dispatches that start between consecutive timing_mark dispatches
    (pairs 1-2, 3-4, ...), in the same row format."""
    con = sqlite3.connect(db)
    rows = con.execute("select name, start, end from kernels order by start").fetchall()
    con.close()
    marks = [st for name, st, _ in rows if "timing_mark" in name]
    spans = list(zip(marks[0::2], marks[1::2]))
    per = collections.defaultdict(list)
    for name, st, en in rows:
        if "timing_mark" not in name and any(a < st < b for a, b in spans):
            per[name].append(en - st)
    out = [(k, len(v), sum(v) / len(v), min(v), max(v)) for k, v in per.items()]
    return sorted(out, key=lambda r: -r[1] * r[2])


def kernel_regions(db: str):
    """[(span ns, [(name, n, avg, min, max), ...]), ...] per pair of timing marks, in time order."""
    con = sqlite3.connect(db)
    rows = con.execute("select name, start, end from kernels order by start").fetchall()
    con.close()
    marks = [(st, en) for name, st, en in rows if "timing_mark" in name]
    out = []
    for (a0, a1), (b0, _) in zip(marks[0::2], marks[1::2]):
        per = collections.defaultdict(list)
        for name, st, en in rows:
            if "timing_mark" not in name and a0 < st < b0:
                per[name].append(en - st)
        stats = [(k, len(v), sum(v) / len(v), min(v), max(v)) for k, v in per.items()]
        out.append((b0 - a1, sorted(stats, key=lambda r: -r[1] * r[2])))
    return out


def short_name(name: str) -> str:
    """A kernel's name without namespaces, return type and parameter list: `q4_gemv<1, 2, ...>`.
    A mangled name (`_ZN5byhip12_GLOBAL__N_114split_rows_f16E...`) gives its last nested part."""
    if name.startswith("_ZN"):
        parts, i = [], 3
        while i < len(name) and name[i].isdigit():
            j = i
            while name[j].isdigit():
                j += 1
            n = int(name[i:j])
            parts.append(name[j:j + n])
            i = j + n
        return parts[-1] if parts else name
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for k, ch in enumerate(name):  # cut at the parameter list: the first "(" outside <...>
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and k > 0 and name[k - 1] != ":" and name[k - 1] != " ":
            name = name[:k]
            break
    return name.replace("byhip::(anonymous namespace)::", "").replace("(anonymous namespace)::", "")


def counter_per_dispatch(db: str, counter: str):
    """{kernel name: [value summed over counter instances, per dispatch]}"""
    con = sqlite3.connect(db)
    rows = con.execute("select dispatch_id, kernel_name, value from counters_collection "
                       "where counter_name = ?", (counter,)).fetchall()
    con.close()
    per = collections.defaultdict(lambda: collections.defaultdict(float))
    for d, k, v in rows:
        per[k][d] += v
    return {k: list(v.values()) for k, v in per.items()}


def _pick(per: dict, substring: str):
    names = [k for k in per if substring in k]
    if len(names) != 1:
        raise SystemExit(f"expected one kernel matching {substring!r}, found {names}")
    vals = per[names[0]]
    return names[0], sum(vals) / len(vals), len(vals)


def traffic(fetch_db: str, write_db: str, copy_bytes: int, kernel: str) -> dict:
    fetch = counter_per_dispatch(fetch_db, "FETCH_SIZE")
    write = counter_per_dispatch(write_db, "WRITE_SIZE")
    _, copy_f, ncf = _pick(fetch, "copy_words")
    _, copy_w, ncw = _pick(write, "copy_words")
    name, kf, nkf = _pick(fetch, kernel)
    _, kw, nkw = _pick(write, kernel)
    ff = copy_bytes / (copy_f * 1024.0)
    fw = copy_bytes / (copy_w * 1024.0)
    return {"kernel": name, "dispatches": {"fetch": nkf, "write": nkw, "copy": [ncf, ncw]},
            "copy_bytes": copy_bytes, "copy_fetch_kib": copy_f, "copy_write_kib": copy_w,
            "fetch_factor": ff, "write_factor": fw,
            "kernel_fetch_kib": kf, "kernel_write_kib": kw,
            "fetch_bytes": kf * 1024.0 * ff, "write_bytes": kw * 1024.0 * fw,
            "traffic_bytes": kf * 1024.0 * ff + kw * 1024.0 * fw}


def counters(dbs, kernel: str) -> dict:
    """{kernel name: {"dispatches": n, "avg_us": duration, counter: average per dispatch}}"""
    out = collections.defaultdict(dict)
    for db in dbs:
        con = sqlite3.connect(db)
        rows = con.execute("select dispatch_id, kernel_name, counter_name, value, duration "
                           "from counters_collection").fetchall()
        con.close()
        per = collections.defaultdict(lambda: collections.defaultdict(lambda: collections.defaultdict(float)))
        dur = collections.defaultdict(dict)
        for d, k, c, v, du in rows:
            if kernel in k:
                per[k][c][d] += v
                dur[k][d] = du
        for k, cs in per.items():
            ds = list(dur[k].values())
            out[k]["dispatches"] = len(ds)
            out[k].setdefault("avg_us", sum(ds) / len(ds) / 1e3)
            for c, byd in cs.items():
                out[k][c] = sum(byd.values()) / len(byd)
    return dict(out)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("db")
    t.add_argument("--between-marks", action="store_true")
    g = sub.add_parser("regions")
    g.add_argument("db")
    g.add_argument("--timed", action="store_true")
    r = sub.add_parser("traffic")
    r.add_argument("--fetch", required=True)
    r.add_argument("--write", required=True)
    r.add_argument("--copy-bytes", type=int, required=True)
    r.add_argument("--kernel", required=True)
    r.add_argument("--json")
    c = sub.add_parser("counters")
    c.add_argument("dbs", nargs="+")
    c.add_argument("--kernel", required=True)
    a = ap.parse_args(argv)
    if a.cmd == "counters":
        for name, vals in counters(a.dbs, a.kernel).items():
            print(f"`{name[:110]}`: {vals['dispatches']} dispatches, {vals['avg_us']:.2f} us")
            for k in sorted(v for v in vals if v not in ("dispatches", "avg_us")):
                print(f"  {k} = {vals[k]:.4g}")
        return 0
    if a.cmd == "regions" and a.timed:
        print("| region | span us | kernel | dispatches | avg us | min us | max us |\n"
              "|---:|---:|---|---:|---:|---:|---:|")
        for i, (span, stats) in enumerate(kernel_regions(a.db)):
            if i % 2 == 0:
                continue
            for j, (name, n, avg, mn, mx) in enumerate(stats):
                head = f"| {i} | {span / 1e3:.2f}" if j == 0 else "| |"
                print(f"{head} | `{short_name(name)}` | {n} | {avg / 1e3:.3f} | {mn / 1e3:.3f} | {mx / 1e3:.3f} |")
        return 0
    if a.cmd == "regions":
        for i, (span, stats) in enumerate(kernel_regions(a.db)):
            total = sum(n * avg for _, n, avg, _, _ in stats)
            print(f"\nRegion {i}: span {span / 1e3:.2f} us, kernel time {total / 1e3:.2f} us\n")
            print("| kernel | dispatches | avg us | min us | max us |\n|---|---:|---:|---:|---:|")
            for name, n, avg, mn, mx in stats:
                print(f"| `{name[:110]}` | {n} | {avg / 1e3:.3f} | {mn / 1e3:.3f} | {mx / 1e3:.3f} |")
        return 0
    if a.cmd == "trace":
        print(f"| kernel | dispatches | avg us | min us | max us |\n|---|---:|---:|---:|---:|")
        rows = kernel_durations_between_marks(a.db) if a.between_marks else kernel_durations(a.db)
        for name, n, avg, mn, mx in rows:
            print(f"| `{name[:110]}` | {n} | {avg / 1e3:.3f} | {mn / 1e3:.3f} | {mx / 1e3:.3f} |")
        return 0
    res = traffic(a.fetch, a.write, a.copy_bytes, a.kernel)
    print(json.dumps(res, indent=1))
    if a.json:
        with open(a.json, "w") as f:
            json.dump(res, f, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
