"""Summaries of rocprofv3 output (the rocpd SQLite database it writes).

    python rocprof_summary.py kernels DIR [--command "..."]
        per-kernel dispatch statistics from a --kernel-trace run (markdown)
    python rocprof_summary.py timeline DIR [--command "..."]
        idle gaps between consecutive dispatches, by kernel pair (markdown)
    python rocprof_summary.py counters DIR
        per-kernel mean of every collected counter from a --pmc run
    python rocprof_summary.py traffic --fetch DIR --write DIR
        --copy-fetch DIR --copy-write DIR --copy-bytes N --kernel NAME --key KEY
        [--json FILE]
        HBM bytes per dispatch of NAME: FETCH_SIZE and WRITE_SIZE (KiB per
        dispatch, one --pmc run each), each scaled by bytes / counter of a plain
        device-to-device copy of known size measured the same way

DIR is a rocprofv3 -d output directory (searched for *_results.db) or a .db
file. Only the standard library is used, so this runs anywhere the database
was copied to.
"""

from __future__ import annotations

import argparse
import json
import re
import sqlite3
import statistics as st
import sys
from pathlib import Path


def _db(path: str) -> Path:
    p = Path(path)
    if p.is_file():
        return p
    found = sorted(p.rglob("*_results.db"))
    if not found:
        raise SystemExit(f"no rocpd database under {path}")
    return found[-1]


def short_name(name: str) -> str:
    n = re.sub(r"^void ", "", name)
    n = re.sub(r"focr::\(anonymous namespace\)::", "", n)
    n = re.sub(r"\(.*$", "", n)  # drop the parameter list
    return n.strip()


def kernel_rows(path: str):
    c = sqlite3.connect(str(_db(path)))
    q = ("select name, duration, grid_x, grid_y, grid_z, workgroup_x, vgpr_count, accum_vgpr_count, lds_size, "
         "scratch_size from kernels order by start")
    return list(c.execute(q))


def kernels_table(path: str, cmd: str | None = None) -> str:
    agg: dict[str, list] = {}
    for r in kernel_rows(path):
        agg.setdefault(short_name(r[0]), []).append(r)
    out = []
    if cmd:
        out.append(f"command: `{cmd}`\n")
    out.append("| kernel | calls | avg us | median us | min us | max us | grid | wg | vgpr | agpr | lds B | scratch |")
    out.append("|---|---:|---:|---:|---:|---:|---|---:|---:|---:|---:|---:|")
    for k, v in sorted(agg.items(), key=lambda kv: -sum(x[1] for x in kv[1])):
        d = [x[1] / 1000.0 for x in v]
        r = v[0]
        out.append(f"| `{k}` | {len(v)} | {st.mean(d):.3f} | {st.median(d):.3f} | {min(d):.3f} | {max(d):.3f} | "
                   f"{r[2]}x{r[3]}x{r[4]} | {r[5]} | {r[6]} | {r[7]} | {r[8]} | {r[9]} |")
    return "\n".join(out)


def timeline_table(path: str, cmd: str | None = None) -> str:
    """Idle time between consecutive dispatches on the queue, grouped by the
    (previous kernel -> next kernel) pair: the launch/dependency gap a step
    pays per kernel boundary. Gaps over 1 ms (host-side pauses such as the
    bench's phase changes) are left out."""
    c = sqlite3.connect(str(_db(path)))
    rows = list(c.execute("select name, start, duration from kernels order by start"))
    agg: dict[tuple[str, str], list[float]] = {}
    for (n0, s0, d0), (n1, s1, _) in zip(rows, rows[1:]):
        gap = (s1 - (s0 + d0)) / 1000.0
        if gap > 1000.0:
            continue
        agg.setdefault((short_name(n0), short_name(n1)), []).append(gap)
    out = []
    if cmd:
        out.append(f"command: `{cmd}`\n")
    out.append("| previous kernel | next kernel | count | mean gap us | median gap us | min us |")
    out.append("|---|---|---:|---:|---:|---:|")
    for (a, b), v in sorted(agg.items(), key=lambda kv: -len(kv[1])):
        out.append(f"| `{a}` | `{b}` | {len(v)} | {st.mean(v):.3f} | {st.median(v):.3f} | {min(v):.3f} |")
    return "\n".join(out)


def counter_means(path: str) -> dict[tuple[str, str], float]:
    """{(kernel, counter): mean over dispatches of the per-dispatch value}."""
    c = sqlite3.connect(str(_db(path)))
    per: dict[tuple[str, str], dict[int, float]] = {}
    for k, cn, v, d in c.execute("select kernel_name, counter_name, value, dispatch_id from counters_collection"):
        key = (short_name(k), cn)
        per.setdefault(key, {}).setdefault(d, 0.0)
        per[key][d] += float(v)
    return {key: st.mean(dd.values()) for key, dd in per.items()}


def counters_table(path: str) -> str:
    out = ["| kernel | counter | mean per dispatch |", "|---|---|---:|"]
    for (k, cn), v in sorted(counter_means(path).items()):
        out.append(f"| `{k}` | {cn} | {v:.1f} |")
    return "\n".join(out)


def _pick(means: dict, kernel: str, counter: str) -> float:
    hits = [v for (k, cn), v in means.items() if cn == counter and kernel in k]
    if not hits:
        raise SystemExit(f"no {counter} samples for a kernel matching {kernel!r}")
    return hits[0] if len(hits) == 1 else st.mean(hits)


def source_sha16(path) -> str:
    """First 16 hex digits of a source file's SHA-256 (ties a stored
    measurement to the kernel source it was taken on)."""
    import hashlib

    return hashlib.sha256(Path(path).read_bytes()).hexdigest()[:16]


def traffic(args) -> dict:
    fetch_kib = _pick(counter_means(args.fetch), args.kernel, "FETCH_SIZE")
    write_kib = _pick(counter_means(args.write), args.kernel, "WRITE_SIZE")
    copy_fetch = _pick(counter_means(args.copy_fetch), args.copy_kernel, "FETCH_SIZE")
    copy_write = _pick(counter_means(args.copy_write), args.copy_kernel, "WRITE_SIZE")
    f_fetch = args.copy_bytes / (copy_fetch * 1024.0)
    f_write = args.copy_bytes / (copy_write * 1024.0)
    bytes_per = fetch_kib * 1024.0 * f_fetch + write_kib * 1024.0 * f_write
    return {
        "kernel": args.kernel,
        "fetch_kib_per_dispatch": round(fetch_kib, 1),
        "write_kib_per_dispatch": round(write_kib, 1),
        "copy_bytes": args.copy_bytes,
        "copy_fetch_kib": round(copy_fetch, 1),
        "copy_write_kib": round(copy_write, 1),
        "fetch_scale": round(f_fetch, 4),
        "write_scale": round(f_write, 4),
        "bytes_per_dispatch": int(bytes_per),
        **({"source": args.source, "source_sha256_16": source_sha16(args.source)} if args.source else {}),
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="what", required=True)
    k = sub.add_parser("kernels")
    k.add_argument("dir")
    k.add_argument("--command", default=None, help="the profiled command, printed above the table")
    tl = sub.add_parser("timeline")
    tl.add_argument("dir")
    tl.add_argument("--command", default=None, help="the profiled command, printed above the table")
    c = sub.add_parser("counters")
    c.add_argument("dir")
    t = sub.add_parser("traffic")
    for name in ("--fetch", "--write", "--copy-fetch", "--copy-write", "--kernel", "--key"):
        t.add_argument(name, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--copy-kernel", default="copyBuffer")
    t.add_argument("--source", default=None, help="the kernel's source file (its hash is stored with the result)")
    t.add_argument("--json", default=None, help="merge the result into this JSON file under --key")
    a = ap.parse_args(argv)
    if a.what == "kernels":
        print(kernels_table(a.dir, a.command))
    if a.what == "timeline":
        print(timeline_table(a.dir, a.command))
    if a.what == "counters":
        print(counters_table(a.dir))
    if a.what == "traffic":
        res = traffic(a)
        if a.json:
            p = Path(a.json)
            cur = json.loads(p.read_text()) if p.exists() else {}
            cur[a.key] = res
            p.write_text(json.dumps(cur, indent=1, sort_keys=True) + "\n")
        print(json.dumps({a.key: res}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
