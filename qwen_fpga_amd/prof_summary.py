"""Summaries of rocprofv3 records for profiles/: per-kernel durations, split into the phases
that bench.py's config section separates with idle gaps.

    python -m qwen_fpga_amd.prof_summary <rocprofv3 output dir or results .db> [--phases LABEL,...]
                                         [--gap-ms 100]

Reads the kernel dispatch records of a `rocprofv3 --kernel-trace` run (its SQLite results
database), keeps this library's kernels (namespace qh::), splits the timeline where the GPU
idled longer than --gap-ms, drops phases of set-up kernels (no kernel dispatched --min-calls
times), and prints per phase every kernel's dispatch count and mean duration, and the mean
kernel time per op call.  With --phases the phases are labelled in order.
"""
import argparse
import glob
import os
import sqlite3
import statistics


def dispatches(path):
    db = path if path.endswith(".db") else sorted(glob.glob(os.path.join(path, "**", "*.db"), recursive=True))[0]
    c = sqlite3.connect(db)
    return [(n, s, e) for n, s, e in c.execute("select name, start, end from kernels order by start")]


def phases(rows, gap_ms):
    out, cur, last = [], [], None
    for n, s, e in rows:
        if last is not None and (s - last) / 1e6 > gap_ms and cur:
            out.append(cur)
            cur = []
        cur.append((n, s, e))
        last = e if last is None else max(last, e)
    if cur:
        out.append(cur)
    return [[r for r in ph if r[0].startswith(("qh::", "void qh::"))] for ph in out]


def summarise(rows):
    """[(kernel, count, mean us)], kernel us per call, calls: the calls are the dispatches of
    the most frequent kernel; a call's kernels are those dispatched at least half as often
    (a phase's one-off set-up kernels are listed but not counted)."""
    agg = {}
    for n, s, e in rows:
        agg.setdefault(n, []).append((e - s) / 1e3)
    ks = sorted(((n, len(d), statistics.mean(d)) for n, d in agg.items()), key=lambda t: -t[1] * t[2])
    calls = max(c for _, c, _ in ks)
    return ks, sum(c * m for _, c, m in ks if 2 * c >= calls) / calls, calls


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("path")
    ap.add_argument("--phases", default="")
    ap.add_argument("--gap-ms", type=float, default=100.0)
    ap.add_argument("--min-calls", type=int, default=10, help="phases whose kernels ran fewer times are set-up")
    args = ap.parse_args(argv)
    labels = [s for s in args.phases.split(",") if s]
    phs = [p for p in phases(dispatches(args.path), args.gap_ms) if p and summarise(p)[2] >= args.min_calls]
    if len(phs) < len(labels):
        raise SystemExit(f"{len(phs)} phases with qh:: kernels, {len(labels)} labels")
    for i, ph in enumerate(phs):   # phases past the labelled ones are listed unlabelled
        ks, per_call, calls = summarise(ph)
        label = labels[i] if i < len(labels) else f"phase {i}"
        print(f"config {label}: kernel_us_per_call {per_call:.2f} calls {calls}")
        for n, c, m in ks:
            print(f"    {n[:90]:90s} n {c:5d} mean_us {m:9.2f}")


if __name__ == "__main__":
    main()
