"""Readers for rocprofv3 result databases (rocpd SQLite) and text summaries.

    python -m tensorpack_amd.profiling summary <results.db> [--command "..."] [--top 12]
    python -m tensorpack_amd.profiling counters <results.db> [--kernel SUBSTR]

`summary` prints the per-kernel table of a `--kernel-trace --stats` run
(calls, total, average, min, max in microseconds); `counters` prints the mean
per-dispatch value of every counter of a `--pmc` run. Only the standard
rocpd views (`kernels`, `counters_collection`) are read.
"""

import argparse
import sqlite3
import sys
from typing import Dict, List, Optional, Tuple


def kernel_stats(db: str) -> List[Tuple[str, int, float, float, float, float]]:
    """(name, calls, total_us, avg_us, min_us, max_us) per kernel, by total time."""
    con = sqlite3.connect(db)
    try:
        rows = con.execute(
            "SELECT name, COUNT(*), SUM(end - start), MIN(end - start), MAX(end - start) FROM kernels "
            "GROUP BY name ORDER BY SUM(end - start) DESC").fetchall()
    finally:
        con.close()
    return [(n, int(c), t / 1e3, t / c / 1e3, lo / 1e3, hi / 1e3) for n, c, t, lo, hi in rows]


def counter_means(db: str, kernel: Optional[str] = None) -> Dict[Tuple[str, str], Tuple[int, float]]:
    """{(kernel_name, counter): (dispatches, mean value per dispatch)}.

    A counter reported per hardware instance (per XCD / shader engine) is summed
    over instances within a dispatch before the mean over dispatches."""
    con = sqlite3.connect(db)
    try:
        rows = con.execute("SELECT kernel_name, counter_name, dispatch_id, SUM(value) FROM counters_collection "
                           "GROUP BY kernel_name, counter_name, dispatch_id").fetchall()
    finally:
        con.close()
    acc: Dict[Tuple[str, str], List[float]] = {}
    for kn, cn, _, v in rows:
        if kernel is not None and kernel not in kn:
            continue
        acc.setdefault((kn, cn), []).append(float(v))
    return {k: (len(v), sum(v) / len(v)) for k, v in acc.items()}


def dispatch_values(db: str, counter: str, kernel: str) -> List[float]:
    """Per-dispatch value of `counter` (summed over hardware instances) for kernels whose
    name contains `kernel`, in dispatch order."""
    con = sqlite3.connect(db)
    try:
        rows = con.execute("SELECT dispatch_id, SUM(value) FROM counters_collection WHERE counter_name = ? "
                           "AND kernel_name LIKE ? GROUP BY dispatch_id ORDER BY dispatch_id",
                           (counter, f"%{kernel}%")).fetchall()
    finally:
        con.close()
    return [float(v) for _, v in rows]


def short_name(name: str, width: int = 90) -> str:
    name = " ".join(name.split())
    return name if len(name) <= width else name[: width - 3] + "..."


def format_summary(db: str, command: Optional[str] = None, top: int = 12) -> str:
    stats = kernel_stats(db)
    total = sum(s[2] for s in stats) or 1.0
    out = []
    if command:
        out.append(f"command: {command}")
    out.append(f"{'kernel':90s} {'calls':>7s} {'total_us':>11s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}")
    for n, c, t, a, lo, hi in stats[:top]:
        out.append(f"{short_name(n):90s} {c:7d} {t:11.1f} {a:9.3f} {lo:9.3f} {hi:9.3f} {100 * t / total:6.2f}")
    return "\n".join(out) + "\n"


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m tensorpack_amd.profiling")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("summary")
    s.add_argument("db")
    s.add_argument("--command")
    s.add_argument("--top", type=int, default=12)
    c = sub.add_parser("counters")
    c.add_argument("db")
    c.add_argument("--kernel")
    a = ap.parse_args(argv)
    if a.cmd == "summary":
        sys.stdout.write(format_summary(a.db, a.command, a.top))
    else:
        for (kn, cn), (n, v) in sorted(counter_means(a.db, a.kernel).items()):
            print(f"{short_name(kn, 70):70s} {cn:24s} dispatches={n:5d} mean={v:.6g}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
