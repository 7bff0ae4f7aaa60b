"""Summaries of rocprofv3 output for the GEMV kernels.

    python -m flatrun_amd.profiling trace  <results.db> [--match SUBSTR]
    python -m flatrun_amd.profiling traffic --fetch <fetch.db> --write <write.db>
            --match SUBSTR [--copy-bytes N]

``trace`` reads a ``rocprofv3 --kernel-trace`` database and prints, per
kernel, the dispatch count and the mean / median / min duration.

``traffic`` reads two ``rocprofv3 --pmc`` databases (one collected with
``FETCH_SIZE``, one with ``WRITE_SIZE``; both in KiB per dispatch, summed over
every L2 channel) and turns the matched kernel's mean counters into HBM bytes
per launch. The counters are scaled by what they read for the library's
streaming copy kernel (``frq_dev_copy``, run in the same command by
``bench.py --copy-calibration``), whose true traffic is known: ``copy-bytes``
read and ``copy-bytes`` written per launch.

The result is printed as one JSON object; ``bench.py`` reads a saved copy of it
(``profiles/q4_k_gemv_3584x18944.traffic.json``) into ``roofline.traffic``.
"""

from __future__ import annotations

import argparse
import collections
import json
import sqlite3
import statistics
import sys

COPY_KERNEL = "copy16_kernel"


def _dispatches(con):
    names = {r[0]: r[1] for r in con.execute("select id, kernel_name from rocpd_info_kernel_symbol")}
    return {eid: (names.get(kid, "?"), end - start)
            for eid, kid, start, end in con.execute(
                "select event_id, kernel_id, start, end from rocpd_kernel_dispatch")}


def kernel_durations(db: str) -> dict[str, list[float]]:
    """Kernel name -> durations in microseconds, dispatch order."""
    con = sqlite3.connect(db)
    out: dict[str, list[float]] = collections.defaultdict(list)
    for _, (name, dur) in sorted(_dispatches(con).items()):
        out[name].append(dur / 1e3)
    return out


def pmc_means(db: str) -> dict[str, dict[str, float]]:
    """Kernel name -> {counter: mean per dispatch (summed over instances)}."""
    con = sqlite3.connect(db)
    disp = _dispatches(con)
    counters = {r[0]: r[1] for r in con.execute("select id, name from rocpd_info_pmc")}
    per_event: dict[int, dict[str, float]] = collections.defaultdict(lambda: collections.defaultdict(float))
    for eid, pid, val in con.execute("select event_id, pmc_id, value from rocpd_pmc_event"):
        per_event[eid][counters.get(pid, str(pid))] += val
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for eid, (name, _) in disp.items():
        for c, v in per_event.get(eid, {}).items():
            acc[name][c].append(v)
    return {k: {c: statistics.fmean(v) for c, v in d.items()} for k, d in acc.items()}


def _pick(table: dict, match: str) -> str:
    hits = [k for k in table if match in k]
    if len(hits) != 1:
        raise SystemExit(f"'{match}' matches {len(hits)} kernels: {hits}")
    return hits[0]


def traffic(fetch_db: str, write_db: str, match: str, copy_bytes: int) -> dict:
    f, w = pmc_means(fetch_db), pmc_means(write_db)
    k_f, k_w = _pick(f, match), _pick(w, match)
    c_f, c_w = _pick(f, COPY_KERNEL), _pick(w, COPY_KERNEL)
    scale_f = copy_bytes / (f[c_f]["FETCH_SIZE"] * 1024.0)
    scale_w = copy_bytes / (w[c_w]["WRITE_SIZE"] * 1024.0)
    fetch_b = f[k_f]["FETCH_SIZE"] * 1024.0 * scale_f
    write_b = w[k_w]["WRITE_SIZE"] * 1024.0 * scale_w
    return {"kernel": k_f, "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
            "traffic_bytes": round(fetch_b + write_b),
            "raw_fetch_kib": f[k_f]["FETCH_SIZE"], "raw_write_kib": w[k_w]["WRITE_SIZE"],
            "copy_bytes": copy_bytes, "copy_fetch_kib": f[c_f]["FETCH_SIZE"], "copy_write_kib": w[c_w]["WRITE_SIZE"],
            "fetch_scale": scale_f, "write_scale": scale_w}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("db")
    t.add_argument("--match", default="")
    tr = sub.add_parser("traffic")
    tr.add_argument("--fetch", required=True)
    tr.add_argument("--write", required=True)
    tr.add_argument("--match", required=True)
    tr.add_argument("--copy-bytes", type=int, default=256 << 20)
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        rows = []
        for name, d in kernel_durations(a.db).items():
            if a.match in name:
                rows.append((statistics.fmean(d), name, d))
        print(f"{'kernel':72s} {'n':>6s} {'mean_us':>9s} {'median_us':>9s} {'min_us':>8s}")
        for mean, name, d in sorted(rows, reverse=True):
            print(f"{name[:72]:72s} {len(d):6d} {mean:9.3f} {statistics.median(d):9.3f} {min(d):8.3f}")
    else:
        print(json.dumps(traffic(a.fetch, a.write, a.match, a.copy_bytes), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
