"""Summaries of rocprofv3 output for the GEMV kernels.

    python -m flatrun_amd.profiling trace  <results.db> [--match SUBSTR]
    python -m flatrun_amd.profiling counters <results.db> [--match SUBSTR]
    python -m flatrun_amd.profiling traffic --fetch <fetch.db> --write <write.db>
            [--match SUBSTR ...] [--copy-bytes N]

Every command takes ``--by-grid``: one row per kernel and launch shape.

``trace`` reads a ``rocprofv3 --kernel-trace`` database and prints, per
kernel, the dispatch count and the mean / median / min duration.

``counters`` reads one ``rocprofv3 --pmc`` database of SQ / GRBM counters and
prints, per matched kernel, the mean counters per dispatch and the derived
figures rocprofv3 defines for them: MFMA utilization
(``SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE * SIMDs)``), bf16 MFMA FLOPs
(``SQ_INSTS_VALU_MFMA_MOPS_BF16 * 512``), LDS utilization and bank-conflict
share (per CU), and mean waves per CU. GRBM counters are reduced by max over
their instances (XCDs), SQ counters by sum, as those definitions do.

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
import re
import shutil
import sqlite3
import statistics
import subprocess
import sys

COPY_KERNEL = "copy16_kernel"


def _short_names(raw: list[str]) -> dict[str, str]:
    """Mangled kernel symbol -> ``kernel<template args>`` (namespace, return
    type, argument list and ``.kd`` dropped), through ``c++filt`` when the
    host has it; otherwise the symbols unchanged."""
    tool = shutil.which("c++filt")
    if not tool or not raw:
        return {r: r for r in raw}
    stripped = [r[:-3] if r.endswith(".kd") else r for r in raw]
    try:
        out = subprocess.run([tool], input="\n".join(stripped), capture_output=True, text=True,
                             check=True).stdout.split("\n")
    except (OSError, subprocess.CalledProcessError):
        return {r: r for r in raw}
    short = {}
    for r, d in zip(raw, out):
        d = re.sub(r"^void ", "", d.strip())
        d = d.replace("(anonymous namespace)::", "")
        depth, cut = 0, len(d)
        for i, ch in enumerate(d):               # drop the argument list after the template arguments
            if ch == "<":
                depth += 1
            elif ch == ">":
                depth -= 1
            elif ch == "(" and depth == 0:
                cut = i
                break
        short[r] = d[:cut] or r
    return short


def _dispatches(con, by_grid: bool = False):
    """event id -> (key, duration in ns). The key is the kernel's name, and
    with ``by_grid`` also its launch shape, ``name [wg GXxGY]`` (workgroups
    per dimension), so that one kernel launched on several matrix shapes
    gives one row per shape."""
    names = {r[0]: r[1] for r in con.execute("select id, kernel_name from rocpd_info_kernel_symbol")}
    short = _short_names(list(names.values()))
    names = {k: short[v] for k, v in names.items()}
    out = {}
    for eid, kid, start, end, gx, gy, wx, wy in con.execute(
            "select event_id, kernel_id, start, end, grid_size_x, grid_size_y, workgroup_size_x, "
            "workgroup_size_y from rocpd_kernel_dispatch"):
        key = names.get(kid, "?")
        if by_grid:
            key = f"{key} [wg {gx // max(wx, 1)}x{gy // max(wy, 1)}]"
        out[eid] = (key, end - start)
    return out


def kernel_durations(db: str, by_grid: bool = False) -> dict[str, list[float]]:
    """Kernel name (or name and launch shape) -> durations in microseconds,
    dispatch order."""
    con = sqlite3.connect(db)
    out: dict[str, list[float]] = collections.defaultdict(list)
    for _, (name, dur) in sorted(_dispatches(con, by_grid).items()):
        out[name].append(dur / 1e3)
    return out


def pmc_means(db: str, by_grid: bool = False) -> dict[str, dict[str, float]]:
    """Kernel name (or name and launch shape) -> {counter: mean per dispatch
    (summed over instances)}."""
    con = sqlite3.connect(db)
    disp = _dispatches(con, by_grid)
    counters = {r[0]: r[1] for r in con.execute("select id, name from rocpd_info_pmc")}
    per_event: dict[int, dict[str, float]] = collections.defaultdict(lambda: collections.defaultdict(float))
    for eid, pid, val in con.execute("select event_id, pmc_id, value from rocpd_pmc_event"):
        per_event[eid][counters.get(pid, str(pid))] += val
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for eid, (name, _) in disp.items():
        for c, v in per_event.get(eid, {}).items():
            acc[name][c].append(v)
    return {k: {c: statistics.fmean(v) for c, v in d.items()} for k, d in acc.items()}


CU_NUM, SIMD_NUM = 256, 1024          # MI355X


def pmc_reduced(db: str, by_grid: bool = False) -> dict[str, dict[str, float]]:
    """Kernel name (or name and launch shape) -> {counter: mean per
    dispatch}, instances summed (SQ) or reduced by max (GRBM)."""
    con = sqlite3.connect(db)
    disp = _dispatches(con, by_grid)
    counters = {r[0]: r[1] for r in con.execute("select id, name from rocpd_info_pmc")}
    per_event: dict[int, dict[str, float]] = collections.defaultdict(dict)
    for eid, pid, val in con.execute("select event_id, pmc_id, value from rocpd_pmc_event"):
        c = counters.get(pid, str(pid))
        d = per_event[eid]
        d[c] = max(d.get(c, val), val) if c.startswith("GRBM_") else d.get(c, 0.0) + val
    acc: dict[str, dict[str, list[float]]] = collections.defaultdict(lambda: collections.defaultdict(list))
    for eid, (name, _) in disp.items():
        for c, v in per_event.get(eid, {}).items():
            acc[name][c].append(v)
    return {k: {c: statistics.fmean(v) for c, v in d.items()} for k, d in acc.items()}


def derived(c: dict[str, float]) -> dict[str, float]:
    out = {}
    gui = c.get("GRBM_GUI_ACTIVE")
    if gui:
        if "SQ_VALU_MFMA_BUSY_CYCLES" in c:
            out["mfma_util_pct"] = 100.0 * c["SQ_VALU_MFMA_BUSY_CYCLES"] / (gui * SIMD_NUM)
        if "SQ_LDS_IDX_ACTIVE" in c:
            out["lds_util_pct"] = 100.0 * c["SQ_LDS_IDX_ACTIVE"] / (gui * CU_NUM)
        if "SQ_LDS_BANK_CONFLICT" in c:
            out["lds_bank_conflict_pct"] = 100.0 * c["SQ_LDS_BANK_CONFLICT"] / (gui * CU_NUM)
        if "SQ_WAVE_CYCLES" in c:
            out["waves_per_cu"] = 4.0 * c["SQ_WAVE_CYCLES"] / (gui * CU_NUM)
    if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in c:
        out["mfma_bf16_flop"] = c["SQ_INSTS_VALU_MFMA_MOPS_BF16"] * 512.0
    return out


def _pick(table: dict, match) -> str:
    """The one key of ``table`` that contains every string of ``match``."""
    parts = [match] if isinstance(match, str) else list(match)
    hits = [k for k in table if all(m in k for m in parts)]
    if len(hits) != 1:
        raise SystemExit(f"{parts} match {len(hits)} kernels: {hits}")
    return hits[0]


def traffic(fetch_db: str, write_db: str, match, copy_bytes: int, by_grid: bool = False) -> dict:
    """HBM bytes per launch of the kernel that ``match`` names; with ``match``
    empty, of every kernel present in both databases (one object per key)."""
    f, w = pmc_means(fetch_db, by_grid), pmc_means(write_db, by_grid)
    c_f, c_w = _pick(f, COPY_KERNEL), _pick(w, COPY_KERNEL)
    scale_f = copy_bytes / (f[c_f]["FETCH_SIZE"] * 1024.0)
    scale_w = copy_bytes / (w[c_w]["WRITE_SIZE"] * 1024.0)

    def one(k_f: str, k_w: str) -> dict:
        fetch_b = f[k_f]["FETCH_SIZE"] * 1024.0 * scale_f
        write_b = w[k_w]["WRITE_SIZE"] * 1024.0 * scale_w
        return {"kernel": k_f, "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
                "traffic_bytes": round(fetch_b + write_b),
                "raw_fetch_kib": f[k_f]["FETCH_SIZE"], "raw_write_kib": w[k_w]["WRITE_SIZE"],
                "copy_bytes": copy_bytes, "copy_fetch_kib": f[c_f]["FETCH_SIZE"],
                "copy_write_kib": w[c_w]["WRITE_SIZE"], "fetch_scale": scale_f, "write_scale": scale_w}

    if match:
        return one(_pick(f, match), _pick(w, match))
    return {k: one(k, k) for k in f if k in w and "FETCH_SIZE" in f[k] and "WRITE_SIZE" in w[k]}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("db")
    t.add_argument("--match", default="")
    cn = sub.add_parser("counters")
    cn.add_argument("db")
    cn.add_argument("--match", default="")
    tr = sub.add_parser("traffic")
    tr.add_argument("--fetch", required=True)
    tr.add_argument("--write", required=True)
    tr.add_argument("--match", action="append", default=[],
                    help="substring of the kernel's key; repeat to require several; none: every kernel")
    tr.add_argument("--copy-bytes", type=int, default=256 << 20)
    for p in (t, cn, tr):
        p.add_argument("--by-grid", action="store_true",
                       help="one row per kernel and launch shape (workgroups per dimension)")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        rows = []
        for name, d in kernel_durations(a.db, a.by_grid).items():
            if a.match in name:
                rows.append((statistics.fmean(d), name, d))
        width = 100 if a.by_grid else 72
        print(f"{'kernel':{width}s} {'n':>6s} {'mean_us':>9s} {'median_us':>9s} {'min_us':>8s}")
        for mean, name, d in sorted(rows, reverse=True):
            short = name if len(name) <= width else name[:width - 22] + "~" + name[-21:]
            print(f"{short:{width}s} {len(d):6d} {mean:9.3f} {statistics.median(d):9.3f} {min(d):8.3f}")
    elif a.cmd == "counters":
        table = pmc_reduced(a.db, a.by_grid)
        out = {name: {"counters": c, "derived": derived(c)} for name, c in table.items() if a.match in name}
        print(json.dumps(out, indent=1))
    else:
        print(json.dumps(traffic(a.fetch, a.write, a.match, a.copy_bytes, a.by_grid), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
