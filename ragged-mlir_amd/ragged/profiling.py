"""rocprofv3 summaries: per-kernel durations and HBM traffic counters.

The analogue of the reference's ``bench/profile.py:120-144`` (which
summarises Nsight Compute metrics) for rocprofv3 output on gfx950:

* ``stats``: rocprofv3 ``--kernel-trace --stats`` output reduced to calls /
  average / total per kernel;
* ``counters``: ``rocprofv3 --pmc X`` output reduced to the mean value per
  dispatch of counter X for each kernel, summing the rows one dispatch
  reports (one per TCC channel on some ROCm versions);
* ``traffic``: FETCH_SIZE and WRITE_SIZE runs of a workload, each scaled by
  the factor the same counter reads for a plain copy of known size
  (``bench.py --copy-probe``), into HBM bytes per launch;
* ``resources``: per kernel, the VGPR / AGPR / SGPR / LDS / scratch figures
  and grid the kernel trace records for its dispatches;
* ``report``: one workload's markdown table per kernel from a stats run, the
  FETCH_SIZE / WRITE_SIZE runs and an occupancy run (OccupancyPercent,
  MeanOccupancyPerCU, VALUBusy, MemUnitStalled) plus the algorithmic bytes a
  ``bench.py --details`` file records per kernel role.
* ``dispatches``: a kernel trace of back-to-back calls of a two-launch
  schedule (classification, then the main kernel) reduced per timed pass to
  the time per call, each kernel's duration and the gaps between them;
* ``item_timeline``: the register-resident softmax's item trace (one call
  under ``rg_module_set_trace``, ``bench.py --timeline``) reduced to each
  item class's phase durations and workgroup time, how many workgroups were
  live and merging over the call, and, per chunk class, where a chunk's merge
  time goes.

Both output formats are read: the SQLite database rocprofv3 writes by
default (``*_results.db``, views ``kernels`` and ``counters_collection``) and
``--output-format csv`` files (``*_kernel_stats.csv``,
``*_counter_collection.csv``). No GPU and no torch, so it also runs as a
script: ``python ragged-mlir_amd/ragged/profiling.py traffic ...``.
"""
from __future__ import annotations

import argparse
import csv
import json
from pathlib import Path
import re
import sqlite3
import sys
from typing import Iterable


def _rows(path: Path) -> list[dict[str, str]]:
    with open(path, newline="", encoding="utf-8") as handle:
        return list(csv.DictReader(handle))


def _column(row: dict[str, str], *names: str) -> str:
    for name in names:
        if name in row:
            return row[name]
    raise KeyError(f"none of {names} in columns {sorted(row)}")


def short_name(kernel: str) -> str:
    """``rg::k_softmax_fused<__bf16, long, 8, 16, false, false>(rg::Params)``
    -> ``k_softmax_fused<__bf16, long, 8, 16, false, false>``."""
    name = re.sub(r"\(.*\)$", "", kernel.strip())
    name = re.sub(r"^void\s+", "", name)
    return name.split("::", 1)[-1] if name.startswith("rg::") else name


def _query(path: Path, sql: str) -> list[tuple]:
    connection = sqlite3.connect(f"file:{path}?mode=ro", uri=True)
    try:
        return connection.execute(sql).fetchall()
    finally:
        connection.close()


def kernel_stats(path: Path) -> dict[str, dict[str, float]]:
    """Per kernel: calls, average and total ns, share of the total."""
    out: dict[str, dict[str, float]] = {}
    if Path(path).suffix == ".db":
        records = [(short_name(name), 1, float(duration))
                   for name, duration in _query(path, "select name, duration from kernels")]
    else:
        records = [(short_name(_column(row, "Name", "KernelName", "Kernel_Name")), int(_column(row, "Calls")),
                    float(_column(row, "TotalDurationNs", "Total_Duration_Ns"))) for row in _rows(path)]
    for name, calls, total in records:
        entry = out.setdefault(name, {"calls": 0, "total_ns": 0.0})
        entry["calls"] += calls
        entry["total_ns"] += total
    grand = sum(e["total_ns"] for e in out.values()) or 1.0
    for entry in out.values():
        entry["avg_ns"] = entry["total_ns"] / max(entry["calls"], 1)
        entry["pct"] = 100.0 * entry["total_ns"] / grand
    return out


def counter_per_dispatch(path: Path, counter: str) -> dict[str, dict[str, float]]:
    """Per kernel: dispatches and mean value of ``counter`` per dispatch."""
    per_dispatch: dict[tuple[str, str], float] = {}
    if Path(path).suffix == ".db":
        records = [(str(dispatch), short_name(name), float(value)) for dispatch, name, value in
                   _query(path, "select dispatch_id, kernel_name, value from counters_collection "
                                f"where counter_name = '{counter}'")]
    else:
        records = [(_column(row, "Dispatch_Id", "Dispatch-Id"), short_name(_column(row, "Kernel_Name", "Kernel-Name")),
                    float(_column(row, "Counter_Value", "Counter-Value"))) for row in _rows(path)
                   if _column(row, "Counter_Name", "Counter-Name") == counter]
    for dispatch, name, value in records:
        key = (dispatch, name)
        per_dispatch[key] = per_dispatch.get(key, 0.0) + value
    out: dict[str, dict[str, float]] = {}
    for (_, name), value in per_dispatch.items():
        entry = out.setdefault(name, {"dispatches": 0, "sum": 0.0})
        entry["dispatches"] += 1
        entry["sum"] += value
    for entry in out.values():
        entry["mean"] = entry["sum"] / entry["dispatches"]
    return out


def _match(table: dict[str, dict[str, float]], pattern: str) -> tuple[str, dict[str, float]]:
    hits = [(name, entry) for name, entry in table.items() if re.search(pattern, name)]
    if not hits:
        raise KeyError(f"no kernel matches {pattern!r}; kernels: {sorted(table)}")
    return max(hits, key=lambda item: item[1].get("total_ns", item[1].get("sum", 0.0)))


def copy_factor(fetch_csv: Path, write_csv: Path, copy_bytes: int, pattern: str) -> dict[str, float]:
    """Bytes per counter unit for FETCH_SIZE and WRITE_SIZE, from a copy that
    reads and writes ``copy_bytes`` per dispatch."""
    _, fetch = _match(counter_per_dispatch(fetch_csv, "FETCH_SIZE"), pattern)
    _, write = _match(counter_per_dispatch(write_csv, "WRITE_SIZE"), pattern)
    return {"fetch_bytes_per_unit": copy_bytes / fetch["mean"], "write_bytes_per_unit": copy_bytes / write["mean"],
            "copy_bytes": copy_bytes, "fetch_units": fetch["mean"], "write_units": write["mean"]}


def traffic(fetch_csv: Path, write_csv: Path, pattern: str, factor: dict[str, float]) -> dict[str, float]:
    """HBM bytes per launch of the kernel matching ``pattern``."""
    name, fetch = _match(counter_per_dispatch(fetch_csv, "FETCH_SIZE"), pattern)
    _, write = _match(counter_per_dispatch(write_csv, "WRITE_SIZE"), pattern)
    read_bytes = fetch["mean"] * factor["fetch_bytes_per_unit"]
    write_bytes = write["mean"] * factor["write_bytes_per_unit"]
    return {"kernel": name, "dispatches": fetch["dispatches"], "fetch_units": fetch["mean"],
            "write_units": write["mean"], "read_bytes": read_bytes, "write_bytes": write_bytes,
            "bytes": read_bytes + write_bytes}


RESOURCE_COLUMNS = ("vgpr_count", "accum_vgpr_count", "sgpr_count", "lds_size", "static_lds_size", "scratch_size",
                    "static_scratch_size", "grid_x", "workgroup_x")


def kernel_resources(path: Path) -> dict[str, dict[str, float]]:
    """Per kernel (database only): dispatches and the mean of each
    RESOURCE_COLUMNS figure over them."""
    columns = ", ".join(RESOURCE_COLUMNS)
    out: dict[str, dict[str, float]] = {}
    for row in _query(path, f"select name, {columns} from kernels"):
        entry = out.setdefault(short_name(row[0]), {"dispatches": 0, **{c: 0.0 for c in RESOURCE_COLUMNS}})
        entry["dispatches"] += 1
        for column, value in zip(RESOURCE_COLUMNS, row[1:]):
            entry[column] += float(value or 0)
    for entry in out.values():
        for column in RESOURCE_COLUMNS:
            entry[column] /= entry["dispatches"]
    return out


# Kernel-name patterns of the library's launch roles (bench.py --details keys).
ROLE_PATTERNS = {"init": r"k_init\b", "classify": r"k_classify", "worker": r"k_worker",
                 "fused": r"k_softmax_fused", "deferred": r"k_softmax_deferred", "naive": r"k_naive"}
# rocprofv3 reports vgpr_count as (descriptor granules) x 4; gfx950 wave64
# allocates VGPRs in granules of 8 (compiler remarks: 44 -> 24, 128 -> 64).
VGPR_DECODE = 2
OCCUPANCY_COUNTERS = ("OccupancyPercent", "MeanOccupancyPerCU", "VALUBusy", "MemUnitStalled")


def report(stats_db: Path, fetch_db: Path, write_db: Path, occupancy_db: Path, factor: dict[str, float],
           roles: dict[str, dict], title: str, peak_gbps: float = 8000.0) -> list[str]:
    """Markdown lines: per launched role, the rocprofv3 average duration,
    algorithmic bytes and GB/s, HBM bytes (counters scaled by the copy
    factor) and their ratio to the algorithmic bytes, occupancy and the
    kernel's register / LDS / scratch use."""
    stats = kernel_stats(stats_db)
    resources = kernel_resources(stats_db)
    fetch = counter_per_dispatch(fetch_db, "FETCH_SIZE")
    write = counter_per_dispatch(write_db, "WRITE_SIZE")
    occupancy = {counter: counter_per_dispatch(occupancy_db, counter) for counter in OCCUPANCY_COUNTERS}
    lines = [f"### {title}", "",
             "| role | kernel | calls | avg µs | algorithmic MB | GB/s (% of peak) | HBM read MB | HBM write MB | "
             "HBM / algorithmic | occupancy % | waves/CU | VALU busy % | mem stalled % | VGPR alloc | AGPR alloc | "
             "SGPR | LDS B | scratch B/lane | grid |",
             "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for role, info in roles.items():
        pattern = ROLE_PATTERNS.get(role)
        if pattern is None:
            continue
        try:
            name, stat = _match(stats, pattern)
        except KeyError:
            continue
        avg_us = stat["avg_ns"] / 1e3
        algorithmic = float(info.get("bytes") or 0)
        gbps = algorithmic / (avg_us * 1e-6) / 1e9 if avg_us > 0 else 0.0

        def mean(table, default=float("nan")):
            try:
                return _match(table, pattern)[1]["mean"]
            except KeyError:
                return default

        read_bytes = mean(fetch) * factor["fetch_bytes_per_unit"]
        write_bytes = mean(write) * factor["write_bytes_per_unit"]
        ratio = (read_bytes + write_bytes) / algorithmic if algorithmic else float("nan")
        res = _match(resources, pattern)[1]
        occ = {counter: mean(table) for counter, table in occupancy.items()}
        lines.append(
            f"| {role} | `{name}` | {stat['calls']} | {avg_us:.2f} | {algorithmic / 1e6:.2f} | "
            f"{gbps:.0f} ({100 * gbps / peak_gbps:.1f}%) | {read_bytes / 1e6:.2f} | {write_bytes / 1e6:.2f} | "
            f"{ratio:.3f} | {occ['OccupancyPercent']:.1f} | {occ['MeanOccupancyPerCU']:.1f} | "
            f"{occ['VALUBusy']:.1f} | {occ['MemUnitStalled']:.1f} | {VGPR_DECODE * res['vgpr_count']:.0f} | "
            f"{VGPR_DECODE * res['accum_vgpr_count']:.0f} | {res['sgpr_count']:.0f} | {res['lds_size']:.0f} | "
            f"{res['scratch_size']:.0f} | {res['grid_x'] / max(res['workgroup_x'], 1):.0f} |")
    lines += ["", f"VGPR / AGPR alloc: rocprofv3's `vgpr_count` x {VGPR_DECODE} (it decodes the kernel "
                  "descriptor's register granule as 4; gfx950 wave64 allocates 8 per granule, which the compiler's "
                  "resource remarks confirm). Occupancy counters come from a separate --pmc run."]
    return lines


def dispatch_times(path: Path) -> list[tuple[str, int, int]]:
    """(kernel, start ns, end ns) of every dispatch of a kernel-trace
    database, in start order."""
    try:
        rows = _query(path, "select name, start, end from kernels order by start")
    except sqlite3.OperationalError:
        rows = _query(path, "select s.kernel_name, d.start, d.end from rocpd_kernel_dispatch d "
                            "join rocpd_info_kernel_symbol s on d.kernel_id = s.id order by d.start")
    return [(short_name(name), int(start), int(end)) for name, start, end in rows]


def call_passes(dispatches: list[tuple[str, int, int]], first: str, last: str, skip: int, steps: int,
                passes: int) -> list[dict[str, float]]:
    """Calls of a two-launch schedule: each dispatch of a kernel matching
    ``first`` followed by the next one matching ``last`` (other kernels are
    ignored). After ``skip`` calls, ``passes`` runs of ``steps`` calls each:
    per run, the time per call (first start to last end over the run,
    divided by ``steps``), the mean duration of both kernels, the mean gap
    from the first kernel's end to the second's start, and the mean gap from
    a call's end to the next call's start within the run (µs)."""
    calls, pending = [], None
    for name, start, end in dispatches:
        if re.search(first, name):
            pending = (start, end)
        elif re.search(last, name) and pending is not None:
            calls.append((*pending, start, end))
            pending = None
    out = []
    for k in range(passes):
        run = calls[skip + k * steps: skip + (k + 1) * steps]
        if len(run) < steps:
            raise ValueError(f"pass {k}: {len(run)} of {steps} calls in the trace ({len(calls)} calls in all)")
        mean = lambda values: sum(values) / len(values) / 1e3
        out.append({"calls": steps,
                    "per_call_us": (run[-1][3] - run[0][0]) / steps / 1e3,
                    "first_us": mean([c[1] - c[0] for c in run]),
                    "gap_first_last_us": mean([c[2] - c[1] for c in run]),
                    "last_us": mean([c[3] - c[2] for c in run]),
                    "last_min_us": min(c[3] - c[2] for c in run) / 1e3,
                    "last_max_us": max(c[3] - c[2] for c in run) / 1e3,
                    "gap_next_call_us": mean([run[j + 1][0] - run[j][3] for j in range(steps - 1)]) if steps > 1 else 0.0})
    return out


TIMELINE_CLASSES = {0: "whole", 1: "direct", 2: "tree"}
TIMELINE_PHASES = ("load_max", "exp_sum", "merge", "store")


def item_timeline(records, clock_khz: int, part_rows: int, bins: int = 20) -> dict:
    """Summary of one call's k_softmax_fused item trace.

    ``records``: [items, 8] int64 as rg_module_set_trace writes them: ticket,
    wall-clock stamps at the item's start, after its loads and column max,
    after its column sums (a chunk publishes its statistics next), after the
    segment merge and after its stores are issued, hw_id, and kind (0 whole
    segment, 1 chunk merged directly, 2 chunk merged by tree, +4 deferred,
    plus rows << 8); unused records are zero. Per class: items, mean rows,
    mean phase durations (µs) and workgroup-µs. ``profile``: per 1/bins of the
    call, the items live and merging at its midpoint. ``merge_split``, per
    chunk class: its chunks' merge time split into waiting for the segment's
    last chunk to publish, the chain from that publication until the
    segment's first chunk has the merged statistics (its median per segment
    too), and the others' later wake-ups. Segments are recovered from the
    ticket order (a segment's chunks hold consecutive tickets, all but its
    last of part_rows rows; two segments whose first is a multiple of
    part_rows long are counted as one); segments with a deferred chunk are
    left out of the split."""
    import numpy as np
    trace = np.asarray(records, dtype=np.int64).reshape(-1, 8)
    trace = trace[trace[:, 1] > 0]
    if not len(trace):
        return {"items": 0}
    trace = trace[np.argsort(trace[:, 0], kind="stable")]
    us = 1000.0 / clock_khz
    stamps = (trace[:, 1:6] - trace[:, 1].min()) * us
    kind, rows = trace[:, 7] & 0xff, trace[:, 7] >> 8
    cls, deferred = kind & 3, (kind & 4) != 0
    phases = np.diff(stamps, axis=1)
    busy = stamps[:, 4] - stamps[:, 0]
    span = float(stamps[:, 4].max())
    summary = {"items": int(len(trace)), "span_us": round(span, 2), "workgroup_us": round(float(busy.sum()), 1),
               "classes": {}, "profile": []}
    for code, name in TIMELINE_CLASSES.items():
        mask = cls == code
        if not mask.any():
            continue
        summary["classes"][name] = {
            "items": int(mask.sum()), "deferred": int(deferred[mask].sum()),
            "mean_rows": round(float(rows[mask].mean()), 1),
            "phases_us": {phase: round(float(phases[mask, i].mean()), 2) for i, phase in enumerate(TIMELINE_PHASES)},
            "workgroup_us": round(float(busy[mask].sum()), 1)}
    for lo in np.linspace(0.0, span, bins + 1)[:-1]:
        mid = lo + span / bins / 2
        summary["profile"].append([int(((stamps[:, 0] <= mid) & (stamps[:, 4] > mid)).sum()),
                                   int(((stamps[:, 2] <= mid) & (stamps[:, 3] > mid)).sum())])
    for code in (1, 2):
        name = TIMELINE_CLASSES[code]
        if name not in summary["classes"]:
            continue
        segments, current = [], []
        for i in np.flatnonzero(cls == code):
            current.append(i)
            if rows[i] < part_rows:
                segments.append(np.array(current))
                current = []
        if current:
            segments.append(np.array(current))
        total = sibling = chain = 0.0
        chains = []
        for segment in segments:
            if deferred[segment].any():
                continue
            published, merged = stamps[segment, 2], stamps[segment, 3]
            last = published.max()
            total += float((merged - published).sum())
            sibling += float((last - published).sum())
            chains.append(float(merged.min() - last))
            chain += chains[-1] * len(segment)
        if total > 0:
            summary["classes"][name]["merge_split"] = {
                "segments": len(chains), "merge_workgroup_us": round(total, 1),
                "last_sibling": round(sibling / total, 3), "chain": round(chain / total, 3),
                "wake_spread": round((total - sibling - chain) / total, 3),
                "chain_median_us": round(float(np.median(chains)), 2)}
    return summary


def stats_table(stats: dict[str, dict[str, float]], limit: int = 12) -> Iterable[str]:
    yield "| kernel | calls | avg µs | total µs | % |"
    yield "|---|---:|---:|---:|---:|"
    for name, entry in sorted(stats.items(), key=lambda item: -item[1]["total_ns"])[:limit]:
        yield (f"| `{name}` | {entry['calls']} | {entry['avg_ns'] / 1e3:.2f} | {entry['total_ns'] / 1e3:.1f} | "
               f"{entry['pct']:.1f} |")


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = parser.add_subparsers(dest="command", required=True)
    s = sub.add_parser("stats", help="per-kernel table of a *_kernel_stats.csv")
    s.add_argument("csv", type=Path)
    s.add_argument("--json", action="store_true")
    c = sub.add_parser("counters", help="mean per dispatch of one counter")
    c.add_argument("csv", type=Path)
    c.add_argument("counter")
    t = sub.add_parser("traffic", help="HBM bytes per launch from FETCH_SIZE / WRITE_SIZE runs")
    t.add_argument("--fetch", type=Path, required=True)
    t.add_argument("--write", type=Path, required=True)
    t.add_argument("--kernel", required=True, help="regex of the kernel name")
    t.add_argument("--copy-fetch", type=Path, required=True)
    t.add_argument("--copy-write", type=Path, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--copy-kernel", default="copy|elementwise", help="regex of the copy kernel")
    t.add_argument("--algorithmic-bytes", type=int, help="per launch, for the ratio")
    t.add_argument("--library", type=Path, help="the libragged_hip.so that was profiled (its sha256 is recorded)")
    t.add_argument("--command", action="append", default=[], help="a command that produced the inputs (repeat)")
    t.add_argument("--out", type=Path, help="also write the result as JSON here")
    r = sub.add_parser("resources", help="VGPR/AGPR/SGPR/LDS/scratch per kernel of a kernel-trace database")
    r.add_argument("db", type=Path)
    g = sub.add_parser("dispatches", help="per timed pass: time per call, both kernels and the gaps between them")
    g.add_argument("db", type=Path, help="--kernel-trace database")
    g.add_argument("--first", default="k_classify", help="regex of a call's first kernel")
    g.add_argument("--last", default="k_softmax_fused|k_worker", help="regex of a call's second kernel")
    g.add_argument("--skip", type=int, required=True, help="calls before the first timed pass")
    g.add_argument("--steps", type=int, required=True, help="calls per timed pass")
    g.add_argument("--passes", type=int, default=2)
    m = sub.add_parser("report", help="markdown per-kernel table of one workload")
    m.add_argument("--stats", type=Path, required=True, help="--kernel-trace --stats database")
    m.add_argument("--fetch", type=Path, required=True)
    m.add_argument("--write", type=Path, required=True)
    m.add_argument("--occupancy", type=Path, required=True, help="--pmc " + " ".join(OCCUPANCY_COUNTERS))
    m.add_argument("--copy-fetch", type=Path, required=True)
    m.add_argument("--copy-write", type=Path, required=True)
    m.add_argument("--copy-bytes", type=int, required=True)
    m.add_argument("--copy-kernel", default="copy|elementwise", help="regex of the copy kernel")
    m.add_argument("--details", type=Path, required=True, help="bench.py --details output")
    m.add_argument("--op", help="the op of the details record to use (default: the first)")
    m.add_argument("--title", required=True)
    args = parser.parse_args(argv)
    if args.command == "resources":
        print(json.dumps(kernel_resources(args.db), indent=1))
        return 0
    if args.command == "dispatches":
        rows = call_passes(dispatch_times(args.db), args.first, args.last, args.skip, args.steps, args.passes)
        print("| pass | calls | per call µs | first kernel µs | gap µs | second kernel µs (min-max) | gap to next call µs |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for k, r in enumerate(rows):
            print(f"| {k + 1} | {r['calls']} | {r['per_call_us']:.1f} | {r['first_us']:.2f} | {r['gap_first_last_us']:.2f} | "
                  f"{r['last_us']:.2f} ({r['last_min_us']:.1f}-{r['last_max_us']:.1f}) | {r['gap_next_call_us']:.2f} |")
        return 0
    if args.command == "report":
        factor = copy_factor(args.copy_fetch, args.copy_write, args.copy_bytes, args.copy_kernel)
        records = json.loads(args.details.read_text())["records"]
        record = next(r for r in records if r["select"] == "auto" and (args.op is None or r["op"] == args.op))
        print("\n".join(report(args.stats, args.fetch, args.write, args.occupancy, factor, record["kernels"],
                               args.title)))
        return 0
    if args.command == "stats":
        table = kernel_stats(args.csv)
        print(json.dumps(table, indent=1) if args.json else "\n".join(stats_table(table)))
    elif args.command == "counters":
        print(json.dumps(counter_per_dispatch(args.csv, args.counter), indent=1))
    else:
        factor = copy_factor(args.copy_fetch, args.copy_write, args.copy_bytes, args.copy_kernel)
        result = {"factor": factor, **traffic(args.fetch, args.write, args.kernel, factor)}
        if args.algorithmic_bytes:
            result["algorithmic_bytes"] = args.algorithmic_bytes
            result["traffic_over_algorithmic"] = result["bytes"] / args.algorithmic_bytes
        if args.library:
            import hashlib
            result["library_sha256"] = hashlib.sha256(args.library.read_bytes()).hexdigest()
        if args.command:
            result["commands"] = args.command
        text = json.dumps(result, indent=1)
        if args.out:
            args.out.write_text(text + "\n")
        print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
