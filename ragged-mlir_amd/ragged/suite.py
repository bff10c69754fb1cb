"""Benchmark suite over the reference's comparison cells, on one MI355X.

Restates the reference's suite runner and timing protocol
(``bench/suite.py:1-60``: one record per (case, seed, repetition), a
complete record is skipped so an interrupted suite resumes; ``bench/run.py``:
complete calls bracketed by events on the calling stream, 5 warm-up calls
and 30 timed ones, "cold" = a flush buffer overwritten before every call,
"graph" = one complete call captured and replayed) for its "compare" group:
sum, max and softmax at f32 for D=1 (16,384 segments, 1,048,576 rows) and
D=128 (4,096 segments, 262,144 rows) over uniform, long_tail and burst
lengths, plus the bf16 D=128 long-tail softmax, seeds 711-713. The inputs are
regenerated bit-identically by ``ragged.workloads`` (their sha256 equal the
reference's records).

Methods, each a complete call that allocates its output as the reference's
do (``bench/run.py:186-193``): ``ragged-auto`` (given ``max_len``, as the
reference's compare runs give it: the cost model decides),
``ragged-auto-no-max-len`` (device classification unless the decision rule
says otherwise), ``ragged-classified`` and ``ragged-naive`` (forced
schedules), and ``torch-segment``: ``torch.segment_reduce`` on the device
(for softmax, composed from two segment reductions and the exponentials;
the reference has no torch-segment softmax; bf16 through f32). Every
method's output passes
``calibrate.gate`` (the longest segment and 64 others against a float64
reference) before it is timed; a method that fails it is recorded as
``wrong`` and not timed.

    python -m ragged.suite run --output DIR [--seeds 711,712,713] [--cases PREFIX,...] [--flush-mib 1024]
    python -m ragged.suite summarize DIR [--reference FILE] > table.md

``--reference`` takes the JSON fixture whose ``recorded_timings`` hold the
reference's medians (``tests/golden/reference_cases.json``, extracted from
the reference's ``results/bench/runs/compare/*/seed-*/rep-0``); the summary
then sets them beside this build's.
"""
from __future__ import annotations

import argparse
import json
from pathlib import Path
import sys
import time

import numpy as np

SEEDS = (711, 712, 713)
SHAPES = {1: (16384, 1 << 20), 128: (4096, 1 << 18)}    # D -> (segments, rows)
DISTRIBUTIONS = ("uniform", "long_tail", "burst")
METHODS = ("ragged-auto", "ragged-auto-no-max-len", "ragged-classified", "ragged-naive", "torch-segment")
WARMUP, TIMED = 5, 30


def compare_cases() -> list[dict]:
    """The comparison group's cases in the reference's naming
    (op-dtype-dD-distribution)."""
    cases = []
    for op in ("max", "softmax", "sum"):
        for d in (1, 128):
            for distribution in DISTRIBUTIONS:
                cases.append({"op": op, "dtype": "f32", "d": d, "distribution": distribution})
    cases.append({"op": "softmax", "dtype": "bf16", "d": 128, "distribution": "long_tail"})
    for case in cases:
        case["segments"], case["rows"] = SHAPES[case["d"]]
        case["key"] = f"{case['op']}-{case['dtype']}-d{case['d']}-{case['distribution']}"
    return sorted(cases, key=lambda c: c["key"])


def cell_inputs(torch, case: dict, seed: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Lengths, i64 offsets and f32 values of one cell, as the reference's
    ``bench/run.py:51-64`` makes them: bf16 cells carry the values rounded to
    bf16 (to nearest, ties to even), which is what their hash covers."""
    from .workloads import make_lengths, offsets_from_lengths, reference_values

    lengths = make_lengths(case["distribution"], case["segments"], seed=seed, total_elements=case["rows"])
    offsets = offsets_from_lengths(lengths, "i64")
    values = reference_values(seed, int(offsets[-1]), case["d"])
    if case["dtype"] == "bf16":
        values = torch.from_numpy(values).to(torch.bfloat16).float().numpy()
    return lengths, offsets, values


def _stats(samples_ms: list[float]) -> dict:
    values = np.array(samples_ms, dtype=np.float64)
    return {"count": int(values.size), "median": float(np.median(values)), "min": float(values.min()),
            "p90": float(np.percentile(values, 90))}


def _time_each(torch, run, calls: int, before=None) -> list[float]:
    """ms of each of `calls` calls, events around every call on the current
    stream; `before` (untimed) runs ahead of each call, followed by a
    synchronisation."""
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(calls)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(calls)]
    for i in range(calls):
        if before is not None:
            before()
            torch.cuda.synchronize()
        starts[i].record()
        run()
        ends[i].record()
    torch.cuda.synchronize()
    return [s.elapsed_time(e) for s, e in zip(starts, ends)]


def _torch_segment(torch, op: str, x, offsets, lengths, n: int):
    """torch's own segmented ops on the device, as the reference's torch
    baseline composes them (bf16 promoted to f32 and converted back)."""
    work = x.float() if x.dtype == torch.bfloat16 else x
    if op in ("sum", "max"):
        return torch.segment_reduce(work, op, offsets=offsets, axis=0).to(x.dtype)
    maxima = torch.segment_reduce(work, "max", offsets=offsets, axis=0)
    weights = torch.exp(work - torch.repeat_interleave(maxima, lengths, dim=0, output_size=n))
    sums = torch.segment_reduce(weights, "sum", offsets=offsets, axis=0)
    return (weights / torch.repeat_interleave(sums, lengths, dim=0, output_size=n)).to(x.dtype)


def _graph(torch, call, check) -> dict:
    """One complete call captured on a side stream and replayed: replay
    times, with the captured output gated after the first replay and again
    after the timed ones (a capture that records work whose replays differ
    fails the second gate)."""
    try:
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            call()                                         # plans and workspaces of this stream
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            y = call()
        graph.replay()
        torch.cuda.synchronize()
        first = check(y)["max_fraction_of_tolerance"]
        times = _stats(_time_each(torch, graph.replay, TIMED))
        last = check(y)["max_fraction_of_tolerance"]
        return {"graph_ms": times, "graph_gate": max(first, last)}
    except Exception as exc:   # noqa: BLE001 - a call that cannot be captured (or replays wrong) is recorded as such
        torch.cuda.synchronize()
        return {"graph_ms": None, "graph_status": f"not measured: {type(exc).__name__}: {exc}"[:300]}


def run_cell(torch, case: dict, seed: int, flush, cache, log=print) -> dict:
    from . import Compiler, ProgramSpec, native
    from .calibrate import gate
    from .workloads import describe, sha256

    device = torch.device("cuda", 0)
    lengths, offsets, values = cell_inputs(torch, case, seed)
    n, b, d = int(offsets[-1]), len(lengths), case["d"]
    tdtype = torch.bfloat16 if case["dtype"] == "bf16" else torch.float32
    x = torch.from_numpy(values).to(device).to(tdtype).contiguous()
    off = torch.from_numpy(offsets).to(device)
    lens = torch.from_numpy(lengths.astype(np.int64)).to(device)
    out_rows = n if case["op"] == "softmax" else b
    program = Compiler().compile(ProgramSpec(case["op"], case["dtype"], d, "i64"), cache)
    max_len = int(lengths.max()) if b else 0
    record = {"schema": 1, "status": "running", "case": {**case, "seed": seed, "n": n, "b": b,
                                                          "lengths_sha256": describe(lengths)["lengths_sha256"],
                                                          "values_sha256": sha256(values)},
              "library_sha256": native.library_sha256(), "device": torch.cuda.get_device_name(0),
              "protocol": {"warmup": WARMUP, "timed": TIMED, "flush_bytes": int(flush.numel() * 4),
                           "timing_scope": "events around every complete call on the calling stream; inputs "
                                           "resident on the device"}, "methods": []}
    for method in METHODS:
        entry = {"method": method}
        if method.startswith("ragged"):
            select = "auto" if method.startswith("ragged-auto") else method.split("-")[1]
            hint = None if method == "ragged-auto-no-max-len" else max_len
            entry["max_len_given"] = hint is not None
            reports = []

            def call(select=select, hint=hint, reports=reports):
                out = torch.empty((out_rows, d), dtype=tdtype, device=device)
                reports[:] = [program.run(x, off, out, select=select, max_len=hint)]
                return out
        else:
            def call():
                return _torch_segment(torch, case["op"], x, off, lens, n)
        y = call()
        torch.cuda.synchronize()
        if method.startswith("ragged"):
            entry["selected"] = reports[0].selected
        try:
            entry["gate"] = gate(torch, case["op"], case["dtype"], x, offsets, y, seed)["max_fraction_of_tolerance"]
        except AssertionError as exc:
            entry.update(status="wrong", reason=str(exc))
            record["methods"].append(entry)
            log(f"[suite] {case['key']} seed {seed} {method}: WRONG ({exc})")
            continue
        del y
        for _ in range(WARMUP):
            call()
        torch.cuda.synchronize()
        entry["warm_ms"] = _stats(_time_each(torch, call, TIMED))
        entry["cold_ms"] = _stats(_time_each(torch, call, TIMED, before=lambda: flush.fill_(1.0)))
        entry.update(_graph(torch, call, lambda y: gate(torch, case["op"], case["dtype"], x, offsets, y, seed)))
        entry["status"] = "measured"
        record["methods"].append(entry)
        graph_text = (f"{entry['graph_ms']['median'] * 1e3:.1f} us" if entry["graph_ms"] else
                      entry["graph_status"])
        log(f"[suite] {case['key']} seed {seed} {method}: warm {entry['warm_ms']['median'] * 1e3:.1f} us, "
            f"cold {entry['cold_ms']['median'] * 1e3:.1f} us, graph {graph_text}")
    record["status"] = "complete"
    return record


def result_path(output: Path, key: str, seed: int) -> Path:
    return output / key / f"seed-{seed}" / "rep-0" / "results.json"


def pending(output: Path, seeds=SEEDS, pattern: str = "") -> list[tuple[dict, int]]:
    """The (case, seed) cells under `output` without a complete record (a
    missing, unreadable or unfinished results.json is measured again), of
    the cases whose key starts with one of `pattern`'s comma-separated
    prefixes (all cases when it is empty)."""
    cells = []
    for case in compare_cases():
        if pattern and not any(case["key"].startswith(prefix) for prefix in pattern.split(",")):
            continue
        for seed in seeds:
            path = result_path(output, case["key"], seed)
            try:
                if json.loads(path.read_text()).get("status") == "complete":
                    continue
            except (OSError, ValueError):
                pass
            cells.append((case, seed))
    return cells


def run_suite(output: Path, seeds=SEEDS, pattern: str = "", flush_mib: int = 1024, log=print) -> int:
    """Measure every (case, seed) of the comparison group not yet complete
    under `output`; returns how many were measured now."""
    import tempfile

    import torch

    from . import ArtifactCache

    flush = torch.empty((flush_mib << 18,), dtype=torch.float32, device="cuda")
    cache = ArtifactCache(tempfile.mkdtemp(prefix="ragged-suite-"))
    measured = 0
    for case, seed in pending(output, seeds, pattern):
        started = time.perf_counter()
        record = run_cell(torch, case, seed, flush, cache, log=log)
        record["wall_s"] = round(time.perf_counter() - started, 2)
        path = result_path(output, case["key"], seed)
        path.parent.mkdir(parents=True, exist_ok=True)
        temporary = path.with_suffix(".tmp")
        temporary.write_text(json.dumps(record, indent=1) + "\n")
        temporary.replace(path)
        measured += 1
    return measured


def _median_of(records: list[dict], method: str, field: str) -> float | None:
    """Median over seeds of one method's per-seed median of ``field``, µs."""
    values = []
    for record in records:
        entry = next((m for m in record["methods"] if m["method"] == method), None)
        if entry and entry.get("status") == "measured" and entry.get(field):
            values.append(entry[field]["median"])
    return float(np.median(values)) * 1e3 if values else None


def _selected(records: list[dict], method: str) -> str:
    ran = sorted({m.get("selected", "-") for r in records for m in r["methods"] if m["method"] == method})
    return "/".join(ran) or "-"


def _reference_us(cases: list[dict], method: str, field: str) -> float | None:
    values = [c["methods"][method][field] for c in cases
              if method in c["methods"] and c["methods"][method].get(field) is not None]
    return float(np.median(values)) * 1e3 if values else None


def summarize(output: Path, reference: Path | None = None) -> list[str]:
    """Markdown: per case, this build's medians (over seeds of per-seed
    medians of the timed calls, µs) and, with ``reference``, the
    reference's recorded medians for the same cells."""
    recorded: dict[str, list[dict]] = {}
    reference_device = None
    if reference is not None:
        data = json.loads(Path(reference).read_text())["recorded_timings"]
        reference_device = ", ".join(data["devices"])
        for case in data["cases"]:
            recorded.setdefault(f"{case['op']}-{case['dtype']}-d{case['d']}-{case['distribution']}", []).append(case)
    header = ["case", "seeds", "auto warm", "auto cold", "auto graph", "auto ran", "auto, no max_len",
              "classified", "naive", "torch-segment"]
    if recorded:
        header += ["ref auto warm", "ref auto graph", "ref fastest other warm", "ref auto / ours",
                   "ref fastest other / ours"]
    rows, device, protocol, libraries = [], None, None, set()
    wrong, uncaptured, worst = [], [], (0.0, "-")
    for case in compare_cases():
        records = [json.loads(p.read_text()) for p in sorted((output / case["key"]).glob("seed-*/rep-0/results.json"))]
        records = [r for r in records if r.get("status") == "complete"]
        if not records:
            continue
        device, protocol = records[0]["device"], records[0]["protocol"]
        libraries.update(r["library_sha256"] for r in records)
        for record in records:
            for entry in record["methods"]:
                label = f"{case['key']} seed {record['case']['seed']} {entry['method']}"
                if entry.get("status") == "wrong":
                    wrong.append(label)
                for field in ("gate", "graph_gate"):
                    if entry.get(field) is not None and entry[field] >= worst[0]:
                        worst = (entry[field], f"{label} ({field})")
                if entry.get("status") == "measured" and not entry.get("graph_ms"):
                    uncaptured.append(label)
        auto = _median_of(records, "ragged-auto", "warm_ms")
        row = [case["key"], str(len(records)), auto, _median_of(records, "ragged-auto", "cold_ms"),
               _median_of(records, "ragged-auto", "graph_ms"), _selected(records, "ragged-auto"),
               _median_of(records, "ragged-auto-no-max-len", "warm_ms"),
               _median_of(records, "ragged-classified", "warm_ms"), _median_of(records, "ragged-naive", "warm_ms"),
               _median_of(records, "torch-segment", "warm_ms")]
        if recorded:
            cases = recorded.get(case["key"], [])
            ref_auto = _reference_us(cases, "ragged-auto", "warm_ms")
            others = [(_reference_us(cases, m, "warm_ms"), m) for m in sorted({m for c in cases for m in c["methods"]})
                      if not m.startswith("ragged")]
            fastest = min((o for o in others if o[0] is not None), default=(None, "-"))
            row += [ref_auto, _reference_us(cases, "ragged-auto", "graph_ms"),
                    None if fastest[0] is None else f"{fastest[0]:.1f} ({fastest[1]})",
                    None if not (ref_auto and auto) else f"{ref_auto / auto:.2f}x",
                    None if not (fastest[0] and auto) else f"{fastest[0] / auto:.2f}x"]
        rows.append(row)
    lines = [f"This build: {device}, library sha256 {', '.join(sorted(libraries)) or '-'}; reference: "
             f"{reference_device or 'not given'}. Each time is the median over "
             f"seeds of the per-seed median of {protocol['timed'] if protocol else TIMED} complete calls, µs; "
             "`auto` is given max_len, as in the reference's compare runs; cold calls start after a "
             f"{(protocol or {}).get('flush_bytes', 0) >> 20} MiB flush.", ""]
    lines.append("| " + " | ".join(header) + " |")
    lines.append("|" + "---|" * len(header))
    for row in rows:
        lines.append("| " + " | ".join("-" if v is None else f"{v:.1f}" if isinstance(v, float) else str(v)
                                       for v in row) + " |")
    lines += ["", f"Correctness gate (the longest segment and 64 others of every output against float64): "
                  f"{len(wrong)} outputs wrong{': ' + ', '.join(wrong) if wrong else ''}; worst fraction of the "
                  f"tolerance {worst[0]:.3f} ({worst[1]}). Graph replays not measured: "
                  f"{', '.join(uncaptured) if uncaptured else 'none'}."]
    return lines


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = parser.add_subparsers(dest="command", required=True)
    r = sub.add_parser("run")
    r.add_argument("--output", type=Path, required=True)
    r.add_argument("--seeds", default=",".join(str(s) for s in SEEDS))
    r.add_argument("--cases", default="", help="only cases whose key starts with one of these (comma-separated)")
    r.add_argument("--flush-mib", type=int, default=1024, help="cold flush buffer (more than the MALL plus L2)")
    s = sub.add_parser("summarize")
    s.add_argument("output", type=Path)
    s.add_argument("--reference", type=Path)
    args = parser.parse_args(argv)
    if args.command == "run":
        started = time.perf_counter()
        count = run_suite(args.output, tuple(int(x) for x in args.seeds.split(",")), args.cases, args.flush_mib,
                          log=lambda line: print(line, flush=True))
        print(f"[suite] measured {count} cells in {time.perf_counter() - started:.1f}s", flush=True)
        return 0
    print("\n".join(summarize(args.output, args.reference)))
    return 0


if __name__ == "__main__":
    sys.exit(main())
