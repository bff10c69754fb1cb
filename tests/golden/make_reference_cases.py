"""Write tests/golden/reference_cases.json from the reference's recorded runs.

The reference (simon-jd/ragged-mlir) records, for every benchmark cell,
the generator arguments and the sha256 of the generated lengths, offsets and
values (``bench/run.py:51-65`` -> ``results/**/results.json`` "case" and
"command"). Those records are data; this script copies the fields needed to
pin ``ragged.workloads`` (the restated generators) into a small fixture. It
also copies, for the comparison runs of seed 711
(``results/bench/runs/compare/*/seed-711/rep-0``), the oracle statistics the
reference recorded for every measured method (``methods[].oracle``:
max_abs_error, max_fraction_of_tolerance), so the GPU tests can regenerate
those inputs and compare this build's error with the reference's; and, for
every seed of those runs, each method's recorded median times (warm, cold,
graph replay) on the reference's GPU, which ``python -m ragged.suite
summarize`` sets beside this build's. It reads JSON only and runs no
reference code.

Usage: python tests/golden/make_reference_cases.py [/root/reference]
"""
from __future__ import annotations

import json
from pathlib import Path
import sys


def _argument(command: list[str], flag: str, default=None):
    if flag in command:
        return command[command.index(flag) + 1]
    return default


def recorded_oracle(reference: Path) -> list[dict]:
    """Per comparison case (seed 711, first repetition): the op and generator
    arguments, and each measured method's recorded oracle statistics."""
    records = []
    for path in sorted((reference / "results" / "bench" / "runs" / "compare").glob("*/seed-711/rep-0/results.json")):
        record = json.loads(path.read_text())
        case, command = record["case"], record["command"]
        methods = {}
        for method in record["methods"]:
            stats = method.get("oracle")
            if method.get("status", "measured") == "measured" and isinstance(stats, dict):
                methods[method["method"]] = {key: stats[key] for key in
                                             ("max_abs_error", "max_fraction_of_tolerance", "finite_values",
                                              "nan_values")}
        total = _argument(command, "--total-elements")
        records.append({
            "op": case["op"], "distribution": case["distribution"], "segments": int(case["segments"]),
            "total_elements": int(total) if total is not None else None,
            "mean_length": int(_argument(command, "--mean-length", 64)), "seed": int(case["seed"]),
            "d": int(case["D"]), "dtype": case["dtype"], "offsets_dtype": case["offsets_dtype"],
            "lengths_sha256": case["lengths_sha256"], "values_sha256": case["values_sha256"],
            "methods": methods, "source": str(path.relative_to(reference)),
        })
    return records


def _median(block) -> float | None:
    return float(block["median"]) if isinstance(block, dict) and "median" in block else None


def recorded_timings(reference: Path) -> dict:
    """Per comparison case and seed (first repetition): the generator
    arguments and each measured method's median complete-call time in ms,
    warm, after a cache flush, and as a replayed graph (results.json
    "complete_call_cuda_event_ms", "cold_l2", "cuda_graph"), with whether
    the reference's ragged methods were given max_len, and the device."""
    records, devices = [], set()
    for path in sorted((reference / "results" / "bench" / "runs" / "compare").glob("*/seed-*/rep-0/results.json")):
        record = json.loads(path.read_text())
        case, command = record["case"], record["command"]
        if record.get("status") != "complete":
            continue
        device = record.get("device")
        devices.add(device.get("name") if isinstance(device, dict) else str(device))
        methods = {}
        for method in record["methods"]:
            if method.get("status") != "measured":
                continue
            cold, graph = method.get("cold_l2") or {}, method.get("cuda_graph") or {}
            methods[method["method"]] = {
                "warm_ms": _median(method.get("complete_call_cuda_event_ms")),
                "cold_ms": _median(cold.get("complete_call_cuda_event_ms")),
                "graph_ms": _median(graph.get("replay_cuda_event_ms")) if graph.get("status") == "measured" else None,
                "max_len_given": method.get("max_len_given")}
        total = _argument(command, "--total-elements")
        records.append({
            "op": case["op"], "distribution": case["distribution"], "segments": int(case["segments"]),
            "total_elements": int(total) if total is not None else None,
            "mean_length": int(_argument(command, "--mean-length", 64)), "seed": int(case["seed"]),
            "d": int(case["D"]), "dtype": case["dtype"], "offsets_dtype": case["offsets_dtype"],
            "lengths_sha256": case["lengths_sha256"], "values_sha256": case["values_sha256"],
            "methods": methods, "source": str(path.relative_to(reference)),
        })
    return {"devices": sorted(devices), "cases": records}


def main(reference: Path) -> int:
    cases: dict[tuple, dict] = {}
    for path in sorted((reference / "results").rglob("results.json")):
        try:
            record = json.loads(path.read_text())
        except (OSError, ValueError):
            continue
        case, command = record.get("case"), record.get("command")
        if not isinstance(case, dict) or not isinstance(command, list):
            continue
        total = _argument(command, "--total-elements")
        entry = {
            "distribution": case["distribution"],
            "segments": int(case["segments"]),
            "total_elements": int(total) if total is not None else None,
            "mean_length": int(_argument(command, "--mean-length", 64)),
            "seed": int(case["seed"]),
            "d": int(case["D"]),
            "dtype": case["dtype"],
            "offsets_dtype": case["offsets_dtype"],
            "elements": int(case["elements"]),
            "max_length": case["max_length"],
            "histogram_counts": case["histogram_counts"],
            "lengths_sha256": case["lengths_sha256"],
            "offsets_sha256": case["offsets_sha256"],
            "values_sha256": case["values_sha256"],
            "source": str(path.relative_to(reference)),
        }
        key = (entry["distribution"], entry["segments"], entry["total_elements"], entry["mean_length"],
               entry["seed"], entry["d"], entry["dtype"], entry["offsets_dtype"])
        cases.setdefault(key, entry)
    # Keep every distinct generator case whose values are cheap to regenerate.
    chosen = sorted(cases.values(), key=lambda e: (e["elements"] * e["d"], e["source"]))
    small = [e for e in chosen if e["elements"] * e["d"] <= 2**25]
    recorded = recorded_oracle(reference)
    timings = recorded_timings(reference)
    out = Path(__file__).with_name("reference_cases.json")
    out.write_text(json.dumps({"cases": small, "total_distinct": len(chosen), "recorded_oracle": recorded,
                               "recorded_timings": timings}, indent=1) + "\n")
    print(f"wrote {len(small)} of {len(chosen)} distinct cases, {len(recorded)} recorded oracle statistics and "
          f"{len(timings['cases'])} recorded timings ({timings['devices']}) to {out}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")))
