#!/usr/bin/env python3
"""Benchmark of the hot path: one call of ``program.run`` = one step.

Default workload: C5, the long-tail bf16 D=128 segmented softmax (8,192
segments, 4,194,304 rows, longest 200,000, i64 offsets, max_len passed) on
one MI355X, inputs resident in HBM. Prints ONE JSON line:

* ``value``: achieved GB/s of algorithmic bytes (read values + offsets once,
  write the output once) per call; ``us_per_call`` and ``pct_of_peak`` beside it.
* ``roofline``: the dominant kernel's algorithmic bytes / its average
  duration (HIP events recorded around every launch inside the timed calls,
  on the stream the kernels run on), against the 8 TB/s HBM peak.
* ``cpu_baseline``: the fastest of the CPU baselines timed on this host on
  the full input of the same workload: the reference's PyTorch CPU baseline
  (baselines/torch_reference.py:12-16; softmax composed from
  torch.segment_reduce) at one thread and at the process's core share. The
  float64 NumPy oracle on one thread is listed beside them, timed on a
  prefix of segments holding 1/16 of the rows and scaled to a full call (a
  whole C5 call takes it about 90 s); every variant says which it is.

Every measured configuration first passes the oracle (max bit-exact,
sum/softmax within tolerance) on a sample of its segments.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config c5] [--op OP] [--seeds S,..]
                    [--cold [write|read]] [--all] [--details FILE] [--timeline FILE] [--no-cpu]

``--timeline`` records one further call of every register-resident softmax
measured with its item trace on and writes the summary: per item class the
phase durations, workgroups live and merging over the call, and where each
chunk class's merge time goes (ragged.profiling.item_timeline).
"""
from __future__ import annotations

import argparse
import json
import os
from pathlib import Path
import sys
import tempfile
import time

ROOT = Path(__file__).resolve().parent
for _path in (ROOT, ROOT / "ragged-mlir_amd"):
    if str(_path) not in sys.path:
        sys.path.insert(0, str(_path))

import numpy as np  # noqa: E402

PEAK_GBPS = 8000.0
METRIC = "µs/call + achieved HBM GB/s (% of peak), long-tail bf16 D=128 softmax"


def log(message: str) -> None:
    print(message, file=sys.stderr, flush=True)


def sample_segments(lengths: np.ndarray, count: int, seed: int) -> np.ndarray:
    """Segment ids for the oracle gate: the longest, the shortest, empties and
    a random spread."""
    rng = np.random.default_rng(seed)
    b = len(lengths)
    picks = {int(np.argmax(lengths)), int(np.argmin(lengths)), 0, b - 1}
    picks.update(int(i) for i in rng.choice(b, size=min(b, count), replace=False))
    return np.array(sorted(picks), dtype=np.int64)


def gather_segments(values, offsets, ids):
    """Rows of the chosen segments, packed, with their own offsets."""
    lo, hi = offsets[ids].astype(np.int64), offsets[ids + 1].astype(np.int64)
    rows = np.concatenate([np.arange(a, b) for a, b in zip(lo, hi)]) if len(ids) else np.zeros(0, np.int64)
    sub_offsets = np.concatenate([[0], np.cumsum(hi - lo)]).astype(np.int64)
    return rows, sub_offsets


def oracle_gate(op, dtype, values_f32, offsets, out_device, torch, *, max_rows=600_000, seed=0):
    """Check a sample of segments (independent of each other) against the
    float64 oracle. Returns the oracle's error statistics."""
    import oracle
    lengths = np.diff(offsets.astype(np.int64))
    ids = sample_segments(lengths, 64, seed)
    # Keep the sample bounded: drop the largest picks until it fits.
    while lengths[ids].sum() > max_rows and len(ids) > 1:
        ids = np.delete(ids, int(np.argmax(lengths[ids])))
    rows, sub_offsets = gather_segments(values_f32, offsets, ids)
    inputs = values_f32[rows]
    if dtype == "bf16":
        inputs = oracle.quantize_bf16(inputs)
    if op == "softmax":
        actual = out_device[torch.from_numpy(rows).to(out_device.device)].float().cpu().numpy()
    else:
        actual = out_device[torch.from_numpy(ids).to(out_device.device)].float().cpu().numpy()
    stats = oracle.assert_matches(actual.astype(np.float64), inputs, sub_offsets, operation=op, input_dtype=dtype)
    if op == "max":
        expected = oracle.segment_max(inputs, sub_offsets).astype(np.float32)
        if dtype == "bf16":
            expected = oracle.quantize_bf16(expected)
        nan = np.isnan(expected)
        assert np.array_equal(nan, np.isnan(actual)) and np.array_equal(actual[~nan], expected[~nan])
    stats["segments_checked"] = int(len(ids))
    stats["rows_checked"] = int(len(rows))
    return stats


def cpu_model() -> str:
    """The host CPU as lscpu reports it (model name, sockets x cores per
    socket x threads per core), else the model name in /proc/cpuinfo."""
    import subprocess
    try:
        text = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        fields = dict(line.split(":", 1) for line in text.splitlines() if ":" in line)
        fields = {key.strip(): value.strip() for key, value in fields.items()}
        if fields.get("Model name"):
            shape = "/".join(fields.get(key, "?") for key in ("Socket(s)", "Core(s) per socket", "Thread(s) per core"))
            return f"{fields['Model name']} (lscpu; sockets/cores per socket/threads per core {shape}, " \
                   f"{fields.get('CPU(s)', '?')} CPUs)"
    except (OSError, subprocess.SubprocessError, ValueError):
        pass
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_sample(offsets, fraction: int = 16):
    """A prefix of segments holding about 1/``fraction`` of the rows:
    (segments, sample offsets as i64, rows)."""
    lengths = np.diff(offsets.astype(np.int64))
    n = int(offsets[-1])
    cut = int(np.searchsorted(np.cumsum(lengths), max(1, n // fraction))) + 1
    cut = min(cut, len(lengths))
    sample_offsets = offsets[:cut + 1].astype(np.int64)
    return cut, sample_offsets, int(sample_offsets[-1])


def _median_time(function, target_seconds: float) -> tuple[float, int]:
    """Median wall time of ``function()`` over at least 5 runs (1 at least
    when one run exceeds the budget), after one warm-up."""
    function()
    times, started = [], time.perf_counter()
    while len(times) < 5 and (time.perf_counter() - started) < target_seconds or len(times) < 1:
        t0 = time.perf_counter()
        function()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline_oracle(op, dtype, values_f32, offsets, *, target_seconds=15.0):
    """The float64 NumPy oracle (single thread) on a prefix of segments that
    holds about 1/16 of the rows, scaled to µs per full call."""
    import oracle
    n = int(offsets[-1])
    cut, sample_offsets, rows = cpu_sample(offsets)
    inputs = values_f32[:rows]
    if dtype == "bf16":
        inputs = oracle.quantize_bf16(inputs)
    function = {"sum": oracle.segment_sum, "max": oracle.segment_max, "softmax": oracle.segment_softmax}[op]
    seconds, runs = _median_time(lambda: function(inputs, sample_offsets), target_seconds)
    per_call_us = seconds * 1e6 * (n / max(rows, 1))
    return {"per_call_us": round(per_call_us, 1), "cores": 1, "kind": "port", "impl": "oracle-float64-numpy",
            "full_input": False,
            "sample": f"float64 NumPy oracle ({op}, one thread) on the first {cut} of {len(offsets) - 1} segments "
                      f"({rows} of {n} rows), median of {runs} runs after one warm-up, scaled by N/rows"}


def torch_cpu_reference(values, offsets, op):
    """The reference's PyTorch baseline on the CPU (baselines/torch_reference.py:
    12-16: torch.segment_reduce on f32, bf16 promoted and converted back), and
    for softmax the same steps composed: segment max, repeat_interleave,
    exp, segment sum, divide."""
    import torch
    work = values.float() if values.dtype == torch.bfloat16 else values
    if op in ("sum", "max"):
        return torch.segment_reduce(work, op, offsets=offsets, axis=0).to(values.dtype)
    lengths = offsets[1:] - offsets[:-1]
    maxima = torch.segment_reduce(work, "max", offsets=offsets, axis=0)
    weights = torch.exp(work - torch.repeat_interleave(maxima, lengths, dim=0))
    sums = torch.segment_reduce(weights, "sum", offsets=offsets, axis=0)
    return (weights / torch.repeat_interleave(sums, lengths, dim=0)).to(values.dtype)


def cpu_baseline_torch(op, dtype, values_f32, offsets, threads: int, *, target_seconds=15.0, full: bool = True):
    """torch_cpu_reference at ``threads`` intra-op threads on the full input
    (one warm-up, then the median of runs within the time budget, at least
    one), or with ``full`` False on the 1/16 prefix of segments, scaled to µs
    per full call."""
    import torch
    n = int(offsets[-1])
    if full:
        cut, sample_offsets, rows = len(offsets) - 1, offsets.astype(np.int64), n
    else:
        cut, sample_offsets, rows = cpu_sample(offsets)
    values = torch.from_numpy(np.ascontiguousarray(values_f32[:rows]))
    if dtype == "bf16":
        values = values.to(torch.bfloat16)
    off = torch.from_numpy(sample_offsets)
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        seconds, runs = _median_time(lambda: torch_cpu_reference(values, off, op), target_seconds)
    finally:
        torch.set_num_threads(previous)
    per_call_us = seconds * 1e6 * (n / max(rows, 1))
    what = (f"the full input ({len(offsets) - 1} segments, {n} rows)" if full else
            f"the first {cut} of {len(offsets) - 1} segments ({rows} of {n} rows), scaled by N/rows")
    return {"per_call_us": round(per_call_us, 1), "cores": threads, "kind": "port", "full_input": full,
            "impl": f"torch-{torch.__version__}-cpu",
            "sample": f"torch CPU reference ({op}; baselines/torch_reference.py restated, softmax composed) at "
                      f"{threads} threads on {what}, median of {runs} runs after one warm-up"}


def cpu_baselines(op, dtype, values_f32, offsets, algorithmic_bytes: int) -> list[dict]:
    """Every CPU baseline of one workload, each with its GB/s: the torch
    reference on the full input at one thread and at every core this process
    may use (its affinity, capped by OMP_NUM_THREADS: a GPU box shares its
    host between GPUs), and the oracle on one thread on a prefix sample."""
    cores = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    threads_all = min(cores, share) if share > 0 else cores
    variants = [cpu_baseline_oracle(op, dtype, values_f32, offsets)]
    for threads in sorted({1, threads_all}):
        variants.append(cpu_baseline_torch(op, dtype, values_f32, offsets, threads))
    model = cpu_model()
    for variant in variants:
        variant["value"] = round(algorithmic_bytes / (variant["per_call_us"] * 1e-6) / 1e9, 3)
        variant["unit"] = "GB/s"
        variant["cpu_model"] = model
        variant["affinity_cores"] = cores
    return variants


def role_bytes(role: str, op: str, lengths: np.ndarray, d: int, element: int, t_wave: int, t_block: int,
               offset_bytes: int = 8) -> int:
    """Algorithmic bytes of the rows one kernel role owns. The
    register-resident softmax ("fused") reads and writes every row once: the
    segments longer than t_wave held in registers, then the wave class in
    batches (a re-read of a chunk that stopped waiting is not algorithmic);
    "classify" reads the offsets."""
    if role == "fused":
        return 2 * int(lengths.sum()) * d * element
    if role == "classify":
        return (len(lengths) + 1) * offset_bytes
    if role == "worker":
        # The classified worker reads every row once and writes every
        # reduction result, or every softmax row (split segments' rows after
        # a re-read that is not algorithmic).
        if op == "softmax":
            return 2 * int(lengths.sum()) * d * element
        return (int(lengths.sum()) + len(lengths)) * d * element
    if role == "naive":
        rows = lengths
    elif role == "wave":
        rows = lengths[lengths <= t_wave]
    elif role == "block":
        rows = lengths[(lengths > t_wave) & (lengths <= t_block)]
    elif role in ("split_partial", "split_normalize", "split_combine"):
        rows = lengths[lengths > t_block]
    else:
        return 0
    n_rows, segs = int(rows.sum()), int(len(rows))
    if op == "softmax":
        if role == "split_partial":
            return n_rows * d * element          # reads the rows once
        if role == "split_normalize":
            return n_rows * d * element          # writes the rows once (its re-read is not algorithmic)
        if role == "split_combine":
            return 0
        return 2 * n_rows * d * element
    if role == "split_combine":
        return segs * d * element                # writes the outputs
    return n_rows * d * element + (0 if role == "split_partial" else segs * d * element)


def run_config(name: str, args, torch, cache, seed: int = 711) -> list[dict]:
    from ragged import Compiler, ProgramSpec
    from ragged.workloads import CONFIGS, algorithmic_bytes
    from ragged.runtime import _modules

    t0 = time.perf_counter()
    workload = CONFIGS[name](seed)
    log(f"[bench] {workload.name}: N={workload.n} B={workload.b} D={workload.d} generated in "
        f"{time.perf_counter() - t0:.1f}s")
    device = torch.device("cuda", 0)
    tdtype = torch.bfloat16 if workload.dtype == "bf16" else torch.float32
    element = 2 if workload.dtype == "bf16" else 4
    offset_bytes = 4 if workload.offsets_dtype == "i32" else 8
    x = torch.from_numpy(workload.values).to(device).to(tdtype).contiguous()
    off = torch.from_numpy(workload.offsets).to(device)
    lengths = np.diff(workload.offsets.astype(np.int64))
    max_len = workload.max_len if workload.pass_max_len else None
    results = []
    for op in workload.ops:
        if args.op and op != args.op:
            continue
        program = Compiler().compile(ProgramSpec(op, workload.dtype, workload.d, workload.offsets_dtype), cache)
        rows = workload.n if op == "softmax" else workload.b
        out = torch.empty((rows, workload.d), dtype=tdtype, device=device)
        selects = ["auto", "classified", "naive"] if args.all else ["auto"]
        for select in selects:
            report = program.run(x, off, out, select=select, max_len=max_len)
            torch.cuda.synchronize()
            stats = oracle_gate(op, workload.dtype, workload.values, workload.offsets, out, torch, seed=seed)
            log(f"[bench] {workload.name} {op} {select} ({report.selected}): oracle ok, "
                f"max_fraction_of_tolerance={stats['max_fraction_of_tolerance']:.3g} on "
                f"{stats['segments_checked']} segments")
            for _ in range(args.warmup):
                program.run(x, off, out, select=select, max_len=max_len)
            torch.cuda.synchronize()
            # The timed region: K calls bracketed by events on the current
            # stream (the one the kernels run on). A second pass of K calls
            # records a HIP event around every launch (per-kernel times);
            # those events add gaps between launches, so that pass is not
            # the per-call figure.
            chosen = program.naive if report.selected == "naive" else program
            module = _modules[(0, chosen._digest)]
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            # Cold cache: before every call, overwrite (write flush) or read
            # (read flush) 1 GiB, 4x the 256 MiB Infinity Cache plus L2.
            flush = torch.empty((1 << 28,), dtype=torch.float32, device=device).fill_(1) if args.cold else None

            def evict():
                if args.cold == "read":
                    flush.sum()
                else:
                    flush.fill_(1)

            def timed_calls() -> float:
                if args.cold:
                    total_ms, host = 0.0, []
                    for _ in range(args.steps):
                        evict()
                        start.record()
                        t_host = time.perf_counter()
                        program.run(x, off, out, select=select, max_len=max_len)
                        host.append((time.perf_counter() - t_host) * 1e6)
                        end.record()
                        torch.cuda.synchronize()
                        total_ms += start.elapsed_time(end)
                    host_us.append([round(float(np.median(host)), 1), round(float(np.max(host)), 1)])
                    return total_ms / args.steps
                torch.cuda.synchronize()
                host = []
                start.record()
                for _ in range(args.steps):
                    t_host = time.perf_counter()
                    program.run(x, off, out, select=select, max_len=max_len)
                    host.append((time.perf_counter() - t_host) * 1e6)
                end.record()
                torch.cuda.synchronize()
                host_us.append([round(float(np.median(host)), 1), round(float(np.max(host)), 1)])
                return start.elapsed_time(end) / args.steps

            host_us = []     # [median, max] host time of one run() call per timed pass
            ms = timed_calls()
            module.profile_start(args.steps)
            timed_calls()
            profile = module.profile_stop()
            plan = next(v for k, v in chosen._plans.items() if k[0] is module and k[1:3] == (workload.n, workload.b))
            total_bytes = algorithmic_bytes(op, workload.n, workload.b, workload.d, element, offset_bytes)
            kernels = {}
            for role, entry in profile["roles"].items():
                avg = entry["ms"] / max(entry["launches"], 1)
                nbytes = role_bytes(role, op, lengths, workload.d, element, int(plan.t_wave), int(plan.t_block),
                                    offset_bytes)
                kernels[role] = {"avg_ms": round(avg, 5), "bytes": nbytes,
                                 "gbps": round(nbytes / (avg * 1e-3) / 1e9, 1) if avg > 0 else None}
            dominant = max(kernels, key=lambda r: kernels[r]["avg_ms"]) if kernels else None
            gpu_ms = profile["call_ms"] / max(profile["calls"], 1)
            gbps = total_bytes / (ms * 1e-3) / 1e9
            results.append({
                "workload": workload.name, "op": op, "select": select, "selected": report.selected,
                "us_per_call": round(ms * 1e3, 2), "gbps": round(gbps, 1), "pct_of_peak": round(100 * gbps / PEAK_GBPS, 2),
                "gpu_us_per_call": round(gpu_ms * 1e3, 2), "host_us_per_run": host_us[0] if host_us else None,
                "algorithmic_bytes": total_bytes, "kernels": kernels,
                "dominant": dominant, "cold": args.cold or False, "seed": seed, "oracle": stats,
                "n": workload.n, "b": workload.b, "d": workload.d, "dtype": workload.dtype,
                "offsets_dtype": workload.offsets_dtype, "max_len": workload.max_len,
                "kernel_names": list(report.kernel_names), "grids": [list(g) for g in report.grids]})
            if args.timeline and plan.fused:
                results[-1]["timeline"] = item_trace(torch, program, module, plan, x, off, out, select, max_len)
                split = {name: entry.get("merge_split") for name, entry in results[-1]["timeline"]["classes"].items()}
                log(f"[bench] {workload.name} {op} {select}: item timeline merge split {json.dumps(split)}")
            log(f"[bench] {workload.name} {op} {select}: host run() median/max us {host_us[0] if host_us else None}")
            log(f"[bench] {workload.name} {op} {select}: {ms * 1e3:.1f} us/call, {gbps:.0f} GB/s "
                f"({100 * gbps / PEAK_GBPS:.1f}% of peak); kernels {json.dumps(kernels)}")
    return results, workload


def item_trace(torch, program, module, plan, x, off, out, select, max_len) -> dict:
    """One call with the register-resident softmax's item trace on
    (rg_module_set_trace), summarised by ragged.profiling.item_timeline."""
    from ragged import native, profiling
    records = int(plan.items_cap + plan.b)
    trace = torch.zeros((records, 8), dtype=torch.int64, device=x.device)
    torch.cuda.synchronize()
    module.set_trace(trace.data_ptr(), records)
    try:
        program.run(x, off, out, select=select, max_len=max_len)
        torch.cuda.synchronize()
    finally:
        module.set_trace(None)
    return profiling.item_timeline(trace.cpu().numpy(), native.device_clock_khz(x.device.index or 0),
                                   int(plan.part_rows))


def copy_probe(torch, mib: int, steps: int) -> int:
    """A plain device-to-device copy of known size: under rocprofv3 --pmc its
    FETCH_SIZE and WRITE_SIZE per dispatch give the counters' byte scale."""
    n = mib << 20
    src = torch.empty(n, dtype=torch.uint8, device="cuda").fill_(7)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(max(steps, 1)):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / max(steps, 1)
    print(json.dumps({"copy_bytes": n, "ms": round(ms, 4), "gbps": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)
    return 0


def measured_traffic(workload: str, role: str | None):
    """HBM bytes per launch of ``role``'s kernel from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of this workload, if it was measured with
    the library that is loaded now (None otherwise)."""
    if not role:
        return None
    # Summaries are named for the kernel role, the workload and its shape:
    # profiles/<role>_<workload>_<shape>_traffic.json.
    paths = sorted((ROOT / "profiles").glob(f"{role}_{workload}_*traffic.json"))
    if len(paths) != 1:
        return None
    path = paths[0]
    from ragged import native
    data = json.loads(path.read_text())
    if data.get("library_sha256") != native.library_sha256():
        log(f"[bench] {path.name} was measured with another library build; traffic left null")
        return None
    return {"bytes": int(round(data["bytes"])), "source": f"profiles/{path.name}"}


def main(argv=None) -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--config", default="c5", choices=["c1", "c2", "c3", "c4", "c5"])
    parser.add_argument("--cold", nargs="?", const="write", choices=["write", "read"],
                        help="flush 1 GiB (> MALL + L2) before every call, by overwriting it (write, the "
                             "default) or by reading it (read)")
    parser.add_argument("--seeds", help="comma-separated seeds (default: 711, 712, 713 for c1, else 711); "
                                        "the line reports the median seed")
    parser.add_argument("--op", choices=["sum", "max", "softmax"],
                        help="measure only this op of the workload (c2 holds sum and max)")
    parser.add_argument("--all", action="store_true", help="also measure forced classified and naive schedules")
    parser.add_argument("--details", type=Path, help="write every measured record as JSON to this file")
    parser.add_argument("--timeline", type=Path,
                        help="record one call's item trace of the register-resident softmax and write its summary "
                             "(ragged.profiling.item_timeline) as JSON to this file")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--copy-probe", type=int, metavar="MIB",
                        help="instead: time a plain device copy of MIB MiB (--steps times), the known-size "
                             "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 2
    if args.copy_probe:
        return copy_probe(torch, args.copy_probe, args.steps)
    from ragged import ArtifactCache
    seeds = ([int(x) for x in args.seeds.split(",")] if args.seeds
             else [711, 712, 713] if args.config == "c1" else [711])
    with tempfile.TemporaryDirectory(prefix="ragged-bench-") as directory:
        cache = ArtifactCache(directory)
        records, autos = [], []
        for seed in seeds:
            seed_records, workload = run_config(args.config, args, torch, cache, seed=seed)
            records += seed_records
            autos.append((next(r for r in seed_records if r["select"] == "auto"), workload))
        # The line reports the seed of median time (the only one for one seed).
        autos.sort(key=lambda pair: pair[0]["us_per_call"])
        headline, workload = autos[len(autos) // 2]
        baseline, variants = None, []
        if not args.no_cpu:
            variants = cpu_baselines(headline["op"], workload.dtype, workload.values, workload.offsets,
                                     headline["algorithmic_bytes"])
            best = max((v for v in variants if v["full_input"]), key=lambda v: v["value"])
            baseline = {key: best[key] for key in ("value", "unit", "cores", "kind", "sample", "per_call_us",
                                                   "impl", "cpu_model", "affinity_cores")}
            baseline["variants"] = [{key: v[key] for key in ("impl", "cores", "value", "per_call_us", "full_input")}
                                    for v in variants]
            log(f"[bench] cpu baselines: {json.dumps(variants)}")
    dominant = headline["dominant"]
    kernel = headline["kernels"].get(dominant, {})
    measured = measured_traffic(headline["workload"], dominant)
    roofline = {"bound": "hbm", "kernel": dominant, "achieved": kernel.get("gbps"), "peak": PEAK_GBPS,
                "unit": "GB/s", "frac": round(kernel["gbps"] / PEAK_GBPS, 4) if kernel.get("gbps") else None,
                "traffic": measured.get("bytes") if measured else None,
                "traffic_source": measured.get("source") if measured else None,
                "avg_ms": kernel.get("avg_ms"), "bytes_per_launch": kernel.get("bytes"),
                "call_gbps_gpu_time": round(headline["algorithmic_bytes"] / (headline["gpu_us_per_call"] * 1e-6) / 1e9, 1)}
    line = {
        "metric": METRIC, "value": headline["gbps"], "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(headline["us_per_call"] / 1e3, 5),
        "us_per_call": headline["us_per_call"], "pct_of_peak": headline["pct_of_peak"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": headline["dtype"], "data": "synthetic (seeded NumPy generators, resident in HBM)",
        "config": {"workload": headline["workload"], "op": headline["op"], "n": headline["n"], "b": headline["b"],
                   "d": headline["d"], "offsets": headline["offsets_dtype"], "max_len": headline["max_len"],
                   "schedule": headline["selected"],
                   "cache": f"cold ({args.cold} flush)" if args.cold else "warm",
                   "seeds": seeds, "seed": headline["seed"], "parallelism": "single GPU"},
        "roofline": roofline, "cpu_baseline": baseline,
    }
    if args.details:
        args.details.parent.mkdir(parents=True, exist_ok=True)
        args.details.write_text(json.dumps({"line": line, "records": records, "cpu_baselines": variants},
                                           indent=1) + "\n")
    if args.timeline:
        args.timeline.parent.mkdir(parents=True, exist_ok=True)
        args.timeline.write_text(json.dumps([{key: r[key] for key in ("workload", "op", "select", "seed", "timeline")}
                                             for r in records if "timeline" in r], indent=1) + "\n")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
