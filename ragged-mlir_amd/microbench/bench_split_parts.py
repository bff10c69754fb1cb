"""Split parts and block class of large sum / max calls: the library's default
(256 KiB parts, 512 KiB block class) against the runtime's rule for large
calls (parts of about N/512 rows, at most 4 MiB; block class up to N/1024
rows), and the split-part cost behind it. Not part of the library; run on one
MI355X from the repository root:

    python ragged-mlir_amd/microbench/bench_split_parts.py

Prints two Markdown tables:

* through ``program.run(select="classified")`` (µs per call, mean of 10 calls
  after one warm-up, HIP events), the default module (the rule switched off
  by a part share no call reaches) against the shipped rule, with the
  block-per-segment schedule and what ``select="auto"`` takes;
* at the native API, uniform f32 D=128 segments over 2 GiB with chosen
  (t_block, part_rows): the same segments as block items, as one split part
  each and as the default four parts.

Every output of a timed call is compared with the first variant's output of
the same input (sum within float32 reordering, max bit for bit).
"""

from __future__ import annotations

import sys
import tempfile
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

from ragged import ArtifactCache, Compiler, ProgramSpec, native, runtime  # noqa: E402
from ragged.workloads import CONFIGS, offsets_from_lengths  # noqa: E402


def _lognormal(rng, b: int, mean_rows: float, sigma: float) -> np.ndarray:
    lengths = rng.lognormal(np.log(mean_rows) - sigma * sigma / 2, sigma, b).astype(np.int64)
    return np.maximum(lengths, 1)


def _cases():
    rng = np.random.default_rng(5)
    c4 = np.diff(CONFIGS["c4"](711).offsets)
    c5 = np.diff(CONFIGS["c5"](711).offsets)
    lognormal_4g = _lognormal(rng, 2048, 4096, 1.5)
    lognormal_512m = _lognormal(rng, 256, 4096, 1.5)
    return [
        ("sum", "f32", 128, "one 2^22-row segment", np.array([1 << 22])),
        ("sum", "f32", 128, "64 segments of 2^16 rows", np.full(64, 1 << 16)),
        ("max", "bf16", 128, "four 2^20-row segments", np.full(4, 1 << 20)),
        ("sum", "bf16", 128, "C5's lengths", c5),
        ("sum", "f32", 128, "C4's lengths", c4),
        ("sum", "f32", 128, "lognormal B=2048 mean 4096 sigma 1.5", lognormal_4g),
        ("sum", "f32", 128, "4096 x 2048 rows", np.full(4096, 2048)),
        ("max", "bf16", 64, "C5's lengths", c5),
        ("sum", "f32", 128, "lognormal B=256 mean 4096 sigma 1.5", lognormal_512m),
        ("sum", "f32", 128, "three 2^18-row segments", np.full(3, 1 << 18)),
        ("sum", "f32", 128, "384 x 2048 rows", np.full(384, 2048)),
    ]


def _timed(torch, fn, calls: int = 10) -> float:
    fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(calls):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / calls * 1000


def _same(torch, op: str, a, b) -> bool:
    if op == "max":
        return bool(torch.equal(a, b))
    return bool(torch.allclose(a.float(), b.float(), rtol=2e-2, atol=1.0))


def run_program_table(torch) -> None:
    cache = ArtifactCache(tempfile.mkdtemp(prefix="ragged-split-parts-"))
    print("| call | dtype, D | rows (size) | default µs | shipped µs (part, block rows) | naive µs | auto |")
    print("|---|---|---|---:|---:|---:|---|")
    shipped_share = runtime.BIG_PART_SHARE
    for op, dtype, d, name, lengths in _cases():
        program = Compiler().compile(ProgramSpec(op, dtype, d, "i64"), cache)
        offsets = torch.from_numpy(offsets_from_lengths(np.asarray(lengths, dtype=np.int64), "i64")).cuda()
        n, b, max_len = int(offsets[-1]), len(lengths), int(np.max(lengths))
        tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
        x = torch.randn((n, d), device="cuda").to(tdtype)
        out = torch.empty((b, d), dtype=tdtype, device="cuda")
        try:
            runtime.BIG_PART_SHARE = 1 << 62          # no call reaches twice the default part
            default_us = _timed(torch, lambda: program.run(x, offsets, out, select="classified", max_len=max_len))
            reference = out.clone()
            runtime.BIG_PART_SHARE = shipped_share
            report = program.run(x, offsets, out, select="classified", max_len=max_len)
            shipped_us = _timed(torch, lambda: program.run(x, offsets, out, select="classified", max_len=max_len))
            assert _same(torch, op, out, reference), f"{name}: shipped output differs"
            naive_us = _timed(torch, lambda: program.run(x, offsets, out, select="naive"))
            assert _same(torch, op, out, reference), f"{name}: naive output differs"
            chosen = program.run(x, offsets, out, max_len=max_len).selected
        finally:
            runtime.BIG_PART_SHARE = shipped_share
        size = n * d * (2 if dtype == "bf16" else 4)
        part = report.selection.get("part_rows")
        rule = f"{part}, {report.thresholds[1]}" if part else "default module"
        print(f"| {op}, {name} | {dtype}, {d} | {n:,} ({size / 2**30:.2f} GiB) | {default_us:,.1f} | "
              f"{shipped_us:,.1f} ({rule}) | {naive_us:,.1f} | {chosen} |", flush=True)
        del x, out, offsets
        torch.cuda.empty_cache()


def run_native_table(torch) -> None:
    print()
    print("| segment rows | segments | t_block | part_rows | class of each segment | µs | / naive |")
    print("|---:|---:|---:|---:|---|---:|---:|")
    x = torch.randn((1 << 22, 128), device="cuda")
    naive = native.NativeModule(0, native.make_spec("sum", "f32", "i64", 128))
    stream = torch.cuda.current_stream().cuda_stream

    def call(module, plan, offsets, out):
        workspace = torch.zeros((max(1, int(plan.workspace_bytes)),), dtype=torch.uint8, device="cuda")
        args = (plan, x.data_ptr(), offsets.data_ptr(), out.data_ptr(), None, workspace.data_ptr(),
                int(plan.workspace_bytes), stream)
        return _timed(torch, lambda: module.run(*args))

    for rows in (2048, 4096):
        b = (1 << 22) // rows
        offsets_np = offsets_from_lengths(np.full(b, rows, dtype=np.int64), "i64")
        offsets = torch.from_numpy(offsets_np).cuda()
        out = torch.empty((b, 128), device="cuda")
        naive_us = call(naive, naive.plan(1 << 22, b, "naive"), offsets, out)
        reference = out.clone()
        for t_block, part_rows, what in ((-1, -1, "split, default parts"), (1024, rows, "split, one part"),
                                         (rows, 512, "block")):
            module = native.NativeModule(0, native.make_spec("sum", "f32", "i64", 128, t_block=t_block,
                                                             part_rows=part_rows))
            plan = module.plan(1 << 22, b, "classified")
            us = call(module, plan, offsets, out)
            assert _same(torch, "sum", out, reference), f"{rows} rows, {what}: output differs"
            print(f"| {rows} | {b} | {int(plan.t_block)} | {int(plan.part_rows)} | {what} | {us:,.1f} | "
                  f"{us / naive_us:.2f} |", flush=True)
        print(f"| {rows} | {b} | | | naive (one workgroup per segment) | {naive_us:,.1f} | 1.00 |", flush=True)
        del offsets, out


def main() -> int:
    import torch

    if not torch.cuda.is_available():
        print("bench_split_parts: needs a ROCm GPU")
        return 2
    print(f"library sha256 {native.library_sha256()}")
    print()
    run_program_table(torch)
    run_native_table(torch)
    return 0


if __name__ == "__main__":
    sys.exit(main())
