"""GPU parity on the five benchmark configurations at full size.

Each configuration of ``ragged.workloads.CONFIGS`` (C1-C5) is generated
exactly as the benchmark generates it and run through ``program.run`` with
every schedule: ``auto`` as the benchmark calls it (``max_len`` only where
the configuration passes it), ``auto`` given ``max_len``, and the forced
``classified`` and ``naive`` schedules. The reference gates every measured
cell on its oracle the same way (docs/benchmarking.md:56-59) and runs a
workload matrix on its GPU suite (test/gpu/test_workload_matrix.py:24-50).

* C1 (three seeds), C2, C3 and C4 are checked against the full float64
  oracle: the reference's tolerance, the build's stricter one, and max bit
  for bit (C2 injects NaN and -inf into 0.1% of the entries each).
* C5 (4,194,304 rows of bf16 D=128) is checked on every segment through
  size-independent properties computed on the device (every output written,
  finite and in [0, 1]; every segment's columns sum to one), and against the
  oracle on a sample: the longest segment, segments merged through the chunk
  tree and directly, block-class segments and the shortest one.
* Repeating a classified call gives the same bits (the merges fold in a
  fixed order).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import check_expectation, quantized

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, ProgramSpec, native  # noqa: E402
from ragged.workloads import CONFIGS  # noqa: E402

DEVICE = torch.device("cuda", 0)
GUARD = 16
SELECTS = ("auto-bench", "auto-max-len", "classified", "naive")

_workloads: dict = {}
_programs: dict = {}


def workload(name: str, seed: int = 711):
    key = (name, seed)
    if key not in _workloads:
        _workloads.clear()          # one configuration's inputs at a time (C5 holds 2 GiB of f32 values)
        w = CONFIGS[name](seed)
        tdtype = torch.bfloat16 if w.dtype == "bf16" else torch.float32
        x = torch.from_numpy(w.values).to(DEVICE).to(tdtype).contiguous()
        off = torch.from_numpy(w.offsets).to(DEVICE)
        _workloads[key] = (w, x, off)
    return _workloads[key]


def program_for(cache, op, w):
    key = (op, w.dtype, w.d, w.offsets_dtype)
    if key not in _programs:
        _programs[key] = Compiler().compile(ProgramSpec(op, w.dtype, w.d, w.offsets_dtype), cache)
    return _programs[key]


def run_select(program, w, x, off, op, select):
    """One call as ``select`` names it; returns the device output (NaN
    before the call, so an unwritten row shows) and the report. A guard of
    sentinel rows on either side must survive the call."""
    rows = w.n if op == "softmax" else w.b
    guarded = torch.full((rows + 2 * GUARD, w.d), float("nan"), dtype=x.dtype, device=DEVICE)
    guarded[:GUARD] = -64.0
    guarded[GUARD + rows:] = -64.0
    out = guarded[GUARD:GUARD + rows]
    if select == "auto-bench":
        report = program.run(x, off, out, max_len=w.max_len if w.pass_max_len else None)
    elif select == "auto-max-len":
        report = program.run(x, off, out, max_len=w.max_len)
    else:
        report = program.run(x, off, out, select=select, max_len=w.max_len)
        assert report.selected == select
    torch.cuda.synchronize()
    assert bool(torch.all(guarded[:GUARD] == -64.0)) and bool(torch.all(guarded[GUARD + rows:] == -64.0)), \
        "kernel wrote outside the output rows"
    return out, report


def bits(tensor):
    return tensor.view(torch.int16 if tensor.dtype == torch.bfloat16 else torch.int32)


def oracle_inputs(w):
    return quantized(w.values, w.dtype)


@pytest.mark.parametrize("seed", [711, 712, 713])
def test_c1_sum_f32_d1_uniform64(artifact_cache, seed):
    w, x, off = workload("c1", seed)
    assert (w.n, w.b) == (640_000, 10_000) and np.all(w.lengths == 64)
    program = program_for(artifact_cache, "sum", w)
    expectation = oracle.Expectation(oracle_inputs(w), w.offsets, operation="sum", input_dtype="f32")
    for select in SELECTS:
        out, report = run_select(program, w, x, off, "sum", select)
        stats = check_expectation(out.float().cpu().numpy().astype(np.float64), expectation)
        print(f"C1 seed {seed} {select} ({report.selected}): {stats}")


@pytest.mark.parametrize("op", ["sum", "max"])
def test_c2_sum_max_f32_d128_nonfinite(artifact_cache, op):
    w, x, off = workload("c2")
    assert w.b == 4096 and w.d == 128 and int((w.lengths == 0).sum()) >= 20
    inputs = oracle_inputs(w)
    assert np.isnan(inputs).mean() > 5e-4 and np.isneginf(inputs).mean() > 5e-4
    program = program_for(artifact_cache, op, w)
    expectation = oracle.Expectation(inputs, w.offsets, operation=op, input_dtype="f32")
    first = None
    for select in SELECTS:
        out, report = run_select(program, w, x, off, op, select)
        stats = check_expectation(out.float().cpu().numpy().astype(np.float64), expectation)
        print(f"C2 {op} {select} ({report.selected}): {stats}")
        if op == "max":
            # Every schedule selects the same input element: identical bits.
            if first is None:
                first = bits(out).clone()
            else:
                assert torch.equal(bits(out), first)


def test_c3_softmax_f32_d1_geometric(artifact_cache):
    w, x, off = workload("c3")
    assert w.b == 200_000 and w.offsets_dtype == "i32" and w.lengths.min() >= 1 and w.lengths.max() <= 32
    program = program_for(artifact_cache, "softmax", w)
    expectation = oracle.Expectation(oracle_inputs(w), w.offsets, operation="softmax", input_dtype="f32")
    for select in SELECTS:
        out, report = run_select(program, w, x, off, "softmax", select)
        stats = check_expectation(out.float().cpu().numpy().astype(np.float64), expectation)
        print(f"C3 {select} ({report.selected}, {report.kernel_names}): {stats}")


@pytest.mark.parametrize("op", ["sum", "max"])
def test_c4_sum_max_f32_d2_bimodal(artifact_cache, op):
    w, x, off = workload("c4")
    assert w.b == 50_000 and w.d == 2 and w.offsets_dtype == "i32"
    assert int((w.lengths >= 2000).sum()) == 2500
    program = program_for(artifact_cache, op, w)
    expectation = oracle.Expectation(oracle_inputs(w), w.offsets, operation=op, input_dtype="f32")
    for select in SELECTS:
        out, report = run_select(program, w, x, off, op, select)
        stats = check_expectation(out.float().cpu().numpy().astype(np.float64), expectation)
        print(f"C4 {op} {select} ({report.selected}): {stats}")


def c5_sample(w, t_block: int, part_rows: int) -> np.ndarray:
    """Segment ids for the oracle on C5: the longest, the shortest, 8
    segments merged through the chunk tree (more than 16 chunks), 16 merged
    directly (2..16 chunks), 64 block-class segments."""
    rng = np.random.default_rng(5)
    lengths = w.lengths
    chunks = -(-lengths // part_rows)
    picks = {int(np.argmax(lengths)), int(np.argmin(lengths))}
    for pool, count in ((np.flatnonzero((lengths > t_block) & (chunks > 16)), 8),
                        (np.flatnonzero((lengths > t_block) & (chunks <= 16)), 16),
                        (np.flatnonzero(lengths <= t_block), 64)):
        assert len(pool) >= count
        picks.update(int(i) for i in rng.choice(pool, size=count, replace=False))
    return np.array(sorted(picks), dtype=np.int64)


def check_c5_sample(out, w, ids):
    lo, hi = w.offsets[ids].astype(np.int64), w.offsets[ids + 1].astype(np.int64)
    rows = np.concatenate([np.arange(a, b) for a, b in zip(lo, hi)])
    sub_offsets = np.concatenate([[0], np.cumsum(hi - lo)]).astype(np.int64)
    actual = out[torch.from_numpy(rows).to(DEVICE)].float().cpu().numpy().astype(np.float64)
    inputs = oracle.quantize_bf16(w.values[rows])
    stats = oracle.assert_matches(actual, inputs, sub_offsets, operation="softmax", input_dtype="bf16")
    oracle.assert_matches(actual, inputs, sub_offsets, operation="softmax", input_dtype="bf16",
                          tolerances=oracle.STRICT_TOLERANCES)
    stats["rows_checked"] = int(len(rows))
    return stats


def check_c5_properties(out, off):
    """Every row written, finite and in [0, 1]; every segment's columns sum
    to one within the bf16 tolerance (rtol + atol of the strict table),
    totals taken in float64 on the device."""
    assert bool(torch.isfinite(out).all()), "a C5 output is NaN or infinite (unwritten row?)"
    assert bool((out >= 0).all()) and bool((out <= 1).all())
    totals = torch.cumsum(out.double(), dim=0)
    starts, ends = off[:-1].long(), off[1:].long()
    nonempty = ends > starts
    upper = totals[(ends - 1).clamp(min=0)]
    lower = torch.where((starts > 0)[:, None], totals[(starts - 1).clamp(min=0)], torch.zeros_like(upper))
    sums = (upper - lower)[nonempty]
    rtol, atol = oracle.STRICT_TOLERANCES["bf16"]
    worst = float((sums - 1).abs().max())
    assert worst <= rtol + atol, f"a C5 segment column sums to 1 +- {worst}"
    return worst


@pytest.mark.parametrize("select", SELECTS)
def test_c5_softmax_bf16_d128_longtail(artifact_cache, select):
    w, x, off = workload("c5")
    assert (w.n, w.b, w.max_len) == (4_194_304, 8_192, 200_000) and w.pass_max_len
    program = program_for(artifact_cache, "softmax", w)
    spec = native.make_spec("softmax", "bf16", "i64", 128)
    out, report = run_select(program, w, x, off, "softmax", select)
    worst = check_c5_properties(out, off)
    stats = check_c5_sample(out, w, c5_sample(w, int(spec.t_block), int(spec.part_rows)))
    print(f"C5 {select} ({report.selected}, {report.kernel_names}): column sums within {worst:.3g}; "
          f"sampled oracle {stats}")


@pytest.mark.parametrize("name,op", [("c1", "sum"), ("c2", "sum"), ("c2", "max"), ("c3", "softmax"),
                                     ("c4", "sum"), ("c4", "max"), ("c5", "softmax")])
def test_classified_repeats_bit_for_bit(artifact_cache, name, op):
    """The classified schedule's merges fold in a fixed order (split parts in
    part order, softmax chunks in chunk order), whichever workgroup arrives
    last: two calls give the same bits."""
    w, x, off = workload(name)
    program = program_for(artifact_cache, op, w)
    first, _ = run_select(program, w, x, off, op, "classified")
    first = bits(first).clone()
    for _ in range(2):
        again, _ = run_select(program, w, x, off, op, "classified")
        assert torch.equal(bits(again), first)
