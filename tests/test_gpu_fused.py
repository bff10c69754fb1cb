"""GPU tests of the register-resident softmax (k_softmax_fused): segments of
many chunks (both merge levels), non-finite columns split across chunks, the
bounded-wait fallback (the kernel's drain of deferred chunks) forced from the
host, and the debug queue/visit buffers."""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import check, run_program

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, ProgramSpec  # noqa: E402
from ragged.runtime import _modules  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402


def compile_softmax(cache, dtype, d, offsets_dtype="i64", **kwargs):
    program = Compiler().compile(ProgramSpec("softmax", dtype, d, offsets_dtype, **kwargs), cache)
    assert program.metadata["fused"], "expected the register-resident schedule"
    return program


def module_of(program):
    return _modules[(0, program._digest)]


@pytest.mark.parametrize("dtype,d,longest", [("bf16", 128, 100_000), ("f32", 128, 20_000), ("bf16", 64, 40_000),
                                             ("f32", 16, 70_000), ("bf16", 256, 9_000), ("f32", 1024, 3_000)])
def test_many_chunk_segments(artifact_cache, dtype, d, longest):
    program = compile_softmax(artifact_cache, dtype, d)
    lengths = np.array([3, longest, 0, 257, 1, longest // 3, 40, 4096, 5000, 12], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = (np.random.default_rng(d).normal(size=(int(offsets[-1]), d)) * 2).astype(np.float32)
    actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified")
    assert "ragged_0_fused_online" in report.kernel_names
    check(actual, values, offsets, op="softmax", dtype=dtype)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_nonfinite_columns_across_chunks(artifact_cache, dtype):
    d = 16
    program = compile_softmax(artifact_cache, dtype, d)
    capacity = program.metadata["part_rows"]
    lengths = np.array([5 * capacity + 7, capacity, 2 * capacity + 1, 3], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(3).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    first = lengths[0]
    values[:first, 0] = -np.inf                    # all -inf over five chunks
    values[:first:2, 1] = -np.inf                  # mixed
    values[capacity * 3 + 5, 2] = np.inf           # +inf in one chunk poisons all
    values[2, 3] = np.nan                          # NaN in the first chunk
    values[first:first + capacity, 4] = -np.inf    # whole block segment column -inf
    values[first + capacity:first + 2 * capacity, 5] = -np.inf   # one full chunk of -inf, others finite
    actual, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified")
    check(actual, values, offsets, op="softmax", dtype=dtype)


@pytest.mark.parametrize("dtype,kwargs", [("f32", {}), ("bf16", {}), ("bf16", {"scale": 0.5}),
                                          ("f32", {"scale": 2.0})])
def test_deferred_path_matches(artifact_cache, dtype, kwargs):
    """With a zero wait limit almost every chunk of a long segment leaves its
    registers and is normalised by the kernel's drain (a re-read; with a zero
    limit its own wait gives up too and the last workgroup finishes it); the
    bits are those of the default run (bf16 rows held as loaded, f32 rows
    and the f32 logits of a scaled bf16 input)."""
    d = 128
    program = compile_softmax(artifact_cache, dtype, d, **kwargs)
    lengths = make_lengths("long_tail", 200, seed=9, total_elements=60_000)
    lengths[7] = 30_000
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(5).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    baseline, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified")
    module = module_of(program)
    try:
        module.set_spin_limit(0)
        actual, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified")
    finally:
        module.set_spin_limit(-1)
    check(actual, values, offsets, op="softmax", dtype=dtype, scale=kwargs.get("scale", 1.0))
    # The re-read repeats the register path's arithmetic (the same
    # normaliser from the same fold of the segment's statistics): the same
    # bits.
    assert np.array_equal(actual, baseline)


def test_debug_visits_and_queues(artifact_cache):
    """Every segment's final output stage runs exactly once; queue membership
    matches the length thresholds (reference test_classified.py:102-143)."""
    d = 128
    program = Compiler().compile(ProgramSpec("softmax", "bf16", d, "i64", debug_visits=True), artifact_cache)
    thresholds = program.metadata["thresholds"]
    lengths = np.array([0, 1, thresholds[0], thresholds[0] + 1, thresholds[1], thresholds[1] + 1,
                        10 * thresholds[1], 33, 4097, 0], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(1).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    buffers = {}
    actual, _ = run_program(program, values, offsets, dtype="bf16", op="softmax", debug_buffers=buffers)
    check(actual, values, offsets, op="softmax", dtype="bf16")
    counts = buffers["class_counts"].cpu().numpy()
    classes = np.where(lengths <= thresholds[0], 0, np.where(lengths <= thresholds[1], 1, 2))
    np.testing.assert_array_equal(counts[:3], np.bincount(classes, minlength=3))
    ids = buffers["segment_ids"].cpu().numpy()
    for c in range(3):
        np.testing.assert_array_equal(np.sort(ids[c, :counts[c]]), np.flatnonzero(classes == c))
    np.testing.assert_array_equal(buffers["visits"].cpu().numpy(), np.ones(len(lengths), dtype=np.int32))


@pytest.mark.parametrize("chunks", [24, 48])
def test_waits_end_when_workgroups_are_short(chunks):
    """Another process holding most CUs leaves fewer workgroups resident than
    the plan's grid; shrinking the register-resident launch to 4 workgroups
    through the C-ABI shows it. A segment of `chunks` chunks then has all
    resident workgroups waiting for chunks nobody can take: the ticket
    counter, unchanged over two checks 1/20 of the 2 ms spin bound apart,
    ends each wait, the chunks take the re-read pass, and the result is
    exact. Without that rule every round of 4 chunks would wait the full
    2 ms."""
    from gpu_helpers import check as check_result
    from ragged import native
    spec = native.make_spec("softmax", "bf16", "i64", 128)
    module = native.NativeModule(0, spec)
    capacity = int(spec.part_rows)
    lengths = np.array([3, chunks * capacity, 100, capacity + 1, 7], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    n, b = int(offsets[-1]), len(lengths)
    values = np.random.default_rng(chunks).normal(size=(n, 128)).astype(np.float32)
    plan = module.plan(n, b, "classified")
    fused = [i for i in range(plan.launches) if native.ROLES[plan.roles[i]] == "fused"]
    assert len(fused) == 1 and plan.grid[fused[0]][0] > 4
    plan.grid[fused[0]][0] = 4
    x = torch.from_numpy(values).to("cuda").to(torch.bfloat16)
    off = torch.from_numpy(offsets).to("cuda")
    out = torch.full_like(x, float("nan"))
    workspace = torch.zeros((int(plan.workspace_bytes),), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    times = []
    for _ in range(2):
        out.fill_(float("nan"))
        start.record()
        module.run(plan, x.data_ptr(), off.data_ptr(), out.data_ptr(), None, workspace.data_ptr(),
                   int(plan.workspace_bytes), stream.cuda_stream)
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end))
        check_result(out.float().cpu().numpy().astype(np.float64), x.float().cpu().numpy(), offsets, op="softmax",
                     dtype="bf16")
    rounds = chunks // 4
    print(f"{chunks} chunks on 4 workgroups: {times} ms")
    assert min(times) < 0.25 * rounds * 2.0, f"waits ran to their 2 ms bound: {times} ms for {rounds} rounds"
    module.close()


@pytest.mark.parametrize("dtype,d,longest,scale", [("bf16", 128, 300_000, 1.0), ("f32", 16, 1_500_000, 1.0),
                                                  ("bf16", 64, 500_000, 0.5)])
def test_segments_beyond_the_resident_grid(artifact_cache, dtype, d, longest, scale):
    """A segment of more chunks than the device holds at once: its chunks
    publish their statistics without waiting and are all finished by the
    kernel's drain (re-read with the register path's row mapping and
    arithmetic), next to segments that wait; the deferred list is swept by
    the last workgroup a block of entries at a time."""
    kwargs = {"scale": scale} if scale != 1.0 else {}
    program = compile_softmax(artifact_cache, dtype, d, **kwargs)
    capacity = int(program.metadata["part_rows"])
    lengths = np.array([17, longest, 3 * capacity + 5, 0, 40 * capacity, 1], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(longest).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    for select in ("classified", "naive"):
        actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select=select)
        assert report.selected == select
        check(actual, values, offsets, op="softmax", dtype=dtype, scale=scale)


@pytest.mark.parametrize("dtype,d,scale,masked", [("bf16", 128, 1.0, False), ("bf16", 64, 0.5, False),
                                                  ("f32", 128, 1.0, False), ("bf16", 64, 1.0, True)])
def test_long_segments_take_the_streaming_schedule(artifact_cache, dtype, d, scale, masked):
    """With max_len, run(select="auto") sends a register-resident softmax call
    whose segments too long to hold in registers surely carry at least half
    the rows and 1.5 register limits to the streaming worker's split
    schedule (classify + worker), which matches the oracle; forced classified
    keeps the register-resident kernel, and a long segment that is a small
    share of the rows stays there too."""
    kwargs = {"scale": scale} if scale != 1.0 else {}
    if masked:
        kwargs["mask"] = True
    program = compile_softmax(artifact_cache, dtype, d, **kwargs)
    part = int(program.metadata["part_rows"])
    limit = max(1, program._module(0).resident_blocks("fused") * 7 // 8) * part
    lengths = np.array([17, 2 * limit + 3 * part + 5, 3 * part, 0, 1], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    rng = np.random.default_rng(d)
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    mask = rng.normal(size=values.shape).astype(np.float32) if masked else None
    max_len = int(lengths.max())
    actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select="auto",
                                 max_len=max_len, mask=mask)
    assert report.selection.get("streaming") and report.selected == "classified"
    assert not any("fused" in name for name in report.kernel_names), report.kernel_names
    check(actual, values, offsets, op="softmax", dtype=dtype, scale=scale, mask=mask)
    actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified",
                                 max_len=max_len, mask=mask)
    assert not report.selection.get("streaming")
    assert any("fused" in name for name in report.kernel_names), report.kernel_names
    check(actual, values, offsets, op="softmax", dtype=dtype, scale=scale, mask=mask)
    if masked:
        return
    # The long segment a third of the rows: register-resident (it defers that segment).
    short = np.array([limit + 5] + [part] * (2 * (limit + 5) // part + 1), dtype=np.int64)
    offsets = offsets_from_lengths(short, "i64")
    values = np.random.default_rng(d + 1).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select="auto",
                                 max_len=int(short.max()))
    assert not report.selection.get("streaming") and report.selected == "classified"
    assert any("fused" in name for name in report.kernel_names), report.kernel_names
    check(actual, values, offsets, op="softmax", dtype=dtype, scale=scale)
