"""GPU parity: every op x dtype x width x offsets dtype x length distribution,
both schedules, against the float64 CPU oracle (max bit-exact).

Mirrors the reference's test/gpu/test_correctness.py matrix (:123-130) with
the wave64 classes of this build. Sizes keep each case to well under a
second of oracle time.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import check, quantized, run_program

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, Hints, Optimizations, ProgramSpec, ValidationError, native  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

_programs = {}


def program_for(cache, op, dtype, d, offsets_dtype, **kwargs):
    key = (op, dtype, d, offsets_dtype, tuple(sorted(kwargs.items())))
    if key not in _programs:
        _programs[key] = Compiler().compile(ProgramSpec(op, dtype, d, offsets_dtype, **kwargs), cache)
    return _programs[key]


def lengths_for(distribution: str, segments: int, total: int, seed: int) -> np.ndarray:
    if distribution == "empties":
        lengths = make_lengths("exponential", segments, seed=seed, total_elements=total)
        lengths[::3] = 0
        return lengths
    if distribution == "one_long":
        lengths = np.zeros(segments, dtype=np.int64)
        lengths[segments // 2] = total
        return lengths
    return make_lengths(distribution, segments, seed=seed, total_elements=total)


def case(d: int, distribution: str, seed: int, offsets_dtype: str, rows_budget: int = 400_000):
    total = max(256, min(rows_budget // d, 60_000))
    segments = 97 if distribution == "one_long" else 700
    lengths = lengths_for(distribution, segments, total, seed)
    offsets = offsets_from_lengths(lengths, offsets_dtype)
    values = np.random.default_rng(seed + 1).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    return values, offsets, int(lengths.max())


OPS = ("sum", "max", "softmax")
DISTRIBUTIONS = ("uniform", "long_tail", "bimodal", "burst", "exponential", "empties", "one_long")


@pytest.mark.parametrize("select", ["classified", "naive"])
@pytest.mark.parametrize("distribution", DISTRIBUTIONS)
@pytest.mark.parametrize("d,dtype", [(1, "f32"), (2, "f32"), (3, "f32"), (128, "f32"), (1, "bf16"),
                                     (8, "bf16"), (128, "bf16")])
@pytest.mark.parametrize("op", OPS)
def test_matrix(artifact_cache, op, d, dtype, distribution, select):
    offsets_dtype = "i32" if (d + len(distribution)) % 2 else "i64"
    program = program_for(artifact_cache, op, dtype, d, offsets_dtype)
    values, offsets, longest = case(d, distribution, seed=700 + d, offsets_dtype=offsets_dtype)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select=select, max_len=longest)
    assert report.selected == select
    check(actual, values, offsets, op=op, dtype=dtype)


@pytest.mark.parametrize("d", [5, 64, 96, 256, 1024])
@pytest.mark.parametrize("op", OPS)
def test_other_widths(artifact_cache, op, d):
    program = program_for(artifact_cache, op, "f32", d, "i64")
    values, offsets, _ = case(d, "long_tail", seed=31, offsets_dtype="i64", rows_budget=2_000_000)
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype="f32", op=op, select=select)
        check(actual, values, offsets, op=op, dtype="f32")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("op", OPS)
def test_nonfinite_inputs(artifact_cache, op, dtype):
    """NaN / +inf / -inf per feature column (reference test_oracle.py:37-56,
    test_correctness.py:173-193), including +inf beside -inf and all -inf."""
    d = 8
    program = program_for(artifact_cache, op, dtype, d, "i64")
    rng = np.random.default_rng(5)
    lengths = np.array([3, 0, 1, 40, 600, 5000, 2, 7], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    values[0, 0] = np.nan
    values[3:43, 1] = -np.inf            # an all -inf column of a segment
    values[3, 2] = np.inf
    values[4, 2] = -np.inf               # +inf beside -inf
    values[50, 3] = np.nan
    values[700:5643:7, 4] = -np.inf      # mixed finite / -inf
    values[5643, 5] = np.inf
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype=dtype, op=op, select=select)
        check(actual, values, offsets, op=op, dtype=dtype)


@pytest.mark.parametrize("op", OPS)
def test_empty_inputs(artifact_cache, op):
    program = program_for(artifact_cache, op, "f32", 4, "i64")
    for offsets in (np.array([0], dtype=np.int64), np.array([0, 0, 0, 0], dtype=np.int64)):
        values = np.zeros((0, 4), dtype=np.float32)
        actual, report = run_program(program, values, offsets, dtype="f32", op=op)
        check(actual, values, offsets, op=op, dtype="f32")
        if len(offsets) == 1:
            assert report.kernel_names == () and report.workspace_bytes == 0


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_accumulation_accuracy_long_segment(artifact_cache, dtype):
    """A 16,384-row segment of 0.1 and -ln(10) (reference
    test_correctness.py:204-217) and the 131,073-row exact sums of
    test_oracle.py:188-193."""
    program = program_for(artifact_cache, "sum", dtype, 3, "i64")
    values = np.tile(np.array([[1, -1, 0.5]], dtype=np.float32), (131073, 1))
    offsets = np.array([0, 131073], dtype=np.int64)
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype=dtype, op="sum", select=select)
        if dtype == "f32":
            np.testing.assert_array_equal(actual, [[131073, -131073, 65536.5]])
        check(actual, values, offsets, op="sum", dtype=dtype)
    values = np.tile(np.array([[0.1, -np.log(10.0), 1.0]], dtype=np.float32), (16384, 1))
    offsets = np.array([0, 16384], dtype=np.int64)
    softmax = program_for(artifact_cache, "softmax", dtype, 3, "i64")
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype=dtype, op="sum", select=select)
        check(actual, values, offsets, op="sum", dtype=dtype)
        actual, _ = run_program(softmax, values, offsets, dtype=dtype, op="softmax", select=select)
        check(actual, values, offsets, op="softmax", dtype=dtype)


def test_softmax_rescale_ramps(artifact_cache):
    """Small mass over 65,536 rows and repeated rescaling (reference
    test_class_fusion.py:106-123)."""
    program = program_for(artifact_cache, "softmax", "f32", 4, "i64")
    n = 65536
    ramp = np.arange(n, dtype=np.float64)
    values = np.stack([ramp * 7.457e-9, ramp * 6.613e-5, ramp * 1e-3, -ramp * 1e-3], axis=1).astype(np.float32)
    offsets = np.array([0, n], dtype=np.int64)
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype="f32", op="softmax", select=select)
        check(actual, values, offsets, op="softmax", dtype="f32")


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_scale_and_mask(artifact_cache, dtype):
    """f32(values) * scale + mask (docs/mask-abi.md:28-43) for softmax, and
    scale for the reductions."""
    d = 16
    rng = np.random.default_rng(11)
    lengths = make_lengths("long_tail", 300, seed=3, total_elements=20_000)
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    mask = np.where(rng.random(values.shape) < 0.2, -np.inf, rng.normal(size=values.shape)).astype(np.float32)
    program = program_for(artifact_cache, "softmax", dtype, d, "i64", mask=True, scale=0.5)
    for select in ("classified", "naive"):
        actual, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select=select, mask=mask)
        check(actual, values, offsets, op="softmax", dtype=dtype, mask=mask, scale=0.5)
    for op in ("sum", "max"):
        program = program_for(artifact_cache, op, dtype, d, "i64", scale=-1.5)
        for select in ("classified", "naive"):
            actual, _ = run_program(program, values, offsets, dtype=dtype, op=op, select=select)
            check(actual, values, offsets, op=op, dtype=dtype, scale=-1.5)


def test_unvectorized_unaligned_views(artifact_cache):
    """vectorize=False accepts views at any element offset."""
    d = 8
    program = Compiler().compile(ProgramSpec("sum", "f32", d, "i64", optimizations=Optimizations(vectorize=False)),
                                 artifact_cache)
    lengths = make_lengths("uniform", 50, seed=1, total_elements=5000)
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(2).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    actual, _ = run_program(program, values, offsets, dtype="f32", op="sum", select="classified")
    check(actual, values, offsets, op="sum", dtype="f32")


@pytest.mark.parametrize("op", OPS)
@pytest.mark.parametrize("d,dtype", [(1, "f32"), (2, "f32"), (4, "bf16"), (3, "f32"), (128, "f32"), (8, "bf16")])
def test_short_segment_schedule(artifact_cache, op, d, dtype):
    """With max_len at most alone_rows (segments one lane or lane group
    reduces alone) one worker launch takes the segments in order; a max_len
    below the true longest segment (a caller's mistake) still gives exact
    results."""
    program = program_for(artifact_cache, op, dtype, d, "i64")
    t_wave = native.make_spec(op, dtype, "i64", d).alone_rows
    assert t_wave > 0
    rng = np.random.default_rng(40 + d)
    lengths = rng.integers(0, t_wave + 1, size=3000).astype(np.int64)
    lengths[::7] = 0
    lengths[11] = t_wave
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified",
                                 max_len=int(lengths.max()))
    assert report.selection.get("short_segments") and len(report.kernel_names) == 1
    assert report.workspace_bytes == 0
    check(actual, values, offsets, op=op, dtype=dtype)
    lengths[5] = 5 * t_wave + 17
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified", max_len=t_wave)
    assert report.selection.get("short_segments")
    check(actual, values, offsets, op=op, dtype=dtype)


@pytest.mark.parametrize("d,dtype", [(1, "f32"), (2, "bf16"), (4, "f32"), (3, "f32"), (32, "bf16"), (128, "f32"),
                                     (96, "f32"), (1024, "f32")])
@pytest.mark.parametrize("op", OPS)
def test_wave_class_runs(artifact_cache, op, d, dtype):
    """The wave class in its two runs: segments of at most alone_rows rows
    (one lane or lane group each, queued from the front) and the rest up to
    t_wave (one wave each, queued from the back), mixed with block and split
    segments and empties; exact results, and the debug view presents the
    wave class as one run (reference test_classified.py:102-143)."""
    spec = native.make_spec(op, dtype, "i64", d)
    alone, t_wave, t_block = spec.alone_rows, spec.t_wave, spec.t_block
    assert alone <= t_wave < t_block
    rng = np.random.default_rng(900 + d)
    pieces = [np.zeros(40, dtype=np.int64), rng.integers(1, max(alone, 1) + 1, size=300),
              rng.integers(alone + 1, t_wave + 1, size=300) if t_wave > alone else np.zeros(0, np.int64),
              np.array([t_wave, t_wave + 1, alone, alone + 1, t_block, t_block + 1]),
              rng.integers(t_wave + 1, min(t_block, t_wave + 4000) + 1, size=20)]
    lengths = rng.permutation(np.concatenate(pieces)).astype(np.int64)
    lengths = np.maximum(lengths, 0)
    budget = 3_000_000 // d
    while lengths.sum() > budget:     # keep the oracle quick: shorten the longest
        lengths[np.argmax(lengths)] //= 2
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    program = program_for(artifact_cache, op, dtype, d, "i64")
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified")
    assert report.selected == "classified"
    check(actual, values, offsets, op=op, dtype=dtype)
    debug = program_for(artifact_cache, op, dtype, d, "i64", debug_visits=True)
    buffers = {}
    actual, _ = run_program(debug, values, offsets, dtype=dtype, op=op, debug_buffers=buffers)
    check(actual, values, offsets, op=op, dtype=dtype)
    thresholds = debug.metadata["thresholds"]
    classes = np.where(lengths <= thresholds[0], 0, np.where(lengths <= thresholds[1], 1, 2))
    counts = buffers["class_counts"].cpu().numpy()
    np.testing.assert_array_equal(counts[:3], np.bincount(classes, minlength=3))
    ids = buffers["segment_ids"].cpu().numpy()
    for c in range(3):
        np.testing.assert_array_equal(np.sort(ids[c, :counts[c]]), np.flatnonzero(classes == c))
    np.testing.assert_array_equal(buffers["visits"].cpu().numpy(), np.ones(len(lengths), dtype=np.int32))


@pytest.mark.parametrize("d,dtype,masked", [(1, "f32", False), (2, "f32", True), (4, "bf16", False), (1, "bf16", True)])
def test_softmax_split_parts_normalised_by_worker(artifact_cache, d, dtype, masked):
    """Softmax with many split segments of several parts each (streaming
    worker geometries): the worker normalises every part once its segment's
    statistics are out; exact results, every segment written once, and no
    separate normalisation launch."""
    spec = native.make_spec("softmax", dtype, "i64", d)
    t_block, part_rows = spec.t_block, spec.part_rows
    rng = np.random.default_rng(41 + d)
    long = rng.integers(t_block + 1, t_block + 2 * part_rows, size=8)
    lengths = rng.permutation(np.concatenate([long, rng.integers(0, 300, size=3000), [t_block + 1]]))
    lengths = lengths.astype(np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    kwargs = dict(mask=True, scale=0.75) if masked else {}
    mask = np.where(rng.random(values.shape) < 0.1, -np.inf, rng.normal(size=values.shape)).astype(np.float32) \
        if masked else None
    program = program_for(artifact_cache, "softmax", dtype, d, "i64", **kwargs)
    actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified", mask=mask)
    assert "split_normalize" not in " ".join(report.kernel_names)
    check(actual, values, offsets, op="softmax", dtype=dtype, mask=mask, scale=0.75 if masked else 1.0)
    debug = program_for(artifact_cache, "softmax", dtype, d, "i64", debug_visits=True, **kwargs)
    buffers = {}
    actual, _ = run_program(debug, values, offsets, dtype=dtype, op="softmax", mask=mask, debug_buffers=buffers)
    check(actual, values, offsets, op="softmax", dtype=dtype, mask=mask, scale=0.75 if masked else 1.0)
    assert int(buffers["class_counts"].cpu().numpy()[2]) == int((lengths > t_block).sum())
    np.testing.assert_array_equal(buffers["visits"].cpu().numpy(), np.ones(len(lengths), dtype=np.int32))


def test_misaligned_workspace_rejected(artifact_cache):
    """rg_run takes the workspace at a 256-byte aligned address (its buffers
    sit at 256-byte offsets and are filled with 16-byte stores): a shifted
    pointer is rejected before any launch, the aligned one runs."""
    program = program_for(artifact_cache, "softmax", "bf16", 128, "i64")
    lengths = np.array([300, 5, 700, 0, 40], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    device = torch.device("cuda", 0)
    values = torch.randn(int(offsets[-1]), 128, device=device).to(torch.bfloat16)
    off = torch.from_numpy(offsets).to(device)
    out = torch.full_like(values, -7)
    module = program._module(0)
    plan = program._plan(module, values.shape[0], len(lengths), "classified")
    assert plan.workspace_bytes > 0
    workspace = torch.zeros(plan.workspace_bytes + 256, dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    with pytest.raises(ValidationError, match="aligned"):
        module.run(plan, values.data_ptr(), off.data_ptr(), out.data_ptr(), None, workspace.data_ptr() + 16,
                   plan.workspace_bytes, stream)
    torch.cuda.synchronize()
    assert bool(torch.all(out == -7)), "a rejected call wrote its output"
    module.run(plan, values.data_ptr(), off.data_ptr(), out.data_ptr(), None, workspace.data_ptr(),
               plan.workspace_bytes, stream)
    torch.cuda.synchronize()
    check(out.float().cpu().numpy().astype(np.float64), quantized(values.float().cpu().numpy(), "bf16"), offsets,
          op="softmax", dtype="bf16")


ARENA = ("pairs", "final_pairs", "arrive", "deferred")
CLEAN_SLOT, DIRTY_SLOT, DIRTY_RANGES = 12, 14, 3


@pytest.mark.parametrize("op,dtype,d", [("sum", "f32", 1), ("max", "f32", 128), ("softmax", "f32", 1024),
                                        ("softmax", "bf16", 128), ("softmax", "f32", 2), ("sum", "bf16", 1024)])
def test_workspace_counters_return_to_zero(artifact_cache, op, dtype, d):
    """The workspace contract: zero before its first call; every call
    initialises the per-segment state it uses (queues, tables, arrival
    counters) and its last workgroup returns the counters to zero, except
    slot 12 and slots 14-19, the register-resident softmax's arena record:
    such a call leaves its arena (pairs, group rows, group counters, deferred
    list) zero but for the byte ranges of the pairs and group rows it
    published, records its arena bytes + 2 in slot 12 and those ranges in
    slots 14-19; any other call records 1 (arena unknown). The next call's
    classification zeroes what the record names. So after each call the
    counters and the arena read so; garbage (0xFF) everywhere else changes no
    result, nor does garbage in the recorded ranges, nor garbage in the whole
    arena recorded as unknown."""
    rng = np.random.default_rng(77 + d)
    # d >= 128: one segment long enough for the register-resident softmax's
    # tree merge (more than 16 chunks of 256 rows), whose group rows and
    # counters the call must leave as recorded.
    lengths = np.concatenate([np.zeros(30, np.int64), rng.integers(1, 40, size=400),
                              rng.integers(100, 3000, size=12), [20000 // d + 700], [12_000] if d >= 128 else []])
    lengths = rng.permutation(lengths).astype(np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    program = program_for(artifact_cache, op, dtype, d, "i64")
    fused = bool(program.metadata["fused"])
    module = program._module(0)
    plan = program._plan(module, values.shape[0], len(lengths), "classified")
    spans = {name: (offset, nbytes) for name, offset, nbytes in plan.buffers}
    counters = spans["class_counts"]
    arena = None
    if fused:
        lo = min(spans[name][0] for name in ARENA if name in spans)
        hi = max(spans[name][0] + spans[name][1] for name in ARENA if name in spans)
        arena = (lo, (hi + 255) // 256 * 256)

    def set_slot(workspace, slot, value):
        start = counters[0] + 8 * slot
        workspace[start:start + 8] = torch.from_numpy(np.array([value], dtype=np.int64).view(np.uint8)).to(
            workspace.device)

    for call in range(4):
        actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified")
        assert report.workspace_bytes > 0
        assert len(report.kernel_names) == 2      # classify and one worker
        check(actual, values, offsets, op=op, dtype=dtype)
        torch.cuda.synchronize()
        for workspace in program._workspaces.values():
            slots = workspace[counters[0]:counters[0] + counters[1]].view(torch.int64).cpu().numpy().copy()
            if fused:
                assert int(slots[CLEAN_SLOT]) == arena[1] - arena[0] + 2, slots[:20]
                ranges = slots[DIRTY_SLOT:DIRTY_SLOT + 2 * DIRTY_RANGES].reshape(DIRTY_RANGES, 2)
                assert np.all(ranges[:, 0] <= ranges[:, 1]) and ranges.min() >= 0
                assert ranges.max() <= arena[1] - arena[0]
                assert ranges[0, 1] > ranges[0, 0], "published direct pairs recorded"
                image = workspace[arena[0]:arena[1]].cpu().numpy().copy()
                for lo, hi in ranges:
                    image[lo:hi] = 0
                assert not image.any(), "the arena holds nonzero bytes outside the recorded ranges"
                slots[DIRTY_SLOT:DIRTY_SLOT + 2 * DIRTY_RANGES] = 0
            else:
                assert int(slots[CLEAN_SLOT]) == 1, slots[:20]
            slots[CLEAN_SLOT] = 0
            assert not slots.any(), slots[:20]
            workspace[(arena[1] if fused else counters[0] + counters[1]):].fill_(255)
            if fused:
                for lo, hi in ranges:
                    workspace[arena[0] + lo:arena[0] + hi].fill_(255)
                if call % 2:
                    # Another plan's buffers over the arena: garbage there,
                    # recorded as unknown.
                    workspace[arena[0]:arena[1]].fill_(255)
                    set_slot(workspace, CLEAN_SLOT, 1)
        torch.cuda.synchronize()


@pytest.mark.parametrize("d,dtype,masked", [(1, "f32", False), (2, "bf16", True), (4, "bf16", False)])
def test_worker_deferred_split_parts_match(artifact_cache, d, dtype, masked):
    """A split part whose wait for its segment's statistics runs out writes
    nothing and is normalised by the worker's last workgroup. A zero wait
    limit (set from the host) sends every part that does not find its
    statistics at once down that path: the same bits as the default run,
    every segment written once."""
    spec = native.make_spec("softmax", dtype, "i64", d)
    t_block, part_rows = spec.t_block, spec.part_rows
    rng = np.random.default_rng(23 + d)
    long = rng.integers(t_block + 1, t_block + 6 * part_rows, size=12)
    lengths = rng.permutation(np.concatenate([long, rng.integers(0, 300, size=2000)])).astype(np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = rng.normal(size=(int(offsets[-1]), d)).astype(np.float32)
    kwargs = dict(mask=True, scale=1.25) if masked else {}
    mask = rng.normal(size=values.shape).astype(np.float32) if masked else None
    program = program_for(artifact_cache, "softmax", dtype, d, "i64", debug_visits=True, **kwargs)
    assert not program.metadata["fused"]
    baseline, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified", mask=mask,
                              debug_buffers={})
    module = program._module(0)
    try:
        module.set_spin_limit(0)
        buffers = {}
        actual, _ = run_program(program, values, offsets, dtype=dtype, op="softmax", select="classified",
                                mask=mask, debug_buffers=buffers)
    finally:
        module.set_spin_limit(-1)
    np.testing.assert_array_equal(buffers["visits"].cpu().numpy(), np.ones(len(lengths), dtype=np.int32))
    deferred = int(buffers["class_counts"].cpu().numpy()[5])
    print(f"split parts deferred to the last workgroup: {deferred}")
    check(actual, values, offsets, op="softmax", dtype=dtype, mask=mask, scale=1.25 if masked else 1.0)
    assert np.array_equal(actual, baseline, equal_nan=True)


@pytest.mark.parametrize("dtype,offsets_dtype", [("f32", "i64"), ("bf16", "i32")])
@pytest.mark.parametrize("op", ["sum", "max"])
def test_big_reduce_calls_take_larger_split_parts(artifact_cache, monkeypatch, op, dtype, offsets_dtype):
    """Sum / max calls of more than about 256 MiB of rows split long segments
    into parts of about N/512 rows and send segments of up to N/1024 rows to
    the block class (a companion module): on a 742 MB (f32) or 371 MB (bf16,
    i32 offsets) call the result matches
    the oracle (max bit-exact) and the report names the part size and block
    threshold. The same (N, B) on a module with another block threshold gets
    a plan of its own (plans are keyed by module). A call whose max_len fits
    the block class and a small call keep the default."""
    from ragged import runtime
    from ragged.workloads import offsets_from_lengths
    from gpu_helpers import check, run_program
    program = Compiler().compile(ProgramSpec(op, dtype, 128, offsets_dtype), artifact_cache)
    default_rows = int(program.metadata["part_rows"])
    default_block = int(program.metadata["thresholds"][1])
    row_bytes = 128 * (2 if dtype == "bf16" else 4)
    # f32: around the default block threshold (1,024 rows), the raised one
    # (1,280) and the part (2,048): block, one split part, two parts. bf16:
    # the default block threshold is the part (2,048 rows).
    lengths = np.array([(1 << 20) + (1 << 18), 1 << 17, 2049, 2048, 1500, 1025, default_block, 100, 0, 7],
                       dtype=np.int64)
    offsets = offsets_from_lengths(lengths, offsets_dtype)
    values = np.random.default_rng(5).normal(size=(int(offsets[-1]), 128)).astype(np.float32)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified")
    rows = runtime.big_part_rows(int(offsets[-1]), row_bytes, default_rows)
    assert report.selection.get("part_rows") == rows == 2048 > default_rows
    t_block = runtime.big_block_rows(int(offsets[-1]), rows, default_block)
    assert report.selection["t_block"] == report.thresholds[1] == t_block == (1280 if dtype == "f32" else 2048)
    check(actual, values, offsets, op=op, dtype=dtype)
    # The same call with the offsets checked on the device first.
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified", mode="checked")
    assert report.mode == "checked" and report.selection["part_rows"] == rows
    check(actual, values, offsets, op=op, dtype=dtype)
    shipped = runtime.big_block_rows
    monkeypatch.setattr(runtime, "big_block_rows", lambda n, part_rows, default_t_block: default_t_block)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select="classified")
    assert report.selection["t_block"] == report.thresholds[1] == default_block
    plans = {int(plan.t_block) for (module, n, b, schedule), plan in program._plans.items()
             if (n, b, schedule) == (int(offsets[-1]), len(lengths), f"parts{rows}")}
    assert plans == {default_block, t_block}
    check(actual, values, offsets, op=op, dtype=dtype)
    monkeypatch.setattr(runtime, "big_block_rows", shipped)
    short = offsets_from_lengths(np.array([default_block] * 4 + [3], dtype=np.int64), offsets_dtype)
    few = values[:int(short[-1])]
    actual, report = run_program(program, few, short, dtype=dtype, op=op, select="classified",
                                 max_len=default_block)
    assert "part_rows" not in report.selection and report.thresholds[1] == default_block
    check(actual, few, short, op=op, dtype=dtype)
    # A small call that provably splits a segment: N/512 is below twice the
    # default part.
    small = offsets_from_lengths(np.array([3 * default_block, 3], dtype=np.int64), offsets_dtype)
    actual, report = run_program(program, values[:int(small[-1])], small, dtype=dtype, op=op, select="classified")
    assert "part_rows" not in report.selection
    check(actual, values[:int(small[-1])], small, op=op, dtype=dtype)
