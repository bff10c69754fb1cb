"""GPU tests that complete the reference's GPU matrix and its scheduling
contracts:

* the feature widths the reference tests that the main matrix does not: bf16
  D = 6, 12, 16, 24, 40 and 1024 and f32 D = 16, every op, both schedules,
  against the float64 oracle (reference test/gpu/test_correctness.py:118-130
  and test/gpu/test_scheduling.py:96-107);
* a call on a caller's stream behind long prior work: later work on that
  stream sees the output, and two streams running one program at once each
  get their own workspace (test/gpu/test_scheduling.py:123-148);
* every persistent grid is one resident wave of workgroups at most, and the
  register-resident softmax's grid is co-resident while it runs (its bounded
  waits assume so; test/gpu/test_scheduling.py:174-191);
* softmax over logits spanning more than a hundred natural-log units: every
  output is a single rounding (relative error, not only the absolute
  tolerance), and classified and block-per-segment agree with the correctly
  rounded result on which outputs are zero.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import check, quantized, run_program

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, ProgramSpec, native  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

DEVICE = torch.device("cuda", 0)
OPS = ("sum", "max", "softmax")
WIDTHS = [(6, "bf16"), (12, "bf16"), (16, "bf16"), (24, "bf16"), (40, "bf16"), (1024, "bf16"), (16, "f32")]

_programs = {}


def program_for(cache, op, dtype, d, offsets_dtype="i64"):
    key = (op, dtype, d, offsets_dtype)
    if key not in _programs:
        _programs[key] = Compiler().compile(ProgramSpec(op, dtype, d, offsets_dtype), cache)
    return _programs[key]


@pytest.mark.parametrize("select", ["classified", "naive"])
@pytest.mark.parametrize("d,dtype", WIDTHS)
@pytest.mark.parametrize("op", OPS)
def test_reference_widths(artifact_cache, op, d, dtype, select):
    rows = max(3_000, min(2_000_000 // d, 60_000))
    lengths = make_lengths("long_tail", 300, seed=41 + d, total_elements=rows)
    # One segment long enough for split parts / tree-merged chunks at every width.
    lengths[7] = rows // 3
    lengths[11] = 0
    offsets_dtype = "i64" if d % 3 == 0 else "i32"
    offsets = offsets_from_lengths(lengths, offsets_dtype)
    values = np.random.default_rng(d).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    program = program_for(artifact_cache, op, dtype, d, offsets_dtype)
    actual, report = run_program(program, values, offsets, dtype=dtype, op=op, select=select,
                                 max_len=int(lengths.max()))
    assert report.selected == select
    check(actual, values, offsets, op=op, dtype=dtype)


def _busy(stream, torch):
    """Long work on `stream` (a spin kernel, or chained products)."""
    with torch.cuda.stream(stream):
        sleep = getattr(torch.cuda, "_sleep", None)
        if sleep is not None:
            sleep(int(3e8))
        else:  # pragma: no cover - torch builds without the spin kernel
            a = torch.randn((4096, 4096), device=DEVICE)
            for _ in range(40):
                a = a @ a
                a = a / a.abs().max()


def test_caller_stream_ordering(artifact_cache):
    """The call is enqueued on the caller's current stream behind its
    earlier work (the input is only written there after a long spin), and
    work enqueued after it on that stream sees the output; nothing is read
    until that stream is synchronised."""
    program = program_for(artifact_cache, "softmax", "bf16", 128)
    lengths = make_lengths("long_tail", 300, seed=4, total_elements=80_000)
    lengths[5] = 20_000
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(4).normal(size=(int(offsets[-1]), 128)).astype(np.float32)
    base = torch.from_numpy(values).to(DEVICE).to(torch.bfloat16)
    off = torch.from_numpy(offsets).to(DEVICE)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    x = torch.zeros_like(base)
    out = torch.full_like(base, float("nan"))
    _busy(side, torch)
    with torch.cuda.stream(side):
        x.copy_(base)
        program.run(x, off, out, max_len=int(lengths.max()))
        result = out.clone()
    side.synchronize()
    check(result.float().cpu().numpy().astype(np.float64), values, offsets, op="softmax", dtype="bf16")


def test_two_streams_at_once(artifact_cache):
    """One program called on two streams without synchronising between the
    calls: each stream has its own workspace, and every result is exact."""
    program = program_for(artifact_cache, "softmax", "bf16", 128)
    cases = []
    for seed in (8, 9):
        lengths = make_lengths("long_tail", 250, seed=seed, total_elements=60_000)
        lengths[3] = 15_000
        offsets = offsets_from_lengths(lengths, "i64")
        values = np.random.default_rng(seed).normal(size=(int(offsets[-1]), 128)).astype(np.float32)
        x = torch.from_numpy(values).to(DEVICE).to(torch.bfloat16)
        cases.append((values, offsets, x, torch.from_numpy(offsets).to(DEVICE)))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [[torch.empty_like(case[2]) for _ in range(4)] for case in cases]
    for call in range(4):
        for (values, offsets, x, off), stream, out in zip(cases, streams, outs):
            with torch.cuda.stream(stream):
                program.run(x, off, out[call])
    torch.cuda.synchronize()
    assert len(program._workspaces) >= 2
    for (values, offsets, x, off), out in zip(cases, outs):
        for result in out:
            check(result.float().cpu().numpy().astype(np.float64), values, offsets, op="softmax", dtype="bf16")


@pytest.mark.parametrize("op,dtype,d", [("softmax", "bf16", 128), ("softmax", "f32", 128), ("softmax", "bf16", 1024),
                                        ("sum", "f32", 1), ("max", "f32", 128), ("softmax", "f32", 2)])
def test_persistent_grids_are_one_resident_wave(op, dtype, d):
    """A persistent worker's grid never has more workgroups than the device
    holds at once (rg_module_resident, from the occupancy query), and exactly
    that many when the input has more work: the register-resident softmax's
    deadlock argument (a chunk waits only for chunks running workgroups have
    started) needs its whole grid resident."""
    spec = native.make_spec(op, dtype, "i64", d)
    module = native.NativeModule(0, spec)
    props = native.device_props(0)
    role = "fused" if native.uses_fused(spec) else "worker"
    resident = module.resident_blocks(role)
    assert resident > 0 and resident % props.cu_count == 0
    if role == "fused":
        # 4 waves per workgroup at 4 waves per SIMD (launch bounds): 4 per CU.
        assert resident == 4 * props.cu_count
    for n, b, big in ((1_000, 10, False), (4_000_000, 8_192, True)):
        plan = module.plan(n, b, "classified")
        grids = [plan.grid[i][0] for i in range(plan.launches) if native.ROLES[plan.roles[i]] == role]
        assert len(grids) == 1 and 1 <= grids[0] <= resident, (n, b, grids, resident)
        if big:
            assert grids[0] == resident
    module.close()


def test_fused_grid_is_co_resident():
    """While the register-resident softmax runs, all its workgroups are
    resident at once: every workgroup's first item (the first grid-many
    tickets, long-segment chunks that take their next ticket only when they
    store) starts before any item ends. A workgroup that could only start
    once another had left would take a later ticket and break this."""
    spec = native.make_spec("softmax", "bf16", "i64", 128)
    module = native.NativeModule(0, spec)
    capacity = int(spec.part_rows)
    lengths = np.array([600 * capacity, 300 * capacity, 400 * capacity, 50], dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    n, b = int(offsets[-1]), len(lengths)
    plan = module.plan(n, b, "classified")
    grid = [plan.grid[i][0] for i in range(plan.launches) if native.ROLES[plan.roles[i]] == "fused"][0]
    x = torch.randn((n, 128), device=DEVICE).to(torch.bfloat16)
    off = torch.from_numpy(offsets).to(DEVICE)
    out = torch.empty_like(x)
    workspace = torch.zeros((int(plan.workspace_bytes),), dtype=torch.uint8, device=DEVICE)
    records = int(plan.items_cap + b + 8)
    trace = torch.zeros((records, 8), dtype=torch.int64, device=DEVICE)
    module.set_trace(trace.data_ptr(), records)
    try:
        module.run(plan, x.data_ptr(), off.data_ptr(), out.data_ptr(), None, workspace.data_ptr(),
                   int(plan.workspace_bytes), torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
    finally:
        module.set_trace(None)
    rows = trace.cpu().numpy()
    rows = rows[rows[:, 1] > 0]
    first = rows[rows[:, 0] < grid]
    assert len(first) == grid
    latest_start = int(first[:, 1].max())
    earliest_end = int(rows[:, 5].min())
    print(f"grid {grid}: last first-item start {latest_start}, first item end {earliest_end} (ticks)")
    assert latest_start < earliest_end
    check(out.float().cpu().numpy().astype(np.float64), x.float().cpu().numpy(), offsets, op="softmax", dtype="bf16")
    module.close()


@pytest.mark.parametrize("sigma", [8.0, 16.0])
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_wide_range_logits(artifact_cache, dtype, sigma):
    """Logits of standard deviation 8 and 16: within a segment they span
    well over a hundred natural-log units, so most probabilities are far
    below the largest. Each output must be one rounding of the exact value
    (bf16: within half a bf16 ulp, i.e. 2^-8 relative; f32: within 2e-5
    relative) wherever the exact value is a normal number, nonzero there, and
    zero wherever the correctly rounded result is zero, in both schedules
    (exact values in the subnormal band may flush either way): the segments
    cover whole items, directly merged and tree-merged chunks, and the wave
    class."""
    d = 128
    program = program_for(artifact_cache, "softmax", dtype, d)
    capacity = int(program.metadata["part_rows"])
    lengths = np.array([20, 3, capacity // 2, capacity, 4 * capacity + 17, 40 * capacity + 5, 1, 0, 60],
                       dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = (np.random.default_rng(int(sigma)).normal(size=(int(offsets[-1]), d)) * sigma).astype(np.float32)
    inputs = quantized(values, dtype)
    expected = oracle.segment_softmax(inputs.astype(np.float64), offsets)
    rounded = oracle.quantize_bf16(expected.astype(np.float32)) if dtype == "bf16" else expected.astype(np.float32)
    tiny = np.finfo(np.float32).tiny
    normal = expected >= tiny
    bound = 2.0 ** -8 * (1 + 2.0 ** -12) if dtype == "bf16" else 2e-5
    for select in ("classified", "naive"):
        actual, report = run_program(program, values, offsets, dtype=dtype, op="softmax", select=select)
        assert report.selected == select
        relative = np.abs(actual[normal] - expected[normal]) / expected[normal]
        print(f"{dtype} sigma {sigma} {select}: max relative error {relative.max():.3g}, "
              f"{int(normal.sum())} normal outputs, {int((actual == 0).sum())} zeros")
        assert relative.max() <= bound
        assert not np.any(actual[normal] == 0), "a normal probability came out zero"
        assert np.all(actual[rounded == 0] == 0), "an output is nonzero where the correctly rounded result is zero"
        check(actual, values, offsets, op="softmax", dtype=dtype)
