"""The allocation-free entry point ``rg_run_static`` against ``rg_run``.

``rg_run_static`` runs a plan on the library's static per-device workspace
(no caller workspace, no allocation). Through the C ABI, for the classified
schedule of every worker kind (register-resident softmax with chunk merges,
the streaming worker's reductions and split softmax), two calls in a row --
the second on a smaller input, so the static array holds the first call's
counters and tables -- must give the same bits as ``rg_run`` with a fresh
caller workspace, and pass the oracle. A plan larger than the static
workspace is rejected before anything is launched.
"""
from __future__ import annotations

import numpy as np
import pytest

from gpu_helpers import check

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import ValidationError, native  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

DEVICE = torch.device("cuda", 0)

CASES = [
    # op, dtype, D, offsets dtype, distribution, rows of the first and second call
    ("softmax", "bf16", 128, "i64", "long_tail", 150_000, 40_000),
    ("sum", "f32", 1, "i64", "long_tail", 800_000, 90_000),
    ("max", "f32", 128, "i32", "burst", 60_000, 9_000),
    ("softmax", "f32", 2, "i32", "burst", 400_000, 70_000),
]


def inputs(distribution, rows, d, offsets_dtype, seed):
    lengths = make_lengths(distribution, 400, seed=seed, total_elements=rows)
    offsets = offsets_from_lengths(lengths, offsets_dtype)
    values = np.random.default_rng(seed + 1).normal(size=(rows, d)).astype(np.float32)
    return values, offsets


@pytest.mark.parametrize("op,dtype,d,offsets_dtype,distribution,first,second", CASES)
def test_static_workspace_matches_rg_run(op, dtype, d, offsets_dtype, distribution, first, second):
    spec = native.make_spec(op, dtype, offsets_dtype, d)
    module = native.NativeModule(0, spec)
    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
    view = torch.int16 if dtype == "bf16" else torch.int32
    stream = torch.cuda.current_stream().cuda_stream
    for call, rows in enumerate((first, second)):
        values, offsets = inputs(distribution, rows, d, offsets_dtype, seed=60 + call)
        b = len(offsets) - 1
        plan = module.plan(rows, b, "classified")
        assert 0 < plan.workspace_bytes <= native.STATIC_WORKSPACE_BYTES
        x = torch.from_numpy(values).to(DEVICE).to(tdtype)
        off = torch.from_numpy(offsets).to(DEVICE)
        out_rows = rows if op == "softmax" else b
        expected = torch.full((out_rows, d), float("nan"), dtype=tdtype, device=DEVICE)
        actual = torch.full_like(expected, float("nan"))
        workspace = torch.zeros((int(plan.workspace_bytes),), dtype=torch.uint8, device=DEVICE)
        module.run(plan, x.data_ptr(), off.data_ptr(), expected.data_ptr(), None, workspace.data_ptr(),
                   int(plan.workspace_bytes), stream)
        module.run_static(plan, x.data_ptr(), off.data_ptr(), actual.data_ptr(), None, stream)
        torch.cuda.synchronize()
        assert torch.equal(actual.view(view), expected.view(view)), f"call {call}: rg_run_static differs from rg_run"
        check(actual.float().cpu().numpy().astype(np.float64), values, offsets, op=op, dtype=dtype)
    module.close()


def test_plan_beyond_the_static_workspace_is_rejected():
    """A plan needing more than RG_STATIC_WORKSPACE_BYTES fails with a
    workspace error before any launch: the output keeps its contents."""
    spec = native.make_spec("sum", "f32", "i64", 1024)
    module = native.NativeModule(0, spec)
    rows, b = 2_000_000, 4
    plan = module.plan(rows, b, "classified")
    assert plan.workspace_bytes > native.STATIC_WORKSPACE_BYTES
    values = torch.zeros((8, 1024), device=DEVICE)      # never read: the call is rejected on the host
    offsets = torch.zeros((b + 1,), dtype=torch.int64, device=DEVICE)
    out = torch.full((b, 1024), 7.0, device=DEVICE)
    with pytest.raises(ValidationError, match="static workspace holds at most"):
        module.run_static(plan, values.data_ptr(), offsets.data_ptr(), out.data_ptr(), None,
                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert bool(torch.all(out == 7.0))
    module.close()


@pytest.mark.parametrize("op,dtype,d,offsets_dtype,distribution,first,second", CASES[:2])
def test_static_call_interrupted_after_a_launch_recovers(op, dtype, d, offsets_dtype, distribution, first, second):
    """A static call that fails after its first launch (the classification
    ran and counted; nothing returned the counters to zero) leaves the
    device's static workspace marked. The next static call first returns
    the counters to zero with a one-workgroup kernel: its result equals
    rg_run's on a fresh workspace, bit for bit."""
    spec = native.make_spec(op, dtype, offsets_dtype, d)
    module = native.NativeModule(0, spec)
    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
    view = torch.int16 if dtype == "bf16" else torch.int32
    stream = torch.cuda.current_stream().cuda_stream
    values, offsets = inputs(distribution, first, d, offsets_dtype, seed=71)
    b = len(offsets) - 1
    plan = module.plan(first, b, "classified")
    x = torch.from_numpy(values).to(DEVICE).to(tdtype)
    off = torch.from_numpy(offsets).to(DEVICE)
    out_rows = first if op == "softmax" else b
    expected = torch.full((out_rows, d), float("nan"), dtype=tdtype, device=DEVICE)
    actual = torch.full_like(expected, float("nan"))
    native.interrupt_static(1)
    try:
        with pytest.raises(RuntimeError, match="interrupted after 1 launches"):
            module.run_static(plan, x.data_ptr(), off.data_ptr(), actual.data_ptr(), None, stream)
    finally:
        native.interrupt_static(-1)
    torch.cuda.synchronize()
    workspace = torch.zeros((int(plan.workspace_bytes),), dtype=torch.uint8, device=DEVICE)
    module.run(plan, x.data_ptr(), off.data_ptr(), expected.data_ptr(), None, workspace.data_ptr(),
               int(plan.workspace_bytes), stream)
    for _ in range(2):
        actual.fill_(float("nan"))
        module.run_static(plan, x.data_ptr(), off.data_ptr(), actual.data_ptr(), None, stream)
        torch.cuda.synchronize()
        assert torch.equal(actual.view(view), expected.view(view)), "a static call after the failed one differs"
    check(actual.float().cpu().numpy().astype(np.float64), values, offsets, op=op, dtype=dtype)
    module.close()
