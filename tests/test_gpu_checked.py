"""GPU tests of checked mode (offsets validated on the device before any
output write, docs/checked-abi.md) and of the in-place softmax (out aliases
values, ProgramSpec(alias="inplace")).

Expected diagnostics come from the CPU restatement ``oracle.offsets_errors``
(pinned in tests/test_oracle.py). Mirrors the behaviour the reference's
test/gpu/test_checked.py exercises: rejection before any write to the output
or the (in-place) input, every failed condition with its earliest index,
extreme i32/i64 endpoints, B = 0, and length hints checked even when the spec
claims checked offsets.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import check, quantized, run_program

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, Hints, ProgramSpec, ValidationError  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

D = 3
_programs = {}


def program(cache, op, offsets_dtype, strategy="auto", hints=None, inplace=False, dtype="f32", d=D):
    key = (op, offsets_dtype, strategy, hints, inplace, dtype, d)
    if key not in _programs:
        spec = ProgramSpec(op, dtype, d, offsets_dtype, hints=hints or Hints(), strategy=strategy,
                           alias="inplace" if inplace else "none")
        _programs[key] = Compiler().compile(spec, cache)
    return _programs[key]


def assert_rejected(prog, offsets, n):
    """The checked call raises with the oracle's diagnostics and writes
    neither the output nor the values."""
    spec = prog.spec
    hints = spec.hints
    expected = oracle.offsets_errors(offsets, n, hints.min_len, hints.max_len)
    assert expected, "a negative case needs an expected violation"
    device = torch.device("cuda", 0)
    tdtype = torch.bfloat16 if spec.dtype == "bf16" else torch.float32
    values = (torch.arange(n * spec.feature_dim, device=device, dtype=torch.float32) / 8)
    values = values.reshape(n, spec.feature_dim).to(tdtype)
    original = values.clone()
    off = torch.tensor(offsets, device=device, dtype=torch.int32 if spec.offsets_dtype == "i32" else torch.int64)
    rows = n if spec.op == "softmax" else len(offsets) - 1
    guard = torch.full((rows + 2, spec.feature_dim), -64, device=device, dtype=tdtype)
    out = values if spec.alias == "inplace" else guard[1:-1]
    with pytest.raises(ValidationError) as caught:
        prog.run(values, off, out, mode="checked")
    error = caught.value
    assert error.errors == expected
    assert (error.condition, error.index) == next(iter(expected.items()))
    for condition, index in expected.items():
        assert f"{condition} at index {index}" in str(error)
    torch.cuda.synchronize()
    assert torch.equal(values, original), "the input (or in-place output) changed"
    assert bool(torch.all(guard == -64)), "the output or its guard was written"


INVALID = {"first": [1, 4, 8], "final": [0, 4, 7], "negative": [0, -1, 8], "above_n": [0, 9, 8],
           "nonmonotone": [0, 4, 3, 8]}


@pytest.mark.parametrize("case", sorted(INVALID))
@pytest.mark.parametrize("strategy", ["auto", "naive"])
@pytest.mark.parametrize("offsets_dtype", ["i32", "i64"])
@pytest.mark.parametrize("op", ["sum", "max", "softmax"])
def test_invalid_offsets_rejected_before_output(artifact_cache, op, offsets_dtype, strategy, case):
    assert_rejected(program(artifact_cache, op, offsets_dtype, strategy), INVALID[case], 8)


@pytest.mark.parametrize("offsets_dtype", ["i32", "i64"])
@pytest.mark.parametrize("op", ["sum", "softmax"])
def test_every_condition_with_its_earliest_index(artifact_cache, op, offsets_dtype):
    hints = Hints(min_len=4, max_len=4, offsets_checked=True)
    offsets = [1, -2, -3, 11, 10, 0, 1, 7, 6]
    assert len(oracle.offsets_errors(offsets, 8, 4, 4)) == 7
    assert_rejected(program(artifact_cache, op, offsets_dtype, "naive", hints), offsets, 8)


@pytest.mark.parametrize("offsets_dtype", ["i32", "i64"])
@pytest.mark.parametrize("claimed", [False, True])
def test_length_hints_checked_even_when_claimed(artifact_cache, offsets_dtype, claimed):
    hints = Hints(min_len=3, max_len=50, offsets_checked=claimed)
    offsets = [0, 2, 2 + 51, 2 + 51 + 10]
    assert oracle.offsets_errors(offsets, offsets[-1], 3, 50) == {"below_min_len": 0, "above_max_len": 1}
    assert_rejected(program(artifact_cache, "sum", offsets_dtype, "auto", hints), offsets, offsets[-1])


@pytest.mark.parametrize("offsets_dtype", ["i32", "i64"])
@pytest.mark.parametrize("op", ["max", "softmax"])
def test_extreme_endpoints_do_not_overflow(artifact_cache, op, offsets_dtype):
    bits = 32 if offsets_dtype == "i32" else 64
    lo, hi = -(1 << (bits - 1)), (1 << (bits - 1)) - 1
    hints = Hints(min_len=9, max_len=100, offsets_checked=True)
    assert_rejected(program(artifact_cache, op, offsets_dtype, "auto", hints), [0, lo, hi, 0, 8], 8)


@pytest.mark.parametrize("n,offsets", [(0, [1]), (0, [-1]), (2, [0]), (2, [2])])
def test_zero_segments_still_check_the_offset(artifact_cache, n, offsets):
    assert_rejected(program(artifact_cache, "sum", "i64"), offsets, n)


@pytest.mark.parametrize("strategy", ["auto", "naive"])
def test_invalid_inplace_softmax_keeps_the_values(artifact_cache, strategy):
    assert_rejected(program(artifact_cache, "softmax", "i64", strategy, inplace=True), [0, 4, 3, 8], 8)


@pytest.mark.parametrize("op,dtype,d", [("sum", "f32", 3), ("max", "bf16", 128), ("softmax", "bf16", 128),
                                        ("softmax", "f32", 1)])
def test_valid_offsets_pass_checked_mode(artifact_cache, op, dtype, d):
    """Checked mode on valid offsets (with satisfied hints) computes the same
    exact results as validated mode and reports the two check kernels first."""
    hints = Hints(min_len=0, max_len=5000)
    prog = program(artifact_cache, op, "i64", "auto", hints, dtype=dtype, d=d)
    lengths = make_lengths("long_tail", 300, seed=4, total_elements=60_000 // d + 400)
    lengths = np.minimum(lengths, 5000)
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(9).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    actual, report = run_program(prog, values, offsets, dtype=dtype, op=op, mode="checked")
    check(actual, values, offsets, op=op, dtype=dtype)
    assert report.kernel_names[:2] == ("ragged_0_offsets_init", "ragged_0_offsets_check")


@pytest.mark.parametrize("select", ["classified", "naive"])
@pytest.mark.parametrize("dtype,d", [("f32", 1), ("f32", 128), ("bf16", 128), ("bf16", 8), ("f32", 1024)])
def test_inplace_softmax(artifact_cache, dtype, d, select):
    """out is values: every row is read before it is overwritten with its
    softmax, in both schedules (including chunked segments of the register-
    resident worker, whose rows are re-read by nobody after the store)."""
    prog = program(artifact_cache, "softmax", "i64", "auto", inplace=True, dtype=dtype, d=d)
    lengths = make_lengths("long_tail", 200, seed=11, total_elements=max(2000, 400_000 // d))
    lengths[::9] = 0
    offsets = offsets_from_lengths(lengths, "i64")
    values = np.random.default_rng(12).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    device = torch.device("cuda", 0)
    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.from_numpy(values).to(device).to(tdtype).contiguous()
    off = torch.from_numpy(offsets).to(device)
    for mode in ("validated", "checked"):
        y = x.clone()
        report = prog.run(y, off, y, select=select, mode=mode)
        torch.cuda.synchronize()
        assert report.selected == select
        check(y.float().cpu().numpy().astype(np.float64), quantized(values, dtype), offsets, op="softmax",
              dtype=dtype)
