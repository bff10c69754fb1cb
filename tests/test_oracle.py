"""Oracle pinning (CPU). Known answers restated from the reference's
test/python/test_oracle.py, plus cross-checks that a plausible mistake in the
restatement (a dropped term, wrong sign or index, a transposed operand)
fails: loop vs vectorised forms, math.fsum brute force, closed forms and
invariants, and torch's own bf16 rounding."""
from __future__ import annotations

import ast
import math
from pathlib import Path

import numpy as np
import pytest

import oracle
from oracle import (assert_matches, masked_logits, quantize_bf16, segment_max, segment_max_loop, segment_reduce,
                    segment_softmax, segment_softmax_loop, segment_sum, segment_sum_loop, validate_offsets)
from ragged.workloads import make_lengths, offsets_from_lengths


@pytest.mark.parametrize("index_dtype", [np.int32, np.int64])
def test_hand_calculated_reductions_and_softmax(index_dtype):
    # reference test_oracle.py:15-22
    values = np.array([[1, 2], [3, 4], [-2, 7]], dtype=np.float32)
    offsets = np.array([0, 2, 2, 3], dtype=index_dtype)
    np.testing.assert_array_equal(segment_sum(values, offsets), [[4, 6], [0, 0], [-2, 7]])
    np.testing.assert_array_equal(segment_max(values, offsets), [[3, 4], [-np.inf, -np.inf], [-2, 7]])
    low = 1 / (1 + np.exp(2))
    np.testing.assert_allclose(segment_softmax(values, offsets), [[low, low], [1 - low, 1 - low], [1, 1]])


@pytest.mark.parametrize("offsets", [[0], [0, 0], [0, 0, 0, 0]])
@pytest.mark.parametrize("d", [1, 3, 16, 128, 1024])
def test_empty_and_all_empty(offsets, d):
    # reference test_oracle.py:25-34
    values = np.empty((0, d), dtype=np.float32)
    offsets = np.array(offsets, dtype=np.int64)
    sums, maxima, softmax = segment_sum(values, offsets), segment_max(values, offsets), segment_softmax(values, offsets)
    assert sums.shape == maxima.shape == (len(offsets) - 1, d)
    assert softmax.shape == (0, d)
    assert np.all(sums == 0) and not np.any(np.signbit(sums))
    assert np.all(np.isneginf(maxima))


def test_nonfinite_is_per_feature_and_nan_propagates():
    # reference test_oracle.py:37-46
    values = np.array([[np.nan, np.inf, -np.inf, -np.inf, 1],
                       [1, 1, -np.inf, 3, 2]], dtype=np.float32)
    offsets = np.array([0, 2], dtype=np.int32)
    np.testing.assert_array_equal(segment_sum(values, offsets), [[np.nan, np.inf, -np.inf, -np.inf, 3]])
    np.testing.assert_array_equal(segment_max(values, offsets), [[np.nan, np.inf, -np.inf, 3, 2]])
    actual = segment_softmax(values, offsets)
    assert np.all(np.isnan(actual[:, :3]))
    np.testing.assert_array_equal(actual[:, 3], [0, 1])
    np.testing.assert_allclose(actual[:, 4], [1 / (1 + np.e), np.e / (1 + np.e)])


def test_opposite_infinities_sum_to_nan():
    # reference test_oracle.py:49-56
    values = np.array([[np.inf], [-np.inf]], dtype=np.float32)
    offsets = np.array([0, 2], dtype=np.int32)
    assert np.isnan(segment_sum(values, offsets)[0, 0])
    assert np.isposinf(segment_max(values, offsets)[0, 0])
    assert np.all(np.isnan(segment_softmax(values, offsets)))


@pytest.mark.parametrize("raw,n,condition", [
    ([1, 3], 3, r"offsets\[0\]"),
    ([0, 3, 2, 3], 3, "nondecreasing"),
    ([0, 2], 3, r"offsets\[-1\]"),
    ([0, -1, 3], 3, r"\[0, N\]"),
    ([0, 4, 3], 3, r"\[0, N\]"),
    ([], 0, "length"),
])
@pytest.mark.parametrize("dtype", [np.int32, np.int64])
def test_invalid_offsets(raw, n, condition, dtype):
    # reference test_oracle.py:59-70
    with pytest.raises(ValueError, match=condition):
        validate_offsets(np.array(raw, dtype=dtype), n)


@pytest.mark.parametrize("offsets", [np.array([0, 1.0]), np.array([0, 1], dtype=np.uint32),
                                     np.array([0, 1], dtype=np.int16)])
def test_offset_dtype(offsets):
    with pytest.raises(TypeError, match="i32 or i64"):
        validate_offsets(offsets, 1)


def test_offset_limits_without_giant_allocation():
    # reference test_oracle.py:79-87
    max32, max64 = np.iinfo(np.int32).max, np.iinfo(np.int64).max
    validate_offsets(np.array([0, max32 - 1, max32], dtype=np.int32), int(max32))
    validate_offsets(np.array([0, max32, max32 + 1], dtype=np.int64), int(max32) + 1)
    validate_offsets(np.array([0, max64], dtype=np.int64), int(max64))
    with pytest.raises(ValueError, match="nondecreasing"):
        validate_offsets(np.array([0, max64, 1, max64], dtype=np.int64), int(max64))
    with pytest.raises(ValueError, match="i64 indexing"):
        validate_offsets(np.array([0], dtype=np.int64), int(max64) + 1)


@pytest.mark.parametrize("values,condition", [
    (np.zeros(2, dtype=np.float32), "rank 2"),
    (np.zeros((1, 0), dtype=np.float32), "D must"),
    (np.zeros((1, 1025), dtype=np.float32), "D must"),
    (np.zeros((2, 3), dtype=np.float32).T, "contiguous"),
])
def test_invalid_values(values, condition):
    with pytest.raises(ValueError, match=condition):
        segment_sum(values, np.array([0, values.shape[0]], dtype=np.int32))


def test_reject_invalid_kind_and_noncontiguous_offsets():
    with pytest.raises(ValueError, match="sum or max"):
        segment_reduce(np.zeros((1, 1), dtype=np.float32), np.array([0, 1], dtype=np.int32), "mean")
    with pytest.raises(ValueError, match="contiguous"):
        validate_offsets(np.array([0, 9, 2, 9], dtype=np.int32)[::2], 2)


def test_bf16_round_ties_even_and_nonfinite():
    # reference test_oracle.py:111-118
    values = np.array([1 + 2**-8, 1 + 3 * 2**-8, np.inf, -np.inf, np.nan, -0.0], dtype=np.float32)
    actual = quantize_bf16(values)
    np.testing.assert_array_equal(actual[:4], [1, 1 + 2**-6, np.inf, -np.inf])
    assert np.isnan(actual[4]) and np.signbit(actual[5])
    tiny_payload = np.array([0x7F800001], dtype=np.uint32).view(np.float32)
    assert np.isnan(quantize_bf16(tiny_payload)[0])


def test_bf16_matches_torch_rounding_exhaustively_on_a_sample():
    """Integer RNE == torch's float32 -> bfloat16 conversion (the device path
    and the test inputs both use it) on 2^22 bit patterns incl. ties."""
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    bits = np.concatenate([rng.integers(0, 2**32, 2**22, dtype=np.uint64).astype(np.uint32),
                           (np.arange(2**16, dtype=np.uint32) << 16) | 0x8000,      # exact ties
                           (np.arange(2**16, dtype=np.uint32) << 16) | 0x7FFF])
    values = bits.view(np.float32)
    finite = np.isfinite(values)
    ours = quantize_bf16(values)[finite]
    theirs = torch.from_numpy(values[finite].copy()).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(ours.view(np.uint32), theirs.view(np.uint32))


@pytest.mark.parametrize("d", [1, 3, 16, 127, 128, 1024])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_finite_softmax_normalization_extremes(d, dtype):
    # reference test_oracle.py:121-133
    rng = np.random.default_rng(8723)
    values = rng.normal(size=(259, d)).astype(np.float32) * 1000
    if dtype == "bf16":
        values = quantize_bf16(values)
    offsets = np.array([0, 0, 1, 258, 259], dtype=np.int64)
    actual = segment_softmax(values, offsets)
    assert np.all(np.isfinite(actual)) and np.all(actual >= 0) and np.all(actual <= 1)
    for start, end in zip(offsets[:-1], offsets[1:]):
        if start != end:
            np.testing.assert_allclose(actual[start:end].sum(axis=0), 1, atol=1e-14)


@pytest.mark.parametrize("operation", [segment_sum, segment_max, segment_softmax])
def test_segment_permutation_and_empty_insertion(operation):
    # reference test_oracle.py:136-150
    rng = np.random.default_rng(9289)
    values = rng.normal(size=(12, 5)).astype(np.float32)
    offsets = np.array([0, 2, 7, 7, 12], dtype=np.int64)
    pieces = [values[a:b] for a, b in zip(offsets[:-1], offsets[1:])]
    permutation = [3, 0, 2, 1]
    permuted_values = np.concatenate([pieces[i] for i in permutation])
    permuted_offsets = np.array([0, *np.cumsum([len(pieces[i]) for i in permutation])], dtype=np.int64)
    original = operation(values, offsets)
    expected = (np.concatenate([original[offsets[i]:offsets[i + 1]] for i in permutation])
                if operation == segment_softmax else original[permutation])
    np.testing.assert_array_equal(operation(permuted_values, permuted_offsets), expected)
    expanded = np.array([0, 0, 2, 7, 7, 12, 12], dtype=np.int64)
    actual = operation(values, expanded)
    np.testing.assert_array_equal(actual if operation == segment_softmax else actual[1:5], original)


def test_split_segment_sum_and_softmax_shift_invariance():
    # reference test_oracle.py:153-159
    rng = np.random.default_rng(773)
    values = rng.normal(size=(129, 7))
    original = np.array([0, 129], dtype=np.int64)
    split = np.array([0, 31, 129], dtype=np.int64)
    np.testing.assert_allclose(segment_sum(values, original)[0], segment_sum(values, split).sum(axis=0), atol=1e-13)
    np.testing.assert_allclose(segment_softmax(values, original), segment_softmax(values + 13, original),
                               rtol=1e-13, atol=1e-15)


def test_tolerance_accepts_rounding_but_rejects_wrong_results_and_nan():
    # reference test_oracle.py:162-172
    values = np.array([[1], [2]], dtype=np.float32)
    offsets = np.array([0, 2], dtype=np.int32)
    stats = assert_matches(np.array([[3.000001]]), values, offsets, operation="sum", input_dtype="f32")
    assert stats["finite_values"] == 1 and stats["max_abs_error"] > 0
    with pytest.raises(AssertionError, match="exceed tolerance"):
        assert_matches(np.array([[4]]), values, offsets, operation="sum", input_dtype="f32")
    with pytest.raises(AssertionError, match="NaN"):
        assert_matches(np.array([[np.nan]]), values, offsets, operation="sum", input_dtype="f32")
    with pytest.raises(AssertionError, match="shape"):
        assert_matches(np.array([3]), values, offsets, operation="sum", input_dtype="f32")


def test_tolerance_is_cancellation_safe():
    values = np.array([[1e8], [1], [-1e8]], dtype=np.float32)
    assert_matches(np.array([[0]]), values, np.array([0, 3], dtype=np.int32), operation="sum", input_dtype="f32")


def test_output_dtype_overflow_is_distinguished_from_bad_infinities():
    # reference test_oracle.py:180-185
    values = np.array([[3e38], [3e38]], dtype=np.float32)
    offsets = np.array([0, 2], dtype=np.int32)
    assert_matches(np.array([[np.inf]]), values, offsets, operation="sum", input_dtype="f32")
    with pytest.raises(AssertionError, match="positive infinity"):
        assert_matches(np.array([[np.inf]]), np.ones((2, 1), dtype=np.float32), offsets, operation="sum",
                       input_dtype="f32")


def test_single_very_long_segment():
    # reference test_oracle.py:188-193
    values = np.tile(np.array([[1, -1, 0.5]], dtype=np.float32), (131073, 1))
    offsets = np.array([0, 131073], dtype=np.int64)
    np.testing.assert_array_equal(segment_sum(values, offsets), [[131073, -131073, 65536.5]])
    np.testing.assert_array_equal(segment_max(values, offsets), [[1, -1, 0.5]])
    np.testing.assert_allclose(segment_softmax(values, offsets), np.full(values.shape, 1 / 131073), rtol=1e-14)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_softmax_absolute_tolerance_cannot_accept_all_zero_long_segment(dtype):
    # reference test_oracle.py:196-200
    values = np.zeros((1_000_000, 1), dtype=np.float32)
    with pytest.raises(AssertionError, match="sum to one"):
        assert_matches(np.zeros_like(values), values, np.array([0, len(values)], dtype=np.int64),
                       operation="softmax", input_dtype=dtype)


def test_softmax_probability_range_is_enforced():
    # Within the bf16 bound of the expected 1.0 but not a probability.
    values = np.array([[0.0]], dtype=np.float32)
    with pytest.raises(AssertionError, match=r"\[0, 1\]"):
        assert_matches(np.array([[1.005]]), values, np.array([0, 1], dtype=np.int64),
                       operation="softmax", input_dtype="bf16")


# --- cross-checks that pin the vectorised forms -------------------------------

@pytest.mark.parametrize("distribution", ["uniform", "long_tail", "bimodal", "burst", "exponential"])
def test_vectorised_equals_loop_restatement(distribution):
    lengths = make_lengths(distribution, 300, seed=4, total_elements=9000)
    lengths[::7] = 0
    offsets = offsets_from_lengths(lengths, "i64")
    rng = np.random.default_rng(4)
    values = rng.normal(size=(int(offsets[-1]), 3)).astype(np.float32)
    values[rng.random(values.shape) < 0.002] = np.nan
    values[rng.random(values.shape) < 0.002] = -np.inf
    values[rng.random(values.shape) < 0.001] = np.inf
    np.testing.assert_allclose(segment_sum(values, offsets), segment_sum_loop(values, offsets), rtol=1e-13,
                               equal_nan=True)
    np.testing.assert_array_equal(segment_max(values, offsets), segment_max_loop(values, offsets))
    np.testing.assert_allclose(segment_softmax(values, offsets), segment_softmax_loop(values, offsets),
                               rtol=1e-12, atol=1e-300, equal_nan=True)


def test_sum_brute_force_fsum():
    rng = np.random.default_rng(21)
    values = (rng.normal(size=(400, 2)) * 10.0 ** rng.integers(-8, 8, size=(400, 2))).astype(np.float32)
    offsets = np.array([0, 5, 5, 130, 399, 400], dtype=np.int32)
    actual = segment_sum(values, offsets)
    for s, (a, b) in enumerate(zip(offsets[:-1], offsets[1:])):
        for f in range(2):
            expected = math.fsum(float(x) for x in values[a:b, f])
            assert abs(actual[s, f] - expected) <= 1e-12 * max(1.0, math.fsum(abs(float(x)) for x in values[a:b, f]))


def test_softmax_closed_forms():
    # Constant segment -> uniform 1/L; two values -> logistic; a dominant
    # value takes (almost) all the mass; feature columns are independent.
    values = np.zeros((10, 2), dtype=np.float32)
    values[:, 1] = np.arange(10)
    values[3, 0] = 0.0
    out = segment_softmax(values, np.array([0, 7, 10], dtype=np.int64))
    np.testing.assert_allclose(out[:7, 0], 1 / 7, rtol=1e-15)
    weights = np.exp(np.arange(7) - 6.0)
    np.testing.assert_allclose(out[:7, 1], weights / weights.sum(), rtol=1e-14)
    np.testing.assert_allclose(out[7:, 1], np.exp([-2, -1, 0]) / np.exp([-2, -1, 0]).sum(), rtol=1e-14)


def test_masked_logits_are_two_rounded_f32_operations():
    values = np.array([[1.0, 3.0e38, -np.inf]], dtype=np.float32)
    mask = np.array([[2.0 ** -30, 3.0e38, -np.inf]], dtype=np.float32)
    out = masked_logits(values, mask, scale=3.0)
    assert out.dtype == np.float32
    assert out[0, 0] == np.float32(3.0) + np.float32(2.0 ** -30)       # rounds back to 3
    assert np.isposinf(out[0, 1])                                        # f32 overflow
    assert np.isneginf(out[0, 2])
    with pytest.raises(ValueError, match="exactly"):
        masked_logits(values, mask[:, :2])
    with pytest.raises(ValueError, match="finite"):
        masked_logits(values, mask, scale=float("inf"))


def test_oracle_does_not_import_product_or_torch():
    for source in Path(oracle.__file__).parent.glob("*.py"):
        for node in ast.walk(ast.parse(source.read_text())):
            if isinstance(node, ast.Import):
                names = [alias.name for alias in node.names]
            elif isinstance(node, ast.ImportFrom):
                names = [node.module or ""]
            else:
                continue
            assert all(name.split(".")[0] not in {"ragged", "torch", "triton"} for name in names)


def test_strict_tolerance_table_is_tighter_and_rejects_what_it_should():
    """The build's bar (rtol 1e-5 f32, 1e-2 bf16) accepts a 5e-6 relative
    error on f32 and rejects 1.5e-5, which the reference's 2e-5 accepts."""
    values = np.array([[1.0], [2.0], [3.0]], dtype=np.float32)
    offsets = np.array([0, 3], dtype=np.int64)
    for dtype in ("f32", "bf16"):
        assert oracle.STRICT_TOLERANCES[dtype][0] < oracle.TOLERANCES[dtype][0]
    ok = np.array([[6.0 * (1 + 5e-6)]])
    oracle.assert_matches(ok, values, offsets, operation="sum", input_dtype="f32",
                          tolerances=oracle.STRICT_TOLERANCES)
    off = np.array([[6.0 * (1 + 1.5e-5)]])
    oracle.assert_matches(off, values, offsets, operation="sum", input_dtype="f32")
    with pytest.raises(AssertionError):
        oracle.assert_matches(off, values, offsets, operation="sum", input_dtype="f32",
                              tolerances=oracle.STRICT_TOLERANCES)


# ---------------------------------------------------------------------------
# Checked-mode offsets conditions (oracle/offsets.py).

def test_offsets_errors_known_answer():
    """The reference's all-conditions case (test/gpu/test_checked.py:125-130):
    N = 8, min_len = max_len = 4."""
    from oracle import CONDITIONS, offsets_errors
    errors = offsets_errors([1, -2, -3, 11, 10, 0, 1, 7, 6], 8, 4, 4)
    assert errors == dict(zip(CONDITIONS, [0, 8, 1, 3, 0, 5, 6]))
    assert list(errors) == list(CONDITIONS)         # slot order


def test_offsets_errors_single_conditions():
    from oracle import offsets_errors
    assert offsets_errors([0, 4, 8], 8) == {}
    assert offsets_errors([1, 4, 8], 8) == {"first_nonzero": 0}
    assert offsets_errors([0, 4, 7], 8) == {"final_mismatch": 2}
    assert offsets_errors([0, -1, 8], 8) == {"negative": 1, "nonmonotone": 0}
    assert offsets_errors([0, 9, 8], 8) == {"above_n": 1, "nonmonotone": 1}
    assert offsets_errors([0, 4, 3, 8], 8) == {"nonmonotone": 1}
    # B = 0: the only offset is both the first and the final one.
    assert offsets_errors([1], 0) == {"first_nonzero": 0, "final_mismatch": 0, "above_n": 0}
    assert offsets_errors([0], 2) == {"final_mismatch": 0}
    # Hints apply only to in-range monotone segments; the extreme pair is
    # never subtracted (it would overflow in i64).
    lo, hi = -(1 << 63), (1 << 63) - 1
    assert offsets_errors([0, lo, hi, 0, 8], 8, 9, 8) == {
        "negative": 1, "above_n": 2, "nonmonotone": 0, "below_min_len": 3}


def test_offsets_errors_brute_force():
    """Against an independent formulation on random small offsets: scan the
    pairs and offsets in index order and keep the first hit per condition."""
    from oracle import offsets_errors
    rng = np.random.default_rng(5)
    for _ in range(3000):
        b = int(rng.integers(0, 6))
        n = int(rng.integers(0, 9))
        offsets = [int(v) for v in rng.integers(-3, 12, size=b + 1)]
        min_len = None if rng.random() < 0.3 else int(rng.integers(0, 5))
        max_len = None if rng.random() < 0.3 else int(rng.integers(0, 6))
        expected = {}
        checks = [("first_nonzero", [0] if offsets[0] != 0 else []),
                  ("final_mismatch", [b] if offsets[-1] != n else []),
                  ("negative", [i for i in range(b + 1) if offsets[i] < 0]),
                  ("above_n", [i for i in range(b + 1) if offsets[i] > n]),
                  ("nonmonotone", [i for i in range(b) if offsets[i + 1] < offsets[i]])]
        valid = [i for i in range(b) if 0 <= offsets[i] <= offsets[i + 1] <= n]
        checks.append(("below_min_len", [i for i in valid if min_len is not None
                                         and offsets[i + 1] - offsets[i] < min_len]))
        checks.append(("above_max_len", [i for i in valid if max_len is not None
                                         and offsets[i + 1] - offsets[i] > max_len]))
        for name, hits in checks:
            if hits:
                expected[name] = hits[0]
        assert offsets_errors(offsets, n, min_len, max_len) == expected
