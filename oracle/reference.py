"""Float64 NumPy specification of packed ``values[N, D]`` plus ``offsets[B+1]``.

TEST INFRASTRUCTURE ONLY (see the package docstring): the checker, never the
product. Restates simon-jd/ragged-mlir ``oracle/reference.py`` and
``docs/semantics.md``. Inputs already carry their source dtype's quantization
(bf16 inputs are exact float32 values, ``quantize_bf16``); all arithmetic is
float64 so comparisons include the device's accumulation and output rounding.

Two forms of each operation exist: a vectorised one (``np.ufunc.reduceat``
over the nonempty segments, used at benchmark sizes) and a per-segment loop
(``*_loop``) that follows the reference's loop structure line by line. Tests
cross-check the two on every distribution; the loop form is the restatement,
the vectorised form is what makes million-row checks finish in seconds.
"""

from __future__ import annotations

import numpy as np

# oracle/reference.py:14 -- (rtol, atol) per input dtype.
TOLERANCES = {"f32": (2e-5, 2e-6), "bf16": (2e-2, 2e-3)}
# The build's own contract for sum and softmax: rtol 1e-5 (f32) and 1e-2
# (bf16), with the reference's absolute floor for values near zero.
STRICT_TOLERANCES = {"f32": (1e-5, 2e-6), "bf16": (1e-2, 2e-3)}


def validate_offsets(offsets: np.ndarray, n: int) -> np.ndarray:
    """Offsets contract without an N-row allocation (oracle/reference.py:17-39).

    Start at zero, nondecreasing (compared, never subtracted), inside [0, N],
    end at N; i32 or i64 contiguous; rank 1 with B+1 >= 1 entries.
    """
    offsets = np.asarray(offsets)
    if isinstance(n, (bool, np.bool_)) or not isinstance(n, (int, np.integer)) or n < 0:
        raise ValueError("N must be a nonnegative integer")
    if n > np.iinfo(np.int64).max:
        raise ValueError("N exceeds the i64 indexing range")
    if offsets.ndim != 1 or offsets.size == 0:
        raise ValueError("offsets must have rank 1 and length B+1 >= 1")
    if offsets.dtype not in (np.dtype("int32"), np.dtype("int64")):
        raise TypeError("offsets dtype must be i32 or i64")
    if not offsets.flags.c_contiguous:
        raise ValueError("offsets must be contiguous")
    if int(offsets[0]) != 0:
        raise ValueError("offsets[0] must equal 0")
    if np.any(offsets < 0) or np.any(offsets > n):
        raise ValueError("offsets must lie in [0, N]")
    if np.any(offsets[1:] < offsets[:-1]):
        raise ValueError("offsets must be nondecreasing")
    if int(offsets[-1]) != n:
        raise ValueError("offsets[-1] must equal N")
    return offsets


def _inputs(values: np.ndarray, offsets: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Shape/dtype checks of oracle/reference.py:42-52; returns float64 values."""
    values = np.asarray(values)
    if values.ndim != 2:
        raise ValueError("values must have rank 2 [N, D]")
    if not 1 <= values.shape[1] <= 1024:
        raise ValueError("D must be in [1, 1024]")
    if values.dtype.kind != "f":
        raise TypeError("values must have a real floating dtype")
    if not values.flags.c_contiguous:
        raise ValueError("values must be row-major contiguous")
    return values.astype(np.float64), validate_offsets(offsets, values.shape[0])


def quantize_bf16(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 round-to-nearest-even, as exact float32 (oracle/reference.py:55-67).

    Integer RNE on the bit pattern: add 0x7FFF plus the kept LSB, clear the low
    16 bits. NaNs map to the canonical quiet NaN so a payload cannot round to
    infinity.
    """
    values = np.asarray(values, dtype=np.float32)
    bits = values.view(np.uint32)
    nan = np.isnan(values)
    with np.errstate(over="ignore"):
        rounded = (bits + np.uint32(0x7FFF) + ((bits >> 16) & 1)) & np.uint32(0xFFFF0000)
    rounded = np.where(nan, np.uint32(0x7FC00000), rounded).astype(np.uint32)
    return rounded.view(np.float32)


def _nonempty(offsets: np.ndarray):
    lengths = np.diff(offsets.astype(np.int64))
    mask = lengths > 0
    return lengths, mask, offsets[:-1].astype(np.int64)[mask]


def segment_reduce(values: np.ndarray, offsets: np.ndarray, kind: str) -> np.ndarray:
    """Per-segment column sum or max in float64 (oracle/reference.py:70-83).

    Empty segments give +0 (sum) and -inf (max). ``np.maximum`` propagates NaN
    like ``np.max`` in the reference (fmax/nanmax would erase it); +inf plus
    -inf is NaN for the sum. ``reduceat`` over the starts of the nonempty
    segments reduces exactly each segment's rows, because an empty segment's
    start equals its neighbour's end.
    """
    if kind not in ("sum", "max"):
        raise ValueError("reduction kind must be sum or max")
    values, offsets = _inputs(values, offsets)
    b, d = len(offsets) - 1, values.shape[1]
    out = np.full((b, d), 0.0 if kind == "sum" else -np.inf, dtype=np.float64)
    _, mask, starts = _nonempty(offsets)
    if starts.size:
        ufunc = np.add if kind == "sum" else np.maximum
        with np.errstate(invalid="ignore", over="ignore"):
            out[mask] = ufunc.reduceat(values, starts, axis=0)
    return out


def segment_sum(values: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    return segment_reduce(values, offsets, "sum")


def segment_max(values: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    return segment_reduce(values, offsets, "max")


def segment_softmax(values: np.ndarray, offsets: np.ndarray) -> np.ndarray:
    """Stable per-feature softmax (oracle/reference.py:94-106).

    ``exp(x - max) / sum(exp(x - max))`` per segment and column. A column with
    NaN, +inf or only -inf becomes all NaN through ordinary IEEE arithmetic
    (inf - inf and -inf - -inf are NaN); mixed finite/-inf columns give 0 at the
    -inf entries. Empty segments store nothing.
    """
    values, offsets = _inputs(values, offsets)
    out = np.empty_like(values)
    lengths, mask, starts = _nonempty(offsets)
    if not starts.size:
        return out
    with np.errstate(invalid="ignore", over="ignore", divide="ignore", under="ignore"):
        maxima = np.maximum.reduceat(values, starts, axis=0)
        repeat = lengths[mask]
        lo, hi = int(starts[0]), int(offsets[-1])
        weights = np.exp(values[lo:hi] - np.repeat(maxima, repeat, axis=0))
        sums = np.add.reduceat(weights, starts - lo, axis=0)
        out[lo:hi] = weights / np.repeat(sums, repeat, axis=0)
    return out


# ---------------------------------------------------------------------------
# Per-segment loop forms: the reference's loop structure, for cross-checks.

def segment_sum_loop(values, offsets):
    """oracle/reference.py:76-79 loop form of the sum."""
    return _loop_reduce(values, offsets, "sum")


def segment_max_loop(values, offsets):
    """oracle/reference.py:80-82 loop form of the NaN-propagating max."""
    return _loop_reduce(values, offsets, "max")


def _loop_reduce(values, offsets, kind):
    values, offsets = _inputs(values, offsets)
    out = np.empty((len(offsets) - 1, values.shape[1]), dtype=np.float64)
    with np.errstate(invalid="ignore", over="ignore"):
        for segment, (begin, end) in enumerate(zip(offsets[:-1], offsets[1:])):
            part = values[int(begin):int(end)]
            if kind == "sum":
                out[segment] = np.sum(part, axis=0, dtype=np.float64)
            else:
                out[segment] = np.max(part, axis=0, initial=-np.inf)
    return out


def segment_softmax_loop(values, offsets):
    """oracle/reference.py:96-106 loop form of the softmax."""
    values, offsets = _inputs(values, offsets)
    out = np.empty_like(values)
    with np.errstate(invalid="ignore", over="ignore", divide="ignore", under="ignore"):
        for begin, end in zip(offsets[:-1], offsets[1:]):
            begin, end = int(begin), int(end)
            if begin == end:
                continue
            part = values[begin:end]
            weights = np.exp(part - np.max(part, axis=0))
            out[begin:end] = weights / np.sum(weights, axis=0, dtype=np.float64)
    return out


class Expectation:
    """The float64 reference of one (values, offsets, operation, dtype),
    computed once and compared with any number of outputs.

    ``check`` is the accuracy contract of oracle/reference.py:109-174 and
    docs/semantics.md:69-88 (see ``assert_matches``, which is one
    ``Expectation(...).check(...)``).
    """

    def __init__(self, values: np.ndarray, offsets: np.ndarray, *, operation: str, input_dtype: str):
        functions = {"sum": segment_sum, "max": segment_max, "softmax": segment_softmax}
        if operation not in functions:
            raise ValueError("operation must be sum, max, or softmax")
        if input_dtype not in TOLERANCES:
            raise ValueError("input_dtype must be f32 or bf16")
        self.operation, self.input_dtype = operation, input_dtype
        self.offsets = np.asarray(offsets)
        reference = functions[operation](values, offsets)
        with np.errstate(over="ignore", invalid="ignore"):
            rounded = reference.astype(np.float32)
            if input_dtype == "bf16":
                rounded = quantize_bf16(rounded)
        # Where rounding the reference to the output dtype overflows, the
        # signed infinity is expected instead.
        self.expected = np.where(np.isinf(rounded), rounded.astype(np.float64), reference)
        self.scale = segment_sum(np.abs(values), offsets) if operation == "sum" else np.abs(self.expected)
        self.finite = np.isfinite(self.expected)

    def check(self, actual: np.ndarray, tolerances: dict[str, tuple[float, float]] = TOLERANCES
              ) -> dict[str, float | int]:
        operation, input_dtype, expected, finite = self.operation, self.input_dtype, self.expected, self.finite
        if input_dtype not in tolerances:
            raise ValueError("input_dtype must be f32 or bf16")
        actual = np.asarray(actual, dtype=np.float64)
        if actual.shape != expected.shape:
            raise AssertionError(f"shape mismatch: {actual.shape} != {expected.shape}")
        if not np.array_equal(np.isnan(actual), np.isnan(expected)):
            raise AssertionError("NaN locations differ from oracle")
        if not np.array_equal(np.isposinf(actual), np.isposinf(expected)):
            raise AssertionError("positive infinity locations differ from oracle")
        if not np.array_equal(np.isneginf(actual), np.isneginf(expected)):
            raise AssertionError("negative infinity locations differ from oracle")
        rtol, atol = tolerances[input_dtype]
        error = np.abs(actual[finite] - expected[finite])
        bound = atol + rtol * self.scale[finite]
        failures = error > bound
        if np.any(failures):
            raise AssertionError(
                f"{operation}/{input_dtype}: {int(np.sum(failures))} finite values exceed "
                f"tolerance; max abs error={float(np.max(error)):.9g}")
        if operation == "softmax":
            if np.any(actual[finite] < 0) or np.any(actual[finite] > 1):
                raise AssertionError("finite softmax probabilities must lie in [0, 1]")
            offsets64 = self.offsets.astype(np.int64)
            lengths, mask, starts = _nonempty(offsets64)
            if starts.size:
                lo, hi = int(starts[0]), int(offsets64[-1])
                # Per segment and column: is every expected entry finite, and
                # the float64 column total of the actual output.
                valid = np.logical_and.reduceat(finite[lo:hi], starts - lo, axis=0)
                with np.errstate(invalid="ignore"):
                    totals = np.add.reduceat(np.where(finite, actual, 0.0)[lo:hi], starts - lo, axis=0)
                if np.any(np.abs(totals[valid] - 1) > rtol + atol):
                    raise AssertionError("finite softmax columns must sum to one within dtype tolerance")
        return {
            "finite_values": int(np.sum(finite)),
            "nan_values": int(np.sum(np.isnan(expected))),
            "max_abs_error": float(np.max(error, initial=0)),
            "max_fraction_of_tolerance": float(np.max(error / bound, initial=0)),
        }


def assert_matches(actual: np.ndarray, values: np.ndarray, offsets: np.ndarray, *,
                   operation: str, input_dtype: str,
                   tolerances: dict[str, tuple[float, float]] = TOLERANCES) -> dict[str, float | int]:
    """Accuracy contract of oracle/reference.py:109-174 and docs/semantics.md:69-88.

    * Expected values are the float64 reference; where rounding the reference
      to the output dtype overflows, the signed infinity is expected instead.
    * NaN masks and the locations of +inf and -inf must agree exactly.
    * Finite entries: ``|actual - expected| <= atol + rtol * scale``, where the
      scale is ``segment_sum(|values|)`` for sum (cancellation safe) and
      ``|expected|`` for max and softmax.
    * Softmax: finite probabilities lie in [0, 1] and every all-finite column
      of a nonempty segment sums to one within ``rtol + atol``.

    Returns the reference's error statistics. ``tolerances`` replaces the
    reference's (rtol, atol) table, e.g. with STRICT_TOLERANCES.
    """
    if input_dtype not in tolerances:
        raise ValueError("input_dtype must be f32 or bf16")
    return Expectation(values, offsets, operation=operation, input_dtype=input_dtype).check(actual, tolerances)
