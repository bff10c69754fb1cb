"""Deterministic synthetic segment lengths and values.

Restates simon-jd/ragged-mlir ``bench/distributions.py`` (length
distributions with exact integer allocation to a fixed N) and the value
generation of ``bench/run.py:51-65``, and defines the five measured
configurations (C1-C5) this package is benchmarked on. NumPy only; no torch.

``allocate``, ``make_lengths``, ``offsets_from_lengths`` and ``describe``
follow the reference's algorithm step for step (they must reproduce its
recorded inputs bit for bit): Copyright (c) 2026 Junrui Duan, MIT License
(NOTICE.md).
"""
from __future__ import annotations

from dataclasses import dataclass, field
import hashlib

import numpy as np

DISTRIBUTIONS = ("uniform", "long_tail", "bimodal", "burst", "exponential")


def allocate(weights: np.ndarray, total_elements: int) -> np.ndarray:
    """Largest-remainder integer allocation of ``total_elements`` rows
    proportionally to ``weights`` (bench/distributions.py:54-64).

    Weights become integer units ``max(1, rint(w * 1024))``; each segment gets
    ``floor(units * total / sum(units))`` and the remainder goes one row each
    to the largest fractional parts, ties to the lower index. Python integers
    keep N exact beyond float64's integer range.
    """
    units = np.maximum(1, np.rint(np.asarray(weights, dtype=np.float64) * 1024).astype(np.int64))
    denominator = sum(map(int, units))
    numerators = [int(unit) * total_elements for unit in units]
    lengths = [numerator // denominator for numerator in numerators]
    remainder = total_elements - sum(lengths)
    order = sorted(range(len(units)), key=lambda i: (-(numerators[i] % denominator), i))
    for i in order[:remainder]:
        lengths[i] += 1
    return np.asarray(lengths, dtype=np.int64)


def make_lengths(distribution: str, segments: int, *, seed: int = 0,
                 total_elements: int | None = None, mean_length: int = 64) -> np.ndarray:
    """Segment lengths of a named distribution (bench/distributions.py:15-64).

    uniform: equal weights; long_tail: Pareto(1.3)+1 capped at 1e5; bimodal:
    4 or 1024 (90/10); exponential: Exp(1); burst: ones with 1% of consecutive
    segments at 16384. With ``total_elements`` the weights are allocated to
    exactly that N, otherwise each length is ``floor(weight * mean_length)``.
    """
    if distribution not in DISTRIBUTIONS:
        raise ValueError(f"distribution must be one of {DISTRIBUTIONS}")
    for name, value in (("segments", segments), ("seed", seed), ("mean_length", mean_length)):
        if type(value) is not int or not 0 <= value <= 2**63 - 1:
            raise ValueError(f"{name} must be a nonnegative signed-64 integer")
    if total_elements is not None and (type(total_elements) is not int or not 0 <= total_elements <= 2**63 - 1):
        raise ValueError("total_elements must be a nonnegative signed-64 integer")
    if segments == 0:
        if total_elements not in (None, 0):
            raise ValueError("nonzero elements cannot belong to zero segments")
        return np.zeros(0, dtype=np.int64)
    rng = np.random.default_rng(seed)
    if distribution == "uniform":
        weights = np.ones(segments)
    elif distribution == "long_tail":
        weights = np.minimum(rng.pareto(1.3, segments) + 1, 100000.0)
    elif distribution == "bimodal":
        weights = np.where(rng.random(segments) < 0.9, 4.0, 1024.0)
    elif distribution == "exponential":
        weights = rng.exponential(1.0, segments)
    else:
        weights = np.ones(segments)
        width = max(1, segments // 100)
        start = int(rng.integers(segments - width + 1))
        weights[start:start + width] = 16384
    if total_elements is None:
        scaled = weights * mean_length
        if np.any(scaled >= float(2**63)):
            raise ValueError("generated length exceeds i64")
        result = np.floor(scaled).astype(np.int64)
        if sum(map(int, result)) > 2**63 - 1:
            raise ValueError("total generated elements exceed i64")
        return result
    return allocate(weights, total_elements)


def offsets_from_lengths(lengths: np.ndarray, dtype: str = "i64") -> np.ndarray:
    """``[0, cumsum(lengths)]`` in i32 or i64 (bench/distributions.py:67-76)."""
    if dtype not in ("i32", "i64"):
        raise ValueError("offsets dtype must be i32 or i64")
    lengths = np.asarray(lengths)
    if lengths.ndim != 1 or lengths.dtype.kind not in "iu" or np.any(lengths < 0):
        raise ValueError("lengths must be a nonnegative integer vector")
    total = sum(map(int, lengths))
    target = np.int32 if dtype == "i32" else np.int64
    if total > np.iinfo(target).max:
        raise ValueError(f"total elements do not fit {dtype}")
    return np.concatenate([np.zeros(1, dtype=target), np.cumsum(lengths, dtype=target)])


HISTOGRAM_EDGES = (0, 1, 2, 8, 32, 33, 128, 1024, 4096, 4097, 16384)


def describe(lengths: np.ndarray) -> dict:
    """Length statistics and sha256 (bench/distributions.py:79-90)."""
    lengths = np.asarray(lengths)
    edges = list(HISTOGRAM_EDGES)
    counts = [int(np.count_nonzero((lengths >= lo) & (lengths < hi))) for lo, hi in zip(edges, edges[1:])]
    counts.append(int(np.count_nonzero(lengths >= edges[-1])))
    return {"segments": int(lengths.size), "elements": sum(map(int, lengths)),
            "min_length": int(lengths.min()) if lengths.size else None,
            "max_length": int(lengths.max()) if lengths.size else None,
            "histogram_lower_bounds": edges, "histogram_counts": counts,
            "lengths_sha256": hashlib.sha256(lengths.astype("<i8").tobytes()).hexdigest()}


def reference_values(seed: int, n: int, d: int) -> np.ndarray:
    """f32 values of a reference benchmark case: ``default_rng(seed + 1)
    .normal(size=(N, D))`` rounded to f32 (bench/run.py:51-55)."""
    return np.random.default_rng(seed + 1).normal(size=(n, d)).astype(np.float32)


def sha256(array: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(array).tobytes()).hexdigest()


# ---------------------------------------------------------------------------
# The five measured configurations.

@dataclass(frozen=True)
class Workload:
    """One generated input: lengths, offsets and f32 values (bf16 workloads
    carry f32 values that the consumer rounds to bf16 with RNE)."""
    name: str
    ops: tuple[str, ...]
    dtype: str
    d: int
    offsets_dtype: str
    lengths: np.ndarray
    offsets: np.ndarray
    values: np.ndarray
    seed: int
    pass_max_len: bool = False
    notes: dict = field(default_factory=dict)

    @property
    def n(self) -> int:
        return int(self.offsets[-1])

    @property
    def b(self) -> int:
        return len(self.offsets) - 1

    @property
    def max_len(self) -> int:
        return int(self.lengths.max()) if self.lengths.size else 0


def _normal_f32(rng: np.random.Generator, n: int, d: int, scale: float = 1.0, rows_per_block: int = 1 << 18):
    """Row blocks of f32 standard normals times ``scale`` (bounded memory)."""
    out = np.empty((n, d), dtype=np.float32)
    for lo in range(0, n, rows_per_block):
        hi = min(n, lo + rows_per_block)
        out[lo:hi] = rng.standard_normal((hi - lo, d), dtype=np.float32)
    if scale != 1.0:
        out *= np.float32(scale)
    return out


def config_c1(seed: int = 711) -> Workload:
    """C1: sum f32 D=1, 10,000 segments of exactly 64 rows, i64 offsets,
    values ``default_rng(seed+1).standard_normal`` (seeds 711-713)."""
    lengths = np.full(10_000, 64, dtype=np.int64)
    offsets = offsets_from_lengths(lengths, "i64")
    values = _normal_f32(np.random.default_rng(seed + 1), int(offsets[-1]), 1)
    return Workload("c1_sum_f32_d1_uniform64", ("sum",), "f32", 1, "i64", lengths, offsets, values, seed)


def config_c2(seed: int = 711) -> Workload:
    """C2: sum and max f32 D=128, 4,096 segments, lengths U{0..512} with ~1%
    forced empty, i64 offsets, N(0,1) values with 0.1% NaN and a disjoint
    0.1% -inf."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(0, 513, 4096).astype(np.int64)
    lengths[rng.random(4096) < 0.01] = 0
    offsets = offsets_from_lengths(lengths, "i64")
    vrng = np.random.default_rng(seed + 1)
    values = _normal_f32(vrng, int(offsets[-1]), 128)
    draw = vrng.random(values.shape)
    values[draw < 0.001] = np.nan
    values[(draw >= 0.001) & (draw < 0.002)] = -np.inf
    return Workload("c2_sum_max_f32_d128_uniform512", ("sum", "max"), "f32", 128, "i64",
                    lengths, offsets, values, seed)


def config_c3(seed: int = 711) -> Workload:
    """C3: softmax f32 D=1, 200,000 segments, lengths geometric(1/16)
    clipped to [1, 32], i32 offsets, N(0, 3) values."""
    rng = np.random.default_rng(seed)
    lengths = np.minimum(rng.geometric(1 / 16, 200_000), 32).astype(np.int64)
    offsets = offsets_from_lengths(lengths, "i32")
    values = _normal_f32(np.random.default_rng(seed + 1), int(offsets[-1]), 1, 3.0)
    return Workload("c3_softmax_f32_d1_geometric16", ("softmax",), "f32", 1, "i32",
                    lengths, offsets, values, seed)


def config_c4(seed: int = 711) -> Workload:
    """C4: sum and max f32 D=2, 50,000 segments: 95% U[1,8], 5% U[2000,8000],
    shuffled, i32 offsets, N(0,1) values."""
    rng = np.random.default_rng(seed)
    b = 50_000
    long_count = b // 20
    short = rng.integers(1, 9, b - long_count)
    long = rng.integers(2000, 8001, long_count)
    lengths = rng.permutation(np.concatenate([short, long])).astype(np.int64)
    offsets = offsets_from_lengths(lengths, "i32")
    values = _normal_f32(np.random.default_rng(seed + 1), int(offsets[-1]), 2)
    return Workload("c4_sum_max_f32_d2_bimodal", ("sum", "max"), "f32", 2, "i32",
                    lengths, offsets, values, seed)


C5_ROWS = 4_194_304
C5_SEGMENTS = 8_192
C5_LONGEST = 200_000


def c5_lengths(seed: int = 711) -> np.ndarray:
    """C5 lengths: Pareto(1.2)+1 weights over 8,192 segments allocated to
    exactly 4,194,304 rows, then the longest set to 200,000 rows and the
    remaining rows re-allocated over the other segments by the same weights."""
    rng = np.random.default_rng(seed)
    weights = rng.pareto(1.2, C5_SEGMENTS) + 1
    lengths = allocate(weights, C5_ROWS)
    longest = int(np.argmax(lengths))
    rest = np.delete(np.arange(C5_SEGMENTS), longest)
    lengths[longest] = C5_LONGEST
    lengths[rest] = allocate(weights[rest], C5_ROWS - C5_LONGEST)
    return lengths


def config_c5(seed: int = 711, *, values: bool = True) -> Workload:
    """C5: softmax bf16 D=128 (f32 accumulation), long-tail lengths (see
    ``c5_lengths``), i64 offsets, N(0, 2) values (f32, rounded to bf16 by the
    consumer), ``max_len`` passed by the caller."""
    lengths = c5_lengths(seed)
    offsets = offsets_from_lengths(lengths, "i64")
    n = int(offsets[-1])
    data = (_normal_f32(np.random.default_rng(seed + 1), n, 128, 2.0) if values
            else np.empty((0, 128), dtype=np.float32))
    return Workload("c5_softmax_bf16_d128_longtail", ("softmax",), "bf16", 128, "i64",
                    lengths, offsets, data, seed, pass_max_len=True)


CONFIGS = {"c1": config_c1, "c2": config_c2, "c3": config_c3, "c4": config_c4, "c5": config_c5}


def algorithmic_bytes(op: str, n: int, b: int, d: int, element_bytes: int, offset_bytes: int) -> int:
    """Bytes a call must move at minimum: read values and offsets once and
    write the output once (sum/max: B rows; softmax: N rows)."""
    out_rows = n if op == "softmax" else b
    return n * d * element_bytes + out_rows * d * element_bytes + (b + 1) * offset_bytes
