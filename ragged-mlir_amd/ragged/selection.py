"""Per-call choice between device classification and one block per segment.

Same decision rule as the reference's ``python/ragged/selection.py``
(:56-126): predict the complete-call time of each schedule from host-known
statistics (N, B, D, element size and the caller's longest segment L) with a
model per operation family and schedule, and classify only when that
is predicted faster by the family's margin; without L keep classification. The
families are the reference's {reduce, softmax} plus ``softmax_fused``: a
softmax whose classified schedule is the register-resident worker pays a
per-segment cost the streaming worker does not, so it gets its own fit.

The terms are re-derived for MI355X (model version 6, eleven terms, µs):

    t = c0 + c1*W + c2*S + c3*B/1000 + c4*F*B/1000 + c5*R*B/1000 + c6*X_l2 + c7*X_mall + c8*W*A
          + c9*W*U + c10*S*U

W = MiB the call moves (rows read; rows written for softmax, B result rows
for sum/max); S = L*D*element_bytes / 2^20, the MiB the one workgroup that
owns the longest segment must stream in block-per-segment; B/1000 the
per-segment cost, with two refinements: F = 1 for the flat mapping (D below
the 16-byte vector: a segment is a run of elements, and block-per-segment
pays most per segment there) and R = row KiB (D*element_bytes / 1024);
X_l2 / X_mall = MiB of the working set (input rows plus output rows) beyond
the total L2 (8 XCDs x 4 MiB) and beyond the 256 MiB Infinity Cache. The
reference's single "beyond the 72 MiB L2" term becomes two because MI355X
has two cache levels of very different size in front of HBM. A = 16 /
access bytes - 1, where a lane's access is the mapping's vector (16 bytes
for D dividing or divided by the 16-byte vector, else the largest power of
two of elements dividing D): the extra cost per MiB of narrower accesses.
U = 1/u - 1 for the row mapping's lane utilisation u (a row's vectors over
the lanes that hold it: D = 80 f32 is 20 vectors on 32 lanes, u = 0.625),
0 for the flat mapping: idle lanes cost the streaming rate of every
workgroup (W) and of the one that owns the longest segment (S).

Model version 7 (the shipped form) keeps the rule and replaces each
family's and schedule's linear terms by a boosted ensemble of regression
trees over nine host statistics (``host_features``): log2 of the MiB moved
over the L2 capacity, of B, of the longest segment's MiB, of L over the mean
length N/B, of the row bytes and of the mean segment's MiB, the flat-mapping
flag, and the narrow-access and idle-lane shares (A and U above). Each
ensemble predicts log(µs); trees are stored complete to their depth
(``features``/``thresholds`` per internal node in heap order, a sample goes
right when its statistic exceeds the threshold; ``leaves`` already scaled by
the learning rate), so a prediction is `depth` gathers per tree. The linear
terms miss where the time depends on the skew of the lengths, which the
ratio of the longest to the mean length carries and a sum of terms cannot
combine with size; fitted on the same suites, the ensembles choose within 3%
more often when each suite is held out in turn. Version 6 files still load.

Each family has its own margin (a register-resident softmax's
classification also writes item descriptors and cleans its statistics
arena, so the schedules' fixed costs differ by family). The runtime consults the model only when the
caller's max_len does not let one lane or lane group reduce every segment
alone: those calls take the one-launch short-segment schedule
(``CompiledProgram.run``), which the model is not fitted on.
"""
from __future__ import annotations

from dataclasses import dataclass
import json
import math
from pathlib import Path
from typing import Any

from .errors import CacheMismatch

MODEL_PATH = Path(__file__).with_name("cost_model.json")
SCHEDULES = ("classified", "naive")
FAMILIES = ("reduce", "softmax", "softmax_fused")
TERMS = 11
HOST_FEATURES = 9
VERSION = 7          # what calibrate.fit writes by default; version 6 (linear terms) still loads
VERSIONS = (6, 7)


def family(op: str, fused: bool = False) -> str:
    if op != "softmax":
        return "reduce"
    return "softmax_fused" if fused else "softmax"


def features(n: int, b: int, d: int, max_len: int, element_bytes: int = 4, op: str = "sum",
             l2_mib: float = 32.0, mall_mib: float = 256.0, flat: bool = False) -> tuple[float, ...]:
    """The eleven prediction terms for one call."""
    row = d * element_bytes
    rows = n * row / 2**20
    output_rows = n if op == "softmax" else b
    moved = rows + output_rows * row / 2**20
    longest = max_len * row / 2**20
    segments = b / 1000.0
    idle = 0.0 if flat else 1.0 / lane_utilisation(d, element_bytes) - 1.0
    return (1.0, moved, longest, segments, segments if flat else 0.0, segments * row / 1024,
            max(0.0, moved - l2_mib), max(0.0, moved - mall_mib), moved * (16 / access_bytes(d, element_bytes) - 1),
            moved * idle, longest * idle)


def access_bytes(d: int, element_bytes: int) -> int:
    """Bytes of one lane's access in the default geometry (Optimizations.geometry)."""
    widest = 16 // element_bytes
    if d < widest and widest % d == 0:
        return 16
    vec = 1
    while vec * 2 <= widest and d % (vec * 2) == 0:
        vec *= 2
    return vec * element_bytes


def lane_utilisation(d: int, element_bytes: int) -> float:
    """Share of the lanes holding a row that hold data in the row mapping of
    the default geometry (Optimizations.geometry): ceil(D / vec) vectors on
    the next power of two of lanes (at most 64, several passes beyond)."""
    vec = access_bytes(d, element_bytes) // element_bytes
    vectors = -(-d // vec)
    lanes = 1
    while lanes < vectors and lanes < 64:
        lanes *= 2
    return vectors / (lanes * -(-vectors // lanes))


def host_features(n: int, b: int, d: int, max_len: int, element_bytes: int = 4, op: str = "sum",
                  l2_mib: float = 32.0, flat: bool = False) -> tuple[float, ...]:
    """The nine statistics a version-7 ensemble splits on (see the module
    docstring): all host-known, logs base 2 of sizes clamped away from zero."""
    row = d * element_bytes
    n, b, longest_rows = max(n, 1), max(b, 1), max(max_len, 1)
    output_rows = n if op == "softmax" else b
    moved = (n + output_rows) * row / 2**20
    mean = n / b
    idle = 0.0 if flat else 1.0 / lane_utilisation(d, element_bytes) - 1.0
    return (math.log2(moved / l2_mib), math.log2(b), math.log2(longest_rows * row / 2**20),
            math.log2(longest_rows / mean), math.log2(row), 1.0 if flat else 0.0,
            16 / access_bytes(d, element_bytes) - 1, idle, math.log2(mean * row / 2**20))


def _leaf_table(depth: int):
    """For a complete tree of ``depth``: the leaf reached for every word of
    node decisions (bit i = node i, heap order, goes right)."""
    import numpy as np
    inner = 2**depth - 1
    codes = np.arange(1 << inner, dtype=np.int64)
    node = np.zeros_like(codes)
    for _ in range(depth):
        node = 2 * node + 1 + ((codes >> node) & 1)
    return node - inner


@dataclass(frozen=True)
class Ensemble:
    """Complete regression trees of one depth: sum of the reached leaves
    plus ``base`` is log(µs)."""
    base: float
    depth: int
    features: Any      # int array [trees, 2**depth - 1]
    thresholds: Any    # float array [trees, 2**depth - 1]
    leaves: Any        # float array [trees, 2**depth]

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "Ensemble":
        import numpy as np
        depth = int(data["depth"])
        features = np.asarray(data["features"], dtype=np.int64)
        thresholds = np.asarray(data["thresholds"], dtype=np.float64)
        leaves = np.asarray(data["leaves"], dtype=np.float64)
        base = float(data["base"])
        trees = len(leaves)
        if (not 1 <= depth <= 8 or trees < 1 or features.shape != (trees, 2**depth - 1)
                or thresholds.shape != features.shape or leaves.shape != (trees, 2**depth)
                or features.min() < 0 or features.max() >= HOST_FEATURES
                or not (np.isfinite(thresholds).all() and np.isfinite(leaves).all() and math.isfinite(base))):
            raise ValueError("ensemble arrays do not match its depth and statistics")
        return cls(base, depth, features, thresholds, leaves)

    @staticmethod
    def pair_log_us(first: "Ensemble", second: "Ensemble", x) -> tuple[float, float]:
        """log(µs) of two ensembles of one depth for one statistics vector."""
        return EnsemblePair(first, second).log_us(x)

    def to_dict(self) -> dict[str, Any]:
        return {"base": self.base, "depth": self.depth, "features": self.features.tolist(),
                "thresholds": self.thresholds.tolist(), "leaves": self.leaves.tolist()}

    def log_us(self, x) -> Any:
        """log(µs) for host statistics ``x`` ([HOST_FEATURES] or [rows,
        HOST_FEATURES]), rounded to float32 before the comparisons, as the
        trees were grown on them."""
        import numpy as np
        x = np.asarray(x, dtype=np.float32).astype(np.float64)
        single = x.ndim == 1
        x = np.atleast_2d(x)
        trees = np.arange(len(self.leaves))
        node = np.zeros((len(x), len(trees)), dtype=np.int64)
        rows = np.arange(len(x))[:, None]
        for _ in range(self.depth):
            f = self.features[trees, node]
            node = 2 * node + 1 + (x[rows, f] > self.thresholds[trees, node])
        out = self.base + self.leaves[trees, node - (2**self.depth - 1)].sum(axis=1)
        return float(out[0]) if single else out


class EnsemblePair:
    """Two ensembles of one depth (a family's classified and block-per-
    segment schedules) flattened for one pass over their trees: the runtime
    pays a prediction once per new call shape. Up to depth 4 every node's
    decision is taken at once and a tree's 15 decision bits index a table of
    the leaf they lead to; deeper trees walk their levels."""

    def __init__(self, first: Ensemble, second: Ensemble):
        import numpy as np
        if first.depth != second.depth:
            raise ValueError("paired ensembles must share a depth")
        self.depth = depth = first.depth
        self.inner = inner = 2**depth - 1
        trees = len(first.leaves) + len(second.leaves)
        self.bases = (first.base, second.base)
        self.features = np.concatenate([first.features, second.features]).ravel()
        self.thresholds = np.concatenate([first.thresholds, second.thresholds]).ravel()
        self.leaves = np.concatenate([first.leaves, second.leaves]).ravel()
        self.node_base = np.arange(trees) * inner
        self.leaf_base = np.arange(trees) * (inner + 1)
        self.split = len(first.leaves)
        self.table = _leaf_table(depth) if depth <= 4 else None
        self.bits = 1 << np.arange(inner, dtype=np.int64)

    def log_us(self, x) -> tuple[float, float]:
        import numpy as np
        x = np.asarray(x, dtype=np.float32).astype(np.float64)
        if self.table is not None:
            decisions = (x.take(self.features) > self.thresholds).reshape(len(self.node_base), self.inner)
            leaf = self.table.take(decisions @ self.bits)
        else:
            node = np.zeros(len(self.node_base), dtype=np.int64)
            for _ in range(self.depth):
                g = self.node_base + node
                node = 2 * node + 1 + (x.take(self.features.take(g)) > self.thresholds.take(g))
            leaf = node - self.inner
        reached = self.leaves.take(self.leaf_base + leaf)
        return self.bases[0] + float(reached[:self.split].sum()), self.bases[1] + float(reached[self.split:].sum())


@dataclass(frozen=True)
class CostModel:
    coefficients: dict[str, dict[str, tuple[float, ...]]]
    margins: dict[str, float]
    calibration: dict[str, Any]
    l2_mib: float = 32.0
    mall_mib: float = 256.0
    version: int = 6
    ensembles: dict[str, dict[str, Ensemble]] | None = None
    pairs: dict[str, EnsemblePair] | None = None

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "CostModel":
        try:
            version = data["version"]
            if version not in VERSIONS:
                raise CacheMismatch("unsupported cost model version")
            coefficients, ensembles = {}, None
            if version == 6:
                coefficients = {name: {schedule: tuple(float(v) for v in data["coefficients"][name][schedule])
                                       for schedule in SCHEDULES} for name in FAMILIES}
            else:
                ensembles = {name: {schedule: Ensemble.from_dict(data["ensembles"][name][schedule])
                                    for schedule in SCHEDULES} for name in FAMILIES}
            margins = {name: float(data["margins"][name]) for name in FAMILIES}
            l2_mib, mall_mib = float(data["l2_mib"]), float(data["mall_mib"])
        except (KeyError, TypeError, ValueError) as exc:
            raise CacheMismatch(f"invalid cost model: {exc}") from exc
        if (any(len(values) != TERMS or any(v < 0 or not math.isfinite(v) for v in values)
                for schedules in coefficients.values() for values in schedules.values())
                or not all(0 <= m < 1 for m in margins.values()) or not l2_mib > 0 or not mall_mib > 0):
            raise CacheMismatch(f"cost model coefficients must be {TERMS} nonnegative terms, margins in [0, 1) "
                                "and positive cache capacities")
        pairs = None if ensembles is None else {
            name: EnsemblePair(ensembles[name]["classified"], ensembles[name]["naive"]) for name in FAMILIES}
        return cls(coefficients, margins, dict(data.get("calibration", {})), l2_mib, mall_mib, version, ensembles,
                   pairs)

    @classmethod
    def load(cls, path: Path = MODEL_PATH) -> "CostModel":
        return cls.from_dict(json.loads(Path(path).read_text()))

    def predict(self, schedule: str, op: str, n: int, b: int, d: int, max_len: int, element_bytes: int = 4,
                l2_mib: float | None = None, fused: bool = False, flat: bool = False) -> float:
        l2 = self.l2_mib if l2_mib is None else l2_mib
        if self.ensembles is not None:
            x = host_features(n, b, d, max_len, element_bytes, op, l2, flat)
            return math.exp(self.ensembles[family(op, fused)][schedule].log_us(x))
        terms = features(n, b, d, max_len, element_bytes, op, l2, self.mall_mib, flat)
        return sum(c * x for c, x in zip(self.coefficients[family(op, fused)][schedule], terms))

    def choose(self, op: str, n: int, b: int, d: int, max_len: int | None, element_bytes: int = 4,
               l2_mib: float | None = None, fused: bool = False,
               flat: bool = False) -> tuple[str, dict[str, Any]]:
        """The schedule to run and the inputs and predictions behind it."""
        if max_len is None:
            return "classified", {"max_len": None, "reason": "no length statistics on the host"}
        if l2_mib is not None and not (isinstance(l2_mib, (int, float)) and l2_mib > 0):
            raise ValueError("l2_mib must be a positive capacity in MiB")
        if self.ensembles is not None:
            x = host_features(n, b, d, max_len, element_bytes, op, self.l2_mib if l2_mib is None else l2_mib, flat)
            classified, naive = (math.exp(v) for v in self.pairs[family(op, fused)].log_us(x))
        else:
            classified = self.predict("classified", op, n, b, d, max_len, element_bytes, l2_mib, fused, flat)
            naive = self.predict("naive", op, n, b, d, max_len, element_bytes, l2_mib, fused, flat)
        selected = "classified" if classified < naive * (1 - self.margins[family(op, fused)]) else "naive"
        return selected, {"max_len": max_len, "l2_mib": self.l2_mib if l2_mib is None else l2_mib,
                          "predicted_us": {"classified": round(classified, 2), "naive": round(naive, 2)}}


_model: CostModel | None = None


def default_model() -> CostModel:
    global _model
    if _model is None:
        _model = CostModel.load()
    return _model
