"""Per-call choice between device classification and one block per segment.

Same decision rule as the reference's ``python/ragged/selection.py``
(:56-126): predict the complete-call time of each schedule from host-known
statistics (N, B, D, element size and the caller's longest segment L) with a
linear model per operation family and schedule, and classify only when that
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

Each family has its own margin (a register-resident softmax pays three
more launches than its streaming counterpart, so the schedules' fixed
costs differ by family). The runtime consults the model only when the
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
VERSION = 6


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


@dataclass(frozen=True)
class CostModel:
    coefficients: dict[str, dict[str, tuple[float, ...]]]
    margins: dict[str, float]
    calibration: dict[str, Any]
    l2_mib: float = 32.0
    mall_mib: float = 256.0

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "CostModel":
        try:
            if data["version"] != VERSION:
                raise CacheMismatch("unsupported cost model version")
            coefficients = {name: {schedule: tuple(float(v) for v in data["coefficients"][name][schedule])
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
        return cls(coefficients, margins, dict(data.get("calibration", {})), l2_mib, mall_mib)

    @classmethod
    def load(cls, path: Path = MODEL_PATH) -> "CostModel":
        return cls.from_dict(json.loads(Path(path).read_text()))

    def predict(self, schedule: str, op: str, n: int, b: int, d: int, max_len: int, element_bytes: int = 4,
                l2_mib: float | None = None, fused: bool = False, flat: bool = False) -> float:
        terms = features(n, b, d, max_len, element_bytes, op, self.l2_mib if l2_mib is None else l2_mib,
                         self.mall_mib, flat)
        return sum(c * x for c, x in zip(self.coefficients[family(op, fused)][schedule], terms))

    def choose(self, op: str, n: int, b: int, d: int, max_len: int | None, element_bytes: int = 4,
               l2_mib: float | None = None, fused: bool = False,
               flat: bool = False) -> tuple[str, dict[str, Any]]:
        """The schedule to run and the inputs and predictions behind it."""
        if max_len is None:
            return "classified", {"max_len": None, "reason": "no length statistics on the host"}
        if l2_mib is not None and not (isinstance(l2_mib, (int, float)) and l2_mib > 0):
            raise ValueError("l2_mib must be a positive capacity in MiB")
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
