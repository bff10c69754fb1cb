"""Optimization requests (reference: python/ragged/optimizations.py:13-59).

The same immutable record of eight switches plus ``feature_tile``. On gfx950
the kernels are hand-written, so a switch either selects a compiled variant
or is recorded as not applicable; ``effective(...)`` reports what actually
runs and every manifest carries both (``requested`` and ``effective``).
"""
from __future__ import annotations

from dataclasses import asdict, dataclass

from .errors import ValidationError

BOOL_OPTIONS = ("classification", "online_fusion", "warp_mapping", "split_mapping", "shuffle", "pointwise_fusion",
                "row_pipelining", "vectorize")
VECTOR_WIDTHS = (1, 2, 4, 8)
FEATURE_TILES = (1, 2, 4, 8, 16, 32)


@dataclass(frozen=True)
class Optimizations:
    """Switches of the reference, mapped to the HIP schedules:

    * ``classification``: device binning plus persistent workers; False keeps
      only the block-per-segment schedule.
    * ``warp_mapping`` / ``split_mapping``: enable the wave64 and the split
      class (disabled classes route their segments to the workgroup class).
    * ``vectorize``: 16-byte accesses (False: one element per access, any
      alignment).
    * ``online_fusion``, ``shuffle``, ``pointwise_fusion``, ``row_pipelining``:
      always in effect on gfx950 (statistics are fused, wave reductions use
      cross-lane operations, scale/mask are fused into loads, rows are loaded
      four per lane before folding); accepted for compatibility.
    * ``feature_tile``: accepted for compatibility; the lane layout is derived
      from D and the 16-byte access width.
    """
    classification: bool = True
    online_fusion: bool = True
    warp_mapping: bool = True
    split_mapping: bool = True
    shuffle: bool = True
    pointwise_fusion: bool = True
    row_pipelining: bool = True
    vectorize: bool = True
    feature_tile: int | None = None

    def __post_init__(self):
        for name in BOOL_OPTIONS:
            if type(getattr(self, name)) is not bool:
                raise ValidationError(f"optimization {name} must be bool")
        if self.feature_tile is not None and (type(self.feature_tile) is not int
                                              or self.feature_tile not in FEATURE_TILES):
            raise ValidationError("feature_tile must be None or a power of two in [1,32]")

    def to_dict(self):
        return asdict(self)

    def geometry(self, d: int, dtype: str = "f32") -> tuple[int, int, str]:
        """(lanes per row of a 64-lane wave, elements per access, mapping).

        Elements per access: the 16-byte vector (4 f32, 8 bf16) when D is
        smaller and divides it ("flat": a segment is read as one contiguous
        run), else the largest power of two dividing D that fits 16 bytes
        ("row"). Lanes per row: next power of two of D / vec, at most 64.
        """
        element = 2 if dtype == "bf16" else 4
        widest = 16 // element
        if not self.vectorize:
            vec, mapping = 1, "row"
        elif d < widest and widest % d == 0:
            return 1, widest, "flat"
        else:
            vec = 1
            while vec * 2 <= widest and d % (vec * 2) == 0:
                vec *= 2
            mapping = "row"
        lanes = -(-d // vec)
        lpr = 1
        while lpr < lanes and lpr < 64:
            lpr *= 2
        return lpr, vec, mapping

    def effective(self) -> dict[str, bool]:
        return {"classification": self.classification, "online_fusion": True, "warp_mapping": self.warp_mapping,
                "split_mapping": self.split_mapping, "shuffle": True, "pointwise_fusion": True,
                "row_pipelining": True, "vectorize": self.vectorize}
