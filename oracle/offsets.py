"""Checked-mode offsets conditions -- TEST INFRASTRUCTURE ONLY (the checker,
never the product; see the package docstring).

Restates the seven conditions of simon-jd/ragged-mlir ``docs/checked-abi.md``
(table "Slot / Condition / Reported index", lines 37-53 of that file): each
failed condition maps to its earliest offending index, in slot order. Python
integers throughout, so extreme i64 offsets cannot overflow.
"""
from __future__ import annotations

CONDITIONS = ("first_nonzero", "final_mismatch", "negative", "above_n",
              "nonmonotone", "below_min_len", "above_max_len")


def offsets_errors(offsets, n: int, min_len: int | None = None, max_len: int | None = None) -> dict[str, int]:
    """Every failed condition with its earliest index (docs/checked-abi.md):

    0 ``offsets[0] != 0`` (index 0); 1 ``offsets[B] != N`` (index B);
    2 ``offsets[i] < 0`` and 3 ``offsets[i] > N`` (offset index i);
    4 ``offsets[i+1] < offsets[i]`` (segment i, compared, never subtracted);
    5 / 6 a length below ``min_len`` / above ``max_len``, only for segments
    whose endpoints are both in [0, N] and monotone (segment i).
    """
    values = [int(v) for v in offsets]
    b = len(values) - 1
    found: dict[str, int] = {}

    def note(condition: str, index: int) -> None:
        if condition not in found or index < found[condition]:
            found[condition] = index

    if values[0] != 0:
        note("first_nonzero", 0)
    if values[b] != n:
        note("final_mismatch", b)
    for i, value in enumerate(values):
        if value < 0:
            note("negative", i)
        if value > n:
            note("above_n", i)
    for i in range(b):
        start, end = values[i], values[i + 1]
        if end < start:
            note("nonmonotone", i)
        elif 0 <= start and end <= n:
            length = end - start
            if min_len is not None and length < min_len:
                note("below_min_len", i)
            if max_len is not None and length > max_len:
                note("above_max_len", i)
    return {condition: found[condition] for condition in CONDITIONS if condition in found}
