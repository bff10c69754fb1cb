"""CPU oracle for segmented sum, max and softmax -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
it. The product path (``ragged`` over ``libragged_hip.so``) never imports,
links or calls anything here, and raises when its HIP library is missing.

Every function restates the reference's float64 NumPy specification
(simon-jd/ragged-mlir ``oracle/reference.py``, ``oracle/masked.py``,
``docs/semantics.md``); each docstring cites the lines it follows. The
restatement imports neither the product nor torch.

Pinning (what fails if the restatement is wrong):
* ``segment_sum/max/softmax``: hand-computed known answers of the reference's
  ``test/python/test_oracle.py`` (tests/test_oracle.py), a float64 per-segment
  loop cross-check (``*_loop``), closed forms (constant segments, shift
  invariance, permutation / empty insertion) and ``math.fsum`` brute force.
* ``assert_matches``: the reference's accept/reject known answers
  (test_oracle.py:162-200) restated in tests/test_oracle.py.
* ``quantize_bf16``: the reference's RNE known answers (test_oracle.py:111-118)
  and an exhaustive check against torch's own bfloat16 rounding.
* ``masked_logits``: closed-form f32 arithmetic checks (tests/test_oracle.py).
* ``offsets_errors``: the reference's all-conditions known answer
  (test/gpu/test_checked.py:125-130) and brute-force properties
  (tests/test_oracle.py).
"""

from .offsets import CONDITIONS, offsets_errors
from .reference import (
    Expectation,
    STRICT_TOLERANCES,
    TOLERANCES,
    assert_matches,
    quantize_bf16,
    segment_max,
    segment_max_loop,
    segment_reduce,
    segment_softmax,
    segment_softmax_loop,
    segment_sum,
    segment_sum_loop,
    validate_offsets,
)
from .masked import assert_masked_softmax_matches, masked_logits

__all__ = [
    "Expectation", "STRICT_TOLERANCES",
    "TOLERANCES", "assert_matches", "quantize_bf16", "segment_max", "segment_max_loop",
    "segment_reduce", "segment_softmax", "segment_softmax_loop", "segment_sum", "segment_sum_loop",
    "validate_offsets", "masked_logits", "assert_masked_softmax_matches", "CONDITIONS", "offsets_errors",
]
