"""Shared helpers of the GPU parity tests: run a program on NumPy inputs
through the public API and check the result against the CPU oracle.

Every output is written into a guarded view (sentinel rows before and after,
as the reference's test/gpu/test_correctness.py:90-115 does) so an
out-of-range store fails the test even when the values look right.
"""
from __future__ import annotations

import numpy as np

import oracle

SENTINEL = -64.0
GUARD_ROWS = 8          # keeps the view 16-byte aligned for every D and dtype


def torch_dtype(torch, dtype: str):
    return torch.bfloat16 if dtype == "bf16" else torch.float32


def quantized(values: np.ndarray, dtype: str) -> np.ndarray:
    """The exact f32 representation of the device input."""
    return oracle.quantize_bf16(values) if dtype == "bf16" else np.asarray(values, dtype=np.float32)


def run_program(program, values: np.ndarray, offsets: np.ndarray, *, dtype: str, op: str, select: str = "auto",
                mask: np.ndarray | None = None, max_len: int | None = None, mode: str = "validated",
                debug_buffers=None):
    """Run ``program`` on the device; returns (output as f64 NumPy, report)."""
    import torch
    device = torch.device("cuda", 0)
    tdtype = torch_dtype(torch, dtype)
    x = torch.from_numpy(np.ascontiguousarray(values, dtype=np.float32)).to(device).to(tdtype).contiguous()
    off = torch.from_numpy(np.ascontiguousarray(offsets)).to(device)
    rows = x.shape[0] if op == "softmax" else off.numel() - 1
    d = x.shape[1]
    guarded = torch.full((rows + 2 * GUARD_ROWS, d), SENTINEL, dtype=tdtype, device=device)
    out = guarded[GUARD_ROWS:GUARD_ROWS + rows]
    m = None if mask is None else torch.from_numpy(np.ascontiguousarray(mask, dtype=np.float32)).to(device)
    report = program.run(x, off, out, mask=m, select=select, max_len=max_len, mode=mode,
                         debug_buffers=debug_buffers)
    torch.cuda.synchronize()
    guard = torch.cat([guarded[:GUARD_ROWS], guarded[GUARD_ROWS + rows:]]).float().cpu().numpy()
    assert np.all(guard == SENTINEL), "kernel wrote outside the output rows"
    return out.float().cpu().numpy().astype(np.float64), report


def check_expectation(actual: np.ndarray, expectation: "oracle.Expectation") -> dict:
    """``check`` against a precomputed oracle reference (one float64
    reference for several outputs of the same input): the reference's
    tolerance, the build's stricter one, and max bit for bit."""
    stats = expectation.check(actual)
    expectation.check(actual, oracle.STRICT_TOLERANCES)
    if expectation.operation == "max":
        expected = expectation.expected.astype(np.float32)
        if expectation.input_dtype == "bf16":
            expected = oracle.quantize_bf16(expected)
        nan = np.isnan(expected)
        assert np.array_equal(nan, np.isnan(actual)), "max NaN mask differs"
        assert np.array_equal(actual[~nan], expected[~nan].astype(np.float64)), "max is not bit-exact"
    return stats


def check(actual: np.ndarray, values: np.ndarray, offsets: np.ndarray, *, op: str, dtype: str,
          mask: np.ndarray | None = None, scale: float = 1.0) -> dict:
    """Oracle contract, plus bit-exactness for max (max selects an input)."""
    inputs = quantized(values, dtype)
    if mask is not None or scale != 1.0:
        logits = oracle.masked_logits(inputs, mask if mask is not None else np.zeros_like(inputs), scale=scale)
        if op == "softmax":
            oracle.assert_matches(actual, logits, offsets, operation=op, input_dtype=dtype,
                                  tolerances=oracle.STRICT_TOLERANCES)
            return oracle.assert_matches(actual, logits, offsets, operation=op, input_dtype=dtype)
        inputs = logits
    stats = oracle.assert_matches(actual, inputs, offsets, operation=op, input_dtype=dtype)
    # The build's own bar: rtol 1e-5 (f32) / 1e-2 (bf16) for sum and softmax,
    # with the reference's absolute floor (oracle.STRICT_TOLERANCES).
    oracle.assert_matches(actual, inputs, offsets, operation=op, input_dtype=dtype,
                          tolerances=oracle.STRICT_TOLERANCES)
    if op == "max":
        expected = oracle.segment_max(inputs, offsets).astype(np.float32)
        if dtype == "bf16":
            expected = oracle.quantize_bf16(expected)
        nan = np.isnan(expected)
        assert np.array_equal(nan, np.isnan(actual)), "max NaN mask differs"
        # Max selects an input value: exact, with -0 == +0 (sign not promised).
        assert np.array_equal(actual[~nan], expected[~nan].astype(np.float64)), "max is not bit-exact"
    return stats
