"""GPU run of the cost-model measurement (reference bench/suite.py:148-191,
bench/calibrate.py:141-157): a few cases of each family through
calibrate.measure, whose every schedule passes the sampled correctness gate
before it is timed warm and cold; and the gate's verdict on one measured
shape agrees with the float64 oracle's."""
from __future__ import annotations

import json

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import ArtifactCache, Compiler, ProgramSpec, calibrate, native  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

CASES = [calibrate.Case("sum", "f32", 3, 60_000, 512, "long_tail", 41),
         calibrate.Case("max", "bf16", 48, 20_000, 4096, "bimodal", 42),
         calibrate.Case("softmax", "bf16", 96, 30_000, 300, "burst", 43),
         calibrate.Case("softmax", "f32", 12, 40_000, 2048, "exponential", 44)]


def test_measure_gates_and_times_both_schedules(tmp_path):
    out = tmp_path / "suite.jsonl"
    assert calibrate.measure(CASES, out, log=lambda s: print(s, flush=True)) == len(CASES)
    records = [json.loads(line) for line in out.read_text().splitlines()]
    assert [r["key"] for r in records] == [c.key for c in CASES]
    for record in records:
        for schedule in ("classified", "naive"):
            assert record["us"][schedule] > 0 and record["us_cold"][schedule] > 0
            assert 0.0 <= record["gate"][schedule] <= 1.0
        assert record["library_sha256"] == native.library_sha256()
    # Resumes: nothing left to measure.
    assert calibrate.measure(CASES, out) == 0


def test_gate_agrees_with_the_oracle_on_a_measured_shape(artifact_cache):
    case = CASES[2]
    lengths = make_lengths(case.distribution, case.b, seed=case.seed, total_elements=case.n)
    offsets = offsets_from_lengths(lengths, "i64")
    values = oracle.quantize_bf16(np.random.default_rng(7).normal(size=(int(offsets[-1]), case.d)).astype(np.float32))
    program = Compiler().compile(ProgramSpec(case.op, case.dtype, case.d, "i64"), artifact_cache)
    x = torch.from_numpy(values).to("cuda").to(torch.bfloat16)
    off = torch.from_numpy(offsets).to("cuda")
    for select in ("classified", "naive"):
        y = torch.full_like(x, float("nan"))
        program.run(x, off, y, select=select, max_len=int(lengths.max()))
        torch.cuda.synchronize()
        report = calibrate.gate(torch, case.op, case.dtype, x, offsets, y, case.seed)
        stats = oracle.Expectation(values, offsets, operation="softmax", input_dtype="bf16").check(
            y.float().cpu().numpy().astype(np.float64), oracle.STRICT_TOLERANCES)
        assert report["max_fraction_of_tolerance"] <= stats["max_fraction_of_tolerance"] + 1e-6
