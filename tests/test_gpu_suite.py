"""GPU run of the benchmark suite runner on one of the reference's compare
cells (reference bench/suite.py, bench/run.py:240-300): every method's
output passes the correctness gate, is timed warm, cold and replayed from a
captured graph, the record names the library and the regenerated inputs'
hashes equal the reference's, and a second run resumes with nothing left."""
from __future__ import annotations

import json
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import native, suite  # noqa: E402

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference_cases.json"


@pytest.mark.parametrize("cell", ["max-f32-d1-burst", "softmax-bf16-d128-long_tail"])
def test_one_cell_through_the_suite(tmp_path, cell):
    assert suite.run_suite(tmp_path, seeds=(711,), pattern=cell, flush_mib=512,
                           log=lambda s: print(s, flush=True)) == 1
    record = json.loads(suite.result_path(tmp_path, cell, 711).read_text())
    assert record["status"] == "complete" and record["library_sha256"] == native.library_sha256()
    reference = next(c for c in json.loads(GOLDEN.read_text())["recorded_timings"]["cases"]
                     if c["seed"] == 711 and f"{c['op']}-{c['dtype']}-d{c['d']}-{c['distribution']}" == cell)
    assert record["case"]["values_sha256"] == reference["values_sha256"]
    assert record["case"]["lengths_sha256"] == reference["lengths_sha256"]
    methods = {m["method"]: m for m in record["methods"]}
    assert set(methods) == set(suite.METHODS)
    for name in ("ragged-auto", "ragged-auto-no-max-len", "ragged-classified", "ragged-naive"):
        entry = methods[name]
        assert entry["status"] == "measured" and 0.0 <= entry["gate"] <= 1.0, entry
        assert entry["warm_ms"]["median"] > 0 and entry["cold_ms"]["median"] > 0
        assert entry["graph_ms"]["median"] > 0 and entry["graph_gate"] <= 1.0, entry
    assert methods["ragged-naive"]["selected"] == "naive"
    assert methods["ragged-classified"]["selected"] == "classified"
    assert suite.run_suite(tmp_path, seeds=(711,), pattern=cell, flush_mib=512) == 0
    assert any(line.startswith(f"| {cell} ") for line in suite.summarize(tmp_path, GOLDEN))
