"""CPU tests of the benchmark suite runner: its cells are the reference's
compare cells (same cases, seeds and regenerated inputs, by sha256 against
the reference's records), an interrupted suite resumes at the first cell
without a complete record, and the summary sets this build's medians beside
the reference's recorded ones. No test here launches a kernel."""
from __future__ import annotations

import json
from pathlib import Path

import pytest

from ragged import suite
from ragged.workloads import describe, make_lengths, sha256

REPO = Path(__file__).resolve().parents[1]
GOLDEN = REPO / "tests" / "golden" / "reference_cases.json"


def recorded() -> dict:
    return json.loads(GOLDEN.read_text())["recorded_timings"]


def key(case: dict) -> str:
    return f"{case['op']}-{case['dtype']}-d{case['d']}-{case['distribution']}"


def test_cells_are_the_reference_compare_cells():
    cells = {(key(c), c["seed"]) for c in recorded()["cases"]}
    ours = {(c["key"], seed) for c in suite.compare_cases() for seed in suite.SEEDS}
    assert ours == cells and len(ours) == 57
    for case in recorded()["cases"]:
        mine = next(c for c in suite.compare_cases() if c["key"] == key(case))
        assert (mine["segments"], mine["rows"]) == (case["segments"], case["total_elements"])


def test_cells_regenerate_the_reference_inputs():
    """Lengths of every cell, values of every D=1 cell and of two D=128 cells
    hash to the reference's records."""
    torch = pytest.importorskip("torch")
    cells = {c["key"]: c for c in suite.compare_cases()}
    for case in recorded()["cases"]:
        if case["d"] == 1 or (case["seed"] == 711 and key(case) in ("softmax-bf16-d128-long_tail",
                                                                     "sum-f32-d128-burst")):
            lengths, offsets, values = suite.cell_inputs(torch, cells[key(case)], case["seed"])
            assert sha256(values) == case["values_sha256"], key(case)
            assert int(offsets[-1]) == case["total_elements"]
        else:
            lengths = make_lengths(case["distribution"], case["segments"], seed=case["seed"],
                                   total_elements=case["total_elements"])
        assert describe(lengths)["lengths_sha256"] == case["lengths_sha256"], key(case)


def _record(case: dict, seed: int, auto_ms: float, status: str = "complete") -> dict:
    timing = lambda ms: {"count": 30, "median": ms, "min": ms, "p90": ms}   # noqa: E731
    methods = [{"method": m, "status": "measured", "selected": "naive", "warm_ms": timing(auto_ms),
                "cold_ms": timing(2 * auto_ms), "graph_ms": timing(auto_ms / 2)} for m in suite.METHODS]
    return {"status": status, "case": {**case, "seed": seed}, "device": "test device", "library_sha256": "abc",
            "protocol": {"warmup": suite.WARMUP, "timed": suite.TIMED, "flush_bytes": 1 << 30}, "methods": methods}


def _write(output: Path, case: dict, seed: int, text: str) -> None:
    path = suite.result_path(output, case["key"], seed)
    path.parent.mkdir(parents=True, exist_ok=True)
    path.write_text(text)


def test_resume_skips_only_complete_cells(tmp_path):
    cases = suite.compare_cases()
    assert len(suite.pending(tmp_path)) == 57
    _write(tmp_path, cases[0], 711, json.dumps(_record(cases[0], 711, 0.01)))
    _write(tmp_path, cases[0], 712, json.dumps(_record(cases[0], 712, 0.01, status="running")))
    _write(tmp_path, cases[0], 713, '{"status": "comp')                  # cut off mid-write
    left = suite.pending(tmp_path)
    assert len(left) == 56 and (cases[0], 711) not in left and (cases[0], 712) in left and (cases[0], 713) in left
    assert [c["key"] for c, _ in suite.pending(tmp_path, pattern="softmax-bf16")] == ["softmax-bf16-d128-long_tail"] * 3
    # Prefixes, not substrings: "max-" names the max cells only, not softmax's.
    assert {c["key"] for c, _ in suite.pending(tmp_path, pattern="max-f32-d1-burst")} == {"max-f32-d1-burst"}
    assert len(suite.pending(tmp_path, pattern="max-,sum-f32-d128")) == 6 * 3 - 1 + 3 * 3


def test_summary_against_the_reference_records(tmp_path):
    case = next(c for c in suite.compare_cases() if c["key"] == "softmax-bf16-d128-long_tail")
    for seed, ms in zip(suite.SEEDS, (0.1, 0.2, 0.3)):
        _write(tmp_path, case, seed, json.dumps(_record(case, seed, ms)))
    lines = suite.summarize(tmp_path, GOLDEN)
    assert "NVIDIA GeForce RTX 4090" in lines[0] and "1024 MiB" in lines[0] and "sha256 abc;" in lines[0]
    header = [c.strip() for c in lines[2].strip("|").split("|")]
    row = [c.strip() for c in next(line for line in lines if line.startswith("| softmax-bf16")).strip("|").split("|")]
    cells = dict(zip(header, row))
    assert cells["seeds"] == "3" and cells["auto warm"] == "200.0" and cells["auto cold"] == "400.0"
    assert cells["auto graph"] == "100.0" and cells["auto ran"] == "naive"
    reference = [c for c in recorded()["cases"] if key(c) == case["key"]]
    ref_auto = sorted(c["methods"]["ragged-auto"]["warm_ms"] for c in reference)[1] * 1e3
    assert cells["ref auto warm"] == f"{ref_auto:.1f}"
    assert cells["ref auto / ours"] == f"{ref_auto / 200.0:.2f}x"
    assert "(" in cells["ref fastest other warm"] and "ragged" not in cells["ref fastest other warm"]
    # Cells without records are left out; without a reference the reference columns are.
    assert len([line for line in lines if line.startswith("| ") and "-f32-" in line]) == 0
    assert "ref auto warm" not in suite.summarize(tmp_path)[2]


def test_gate_rejects_a_wrong_output():
    """The suite gates every method's output before timing it."""
    torch = pytest.importorskip("torch")
    from ragged.calibrate import gate
    import numpy as np

    offsets = np.array([0, 3, 3, 7], dtype=np.int64)
    x = torch.randn(7, 4, dtype=torch.float64).float()
    y = torch.stack([x[0:3].sum(0), torch.zeros(4), x[3:7].sum(0)])
    assert gate(torch, "sum", "f32", x, offsets, y, 711)["max_fraction_of_tolerance"] <= 1.0
    y[2, 1] += 1e-2
    with pytest.raises(AssertionError):
        gate(torch, "sum", "f32", x, offsets, y, 711)
