"""CPU tests of the cost-model calibration (reference test_calibrate.py:16-41:
known coefficients are recovered from synthetic timings) and of the fixed
suites it measures."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from ragged import calibrate
from ragged.optimizations import Optimizations
from ragged.selection import CostModel, features

TRUTH = {"reduce": {"classified": [20.0, 0.02, 0.0, 0.5, 0.0, 0.0, 0.0, 0.0],
                    "naive": [8.0, 0.02, 30.0, 1.0, 3.0, 0.5, 0.0, 0.0]},
         "softmax": {"classified": [25.0, 0.03, 0.0, 0.8, 0.0, 0.0, 0.0, 0.0],
                     "naive": [8.0, 0.03, 60.0, 2.0, 9.0, 1.0, 0.0, 0.0]},
         "softmax_fused": {"classified": [25.0, 0.03, 0.0, 12.0, 0.0, 0.0, 0.0, 0.0],
                           "naive": [8.0, 0.03, 60.0, 3.0, 0.0, 1.0, 0.0, 0.0]}}


def synthetic_records(cases, truth):
    records = []
    for case in cases:
        # Lengths are not generated here: max_len from the distribution's cap.
        max_len = case.n if case.distribution == "burst" else max(1, case.n // case.b * 8)
        mapping = Optimizations().geometry(case.d, case.dtype)[2]
        row = np.array(features(case.n, case.b, case.d, max_len, case.element_bytes, case.op,
                                flat=mapping == "flat"))
        fused = case.op == "softmax" and case.d >= 8
        fam = ("softmax_fused" if fused else "softmax") if case.op == "softmax" else "reduce"
        us = {s: float(row @ np.array(truth[fam][s])) for s in ("classified", "naive")}
        records.append({**case.__dict__, "key": case.key, "max_len": max_len, "fused": fused, "mapping": mapping,
                        "us": us})
    return records


def test_suites_are_fixed_and_disjoint():
    train, heldout = calibrate.suite("train"), calibrate.suite("heldout")
    assert train == calibrate.suite("train") and len(train) == 240 and len(heldout) == 150
    assert {c.d for c in train}.isdisjoint({c.d for c in heldout})
    assert {c.key for c in train}.isdisjoint({c.key for c in heldout})
    # Some held-out working sets (rows read plus rows written) exceed the
    # 256 MiB Infinity Cache.
    assert any(c.n * c.d * c.element_bytes * (2 if c.op == "softmax" else 1) > 256 << 20 for c in heldout)


def test_fit_recovers_known_coefficients():
    records = synthetic_records(calibrate.suite("train")[::3], TRUTH)
    data = calibrate.fit(records)
    model = CostModel.from_dict(data)
    for record in records[:20]:
        for schedule in ("classified", "naive"):
            predicted = model.predict(schedule, record["op"], record["n"], record["b"], record["d"],
                                      record["max_len"], 2 if record["dtype"] == "bf16" else 4,
                                      fused=record["fused"], flat=record["mapping"] == "flat")
            assert predicted == pytest.approx(record["us"][schedule], rel=1e-3)
    assert calibrate.evaluate(model, records)["share"] == 1.0


def test_evaluate_counts_within_three_percent():
    records = synthetic_records(calibrate.suite("heldout")[:10], TRUTH)
    model = CostModel.from_dict({"version": 4, "coefficients": TRUTH, "margin": 0.0, "l2_mib": 32.0,
                                 "mall_mib": 256.0})
    report = calibrate.evaluate(model, records)
    assert report["within_3pct"] == 10 and not report["misses"]
    # A model that always picks the slower schedule misses every case where
    # the schedules differ by more than 3%.
    swapped = json.loads(json.dumps(TRUTH))
    for fam in swapped:
        swapped[fam]["classified"], swapped[fam]["naive"] = TRUTH[fam]["naive"], TRUTH[fam]["classified"]
    bad = CostModel.from_dict({"version": 4, "coefficients": swapped, "margin": 0.0, "l2_mib": 32.0,
                               "mall_mib": 256.0})
    expected = sum(1 for r in records if max(r["us"].values()) > min(r["us"].values()) * 1.03)
    assert len(calibrate.evaluate(bad, records)["misses"]) == expected


def test_shipped_model_meets_the_heldout_target():
    """The committed cost model, fitted on the committed MI355X training
    measurements only, chooses within 3% of the faster schedule on at least
    90% of the committed held-out measurements (suite shapes disjoint from
    training)."""
    base = Path(calibrate.__file__).with_name("calibration")
    train, heldout = calibrate.load(base / "train.jsonl"), calibrate.load(base / "heldout.jsonl")
    assert {r["key"] for r in train} == {c.key for c in calibrate.suite("train")}
    assert {r["key"] for r in heldout} == {c.key for c in calibrate.suite("heldout")}
    model = CostModel.load()
    report = calibrate.evaluate(model, heldout)
    assert report["cases"] == 150 and report["share"] >= 0.90
    assert model.calibration["heldout_within_3pct"] == report["share"]
    # Refitting the training file reproduces the shipped coefficients.
    refit = calibrate.fit(train)
    for fam, schedules in refit["coefficients"].items():
        for schedule, coefficients in schedules.items():
            assert coefficients == pytest.approx(list(model.coefficients[fam][schedule]), rel=1e-4, abs=1e-6)
    assert refit["margin"] == model.margin


def test_transfer_onto_the_shipped_measurements_reproduces_the_shipped_model(tmp_path):
    """`transfer` (reference bench/calibrate.py:229-272) refits on another
    device's train measurements: run on the measurements the shipped model
    was fitted on, its refit equals the shipped model and scores the same
    held-out share; the CLI writes the refit and prints the report."""
    directory = Path(calibrate.__file__).with_name("calibration")
    train = calibrate.load(directory / "train.jsonl")
    heldout = calibrate.load(directory / "heldout.jsonl")
    shipped = CostModel.load()
    data, report = calibrate.transfer(train, heldout, shipped)
    assert data["coefficients"] == json.loads(Path(calibrate.__file__).with_name("cost_model.json").read_text())[
        "coefficients"]
    assert data["margin"] == shipped.margin
    assert report["heldout_cases"] == 150
    recorded = round(shipped.calibration["heldout_within_3pct"] * 150)
    assert report["shipped"]["within_3pct"] == report["refitted"]["within_3pct"] == recorded
    out = tmp_path / "refit.json"
    assert calibrate.main(["transfer", str(directory / "train.jsonl"), str(directory / "heldout.jsonl"),
                           "--out", str(out)]) == 0
    assert json.loads(out.read_text())["coefficients"] == data["coefficients"]


def test_transfer_gives_the_device_l2_to_the_shipped_model():
    """The "shipped with the device's L2" variant passes each record's
    measured L2 capacity to the model; records without one keep the model's."""
    shipped = CostModel.load()
    record = {"op": "sum", "dtype": "f32", "d": 128, "n": 1 << 22, "b": 4096, "distribution": "uniform",
              "seed": 1, "key": "k", "max_len": 2048, "fused": False, "mapping": "row",
              "us": {"classified": 100.0, "naive": 100.0}}
    seen = []

    class Spy(CostModel):
        def choose(self, *args, **kwargs):
            seen.append(kwargs.get("l2_mib"))
            return super().choose(*args, **kwargs)

    spy = Spy.from_dict(json.loads(Path(calibrate.__file__).with_name("cost_model.json").read_text()))
    calibrate.evaluate(spy, [record, {**record, "l2_mib": 8.0}], device_l2=True)
    calibrate.evaluate(spy, [{**record, "l2_mib": 8.0}])
    assert seen == [None, 8.0, None]
    assert shipped.l2_mib == 32.0
