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

TRUTH = {"reduce": {"classified": [20.0, 0.02, 0.0, 0.5, 0.0, 0.0, 0.0, 0.0, 0.01, 0.01, 0.0],
                    "naive": [8.0, 0.02, 30.0, 1.0, 3.0, 0.5, 0.0, 0.0, 0.005, 0.0, 20.0]},
         "softmax": {"classified": [25.0, 0.03, 0.0, 0.8, 0.0, 0.0, 0.0, 0.0, 0.02, 0.02, 0.0],
                     "naive": [8.0, 0.03, 60.0, 2.0, 9.0, 1.0, 0.0, 0.0, 0.0, 0.0, 40.0]},
         "softmax_fused": {"classified": [25.0, 0.03, 0.0, 12.0, 0.0, 0.0, 0.0, 0.0, 0.01, 0.01, 0.0],
                           "naive": [8.0, 0.03, 60.0, 3.0, 0.0, 1.0, 0.0, 0.0, 0.03, 0.0, 30.0]}}
NO_MARGINS = {"reduce": 0.0, "softmax": 0.0, "softmax_fused": 0.0}


def synthetic_records(cases, truth):
    records = []
    for case in cases:
        # Lengths are not generated here: max_len from the distribution's
        # cap, above every alone_rows (64), so the runtime consults the model.
        max_len = case.n if case.distribution == "burst" else max(65, case.n // case.b * 8)
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
    suites = {name: calibrate.suite(name) for name in calibrate.SUITES}
    assert suites["train"] == calibrate.suite("train")
    assert {name: len(cases) for name, cases in suites.items()} == {
        "train": 330, "train_dense": 420, "heldout": 150, "heldout2": 150, "heldout3": 150, "heldout4": 150,
        "heldout5": 150, "heldout6": 150, "heldout7": 150, "heldout8": 150, "heldout9": 150, "heldout10": 150,
        "heldout11": 150, "heldout12": 150}
    held = [name for name in suites if name.startswith("heldout")]
    pairs = [(a, b) for a in held for b in held if a < b] + [(t, h) for t in ("train", "train_dense") for h in held]
    for a, b in pairs:
        assert {c.d for c in suites[a]}.isdisjoint({c.d for c in suites[b]}), (a, b)
        assert {c.b for c in suites[a]}.isdisjoint({c.b for c in suites[b]}), (a, b)
        assert {c.key for c in suites[a]}.isdisjoint({c.key for c in suites[b]}), (a, b)
    heldout2 = suites["heldout2"]
    # Some working sets (rows read plus rows written) of most held-out suites
    # (the shipped model's heldout8 among them) exceed the 256 MiB Infinity Cache.
    for suite in (suites[name] for name in ("heldout", "heldout2", "heldout3", "heldout5", "heldout6", "heldout7",
                                            "heldout8", "heldout9", "heldout10", "heldout11", "heldout12")):
        assert any(c.n * c.d * c.element_bytes * (2 if c.op == "softmax" else 1) > 256 << 20 for c in suite)
    # heldout2's shapes: fixed by its seed (a change of the suite would
    # silently unfreeze it).
    assert [c.key for c in heldout2[:3]] == FROZEN_HELDOUT2_HEAD
    assert [c.key for c in suites["heldout6"][:3]] == FROZEN_HELDOUT6_HEAD
    assert [c.key for c in suites["heldout7"][:3]] == FROZEN_HELDOUT7_HEAD
    assert [c.key for c in suites["heldout8"][:3]] == FROZEN_HELDOUT8_HEAD
    assert [c.key for c in suites["heldout9"][:3]] == FROZEN_HELDOUT9_HEAD
    assert [c.key for c in suites["heldout10"][:3]] == FROZEN_HELDOUT10_HEAD
    assert [c.key for c in suites["heldout11"][:3]] == FROZEN_HELDOUT11_HEAD
    assert [c.key for c in suites["heldout12"][:3]] == FROZEN_HELDOUT12_HEAD


FROZEN_HELDOUT2_HEAD = ["sum-f32-d3-n262144-b8192-long_tail-s9000", "sum-f32-d3-n262144-b8192-burst-s9001",
                        "sum-f32-d3-n2097152-b8192-uniform-s9002"]
FROZEN_HELDOUT6_HEAD = ["sum-f32-d13-n181484-b448-long_tail-s25000", "sum-f32-d13-n181484-b57344-uniform-s25001",
                        "sum-f32-d13-n181484-b57344-bimodal-s25002"]
FROZEN_HELDOUT7_HEAD = ["sum-f32-d15-n192238-b320-burst-s29000", "sum-f32-d15-n192238-b320-exponential-s29001",
                        "sum-f32-d15-n192238-b28672-burst-s29002"]

FROZEN_HELDOUT8_HEAD = ["sum-f32-d17-n200463-b6656-bimodal-s33000", "sum-f32-d17-n1603704-b576-uniform-s33001", "sum-f32-d17-n1603704-b576-exponential-s33002"]
FROZEN_HELDOUT9_HEAD = ["sum-f32-d19-n206955-b704-burst-s37000", "sum-f32-d19-n1655646-b704-uniform-s37001",
                        "sum-f32-d19-n1655646-b704-burst-s37002"]
FROZEN_HELDOUT10_HEAD = ["sum-f32-d21-n1697694-b832-burst-s41000", "sum-f32-d21-n1697694-b4608-burst-s41001",
                         "sum-f32-d21-n3395388-b832-bimodal-s41002"]
FROZEN_HELDOUT11_HEAD = ["sum-f32-d23-n216553-b61440-uniform-s45000", "sum-f32-d23-n216553-b61440-exponential-s45001",
                         "sum-f32-d23-n1732429-b960-burst-s45002"]
FROZEN_HELDOUT12_HEAD = ["sum-f32-d25-n220200-b1088-bimodal-s49000", "sum-f32-d25-n220200-b1088-exponential-s49001",
                         "sum-f32-d25-n220200-b69632-uniform-s49002"]


@pytest.mark.parametrize("op", ["sum", "max", "softmax"])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_gate_accepts_the_oracle_and_rejects_a_planted_error(op, dtype):
    """calibrate.gate (torch float64 on any device) passes outputs computed
    by the float64 NumPy oracle and rounded to the output dtype, and fails
    one with a single planted error in a sampled segment."""
    import oracle
    torch = pytest.importorskip("torch")
    from ragged.workloads import make_lengths, offsets_from_lengths
    lengths = make_lengths("long_tail", 300, seed=5, total_elements=20_000)
    offsets = offsets_from_lengths(lengths, "i64")
    rng = np.random.default_rng(1)
    values = rng.normal(size=(int(offsets[-1]), 3)).astype(np.float32)
    if dtype == "bf16":
        values = oracle.quantize_bf16(values)
    function = {"sum": oracle.segment_sum, "max": oracle.segment_max, "softmax": oracle.segment_softmax}[op]
    expected = function(values, offsets).astype(np.float32)
    if dtype == "bf16":
        expected = oracle.quantize_bf16(expected)
    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.from_numpy(values).to(tdtype)
    y = torch.from_numpy(expected).to(tdtype)
    report = calibrate.gate(torch, op, dtype, x, offsets, y, seed=3)
    assert report["segments"] >= 64 and report["max_fraction_of_tolerance"] <= 1.0
    longest = int(np.argmax(lengths))
    row = int(offsets[longest]) if op == "softmax" else longest
    bad = y.clone()
    # Beyond the tolerance: a sum's bound scales with the sum of |x|.
    bad[row, 1] = bad[row, 1].float() + (1e4 if op == "sum" else 0.5)
    with pytest.raises(AssertionError):
        calibrate.gate(torch, op, dtype, x, offsets, bad, seed=3)


def test_evaluate_cold_uses_cold_timings():
    records = synthetic_records(calibrate.suite("heldout2")[:12], TRUTH)
    model = CostModel.from_dict({"version": 6, "coefficients": TRUTH, "margins": NO_MARGINS, "l2_mib": 32.0,
                                 "mall_mib": 256.0})
    # Cold timings that reverse every choice: warm all good, cold only the ties.
    for r in records:
        r["us_cold"] = {"classified": r["us"]["naive"], "naive": r["us"]["classified"]}
    assert calibrate.evaluate(model, records)["within_3pct"] == 12
    ties = sum(1 for r in records if max(r["us"].values()) <= min(r["us"].values()) * 1.03)
    assert calibrate.evaluate(model, records, cold=True)["within_3pct"] == ties
    assert calibrate.evaluate(model, records[:3] + [{k: v for k, v in records[3].items() if k != "us_cold"}],
                              cold=True)["cases"] == 3


def test_fit_recovers_known_coefficients():
    records = synthetic_records(calibrate.suite("train")[::3], TRUTH)
    data = calibrate.fit(records, "linear")
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
    model = CostModel.from_dict({"version": 6, "coefficients": TRUTH, "margins": NO_MARGINS, "l2_mib": 32.0,
                                 "mall_mib": 256.0})
    report = calibrate.evaluate(model, records)
    assert report["within_3pct"] == 10 and not report["misses"]
    # A model that always picks the slower schedule misses every case where
    # the schedules differ by more than 3%.
    swapped = json.loads(json.dumps(TRUTH))
    for fam in swapped:
        swapped[fam]["classified"], swapped[fam]["naive"] = TRUTH[fam]["naive"], TRUTH[fam]["classified"]
    bad = CostModel.from_dict({"version": 6, "coefficients": swapped, "margins": NO_MARGINS, "l2_mib": 32.0,
                               "mall_mib": 256.0})
    expected = sum(1 for r in records if max(r["us"].values()) > min(r["us"].values()) * 1.03)
    assert len(calibrate.evaluate(bad, records)["misses"]) == expected


TRAIN_SUITES = ("train", "train_dense", "heldout", "heldout2", "heldout3", "heldout4", "heldout5", "heldout6",
                "heldout7", "heldout8", "heldout9", "heldout10")
HELDOUT = "heldout11"
# The commit that froze heldout11's definition (and pinned its first keys)
# before any of it was measured.
HELDOUT_COMMIT = "dc2241397ed0052ea9de74c56e5ce5439ecb535f"


def test_shipped_model_records_its_heldout_scores():
    """The committed cost model (version 7) is the fit of the committed
    MI355X measurements of every suite but heldout11, pooled (refitting
    reproduces its ensembles and margins), all measured with the library
    whose sha256 it records; its choices, as run(select="auto") makes them,
    are scored on heldout11 (its definition committed before any of it was
    measured, disjoint shapes, scored once) warm and cold exactly as
    recorded, and its leave-one-suite-out scores over the train suites are
    recorded as recomputed. Every measured case passed the sampled
    correctness gate."""
    base = Path(calibrate.__file__).with_name("calibration")
    files = {name: calibrate.load(base / f"{name}.jsonl") for name in TRAIN_SUITES + (HELDOUT,)}
    for name, records in files.items():
        assert {r["key"] for r in records} == {c.key for c in calibrate.suite(name)}, name
        assert all(0.0 <= g <= 1.0 for r in records for g in r["gate"].values()), name
        assert all(r["us_cold"]["classified"] > 0 and r["us_cold"]["naive"] > 0 for r in records), name
    model = CostModel.load()
    shas = {r["library_sha256"] for records in files.values() for r in records}
    assert shas == {model.calibration["library_sha256"]}
    heldout = files[HELDOUT]
    warm, cold = calibrate.evaluate(model, heldout), calibrate.evaluate(model, heldout, cold=True)
    assert warm["cases"] == cold["cases"] == 150
    assert model.calibration["heldout_file"] == f"{HELDOUT}.jsonl"
    assert model.calibration["heldout_definition_commit"] == HELDOUT_COMMIT
    assert model.calibration["train_file"] == " + ".join(f"{name}.jsonl" for name in TRAIN_SUITES)
    assert model.calibration["heldout_within_3pct"] == warm["share"]
    assert model.calibration["heldout_within_3pct_cold"] == cold["share"]
    assert model.version == 7
    refit = calibrate.fit([r for name in TRAIN_SUITES for r in files[name]])
    shipped = json.loads(Path(calibrate.__file__).with_name("cost_model.json").read_text())
    assert json.loads(calibrate.dump_model(refit))["ensembles"] == shipped["ensembles"]
    assert refit["margins"] == model.margins
    loso = calibrate.leave_one_suite_out({name: files[name] for name in TRAIN_SUITES})
    assert loso == model.calibration["leave_one_suite_out"]


# The commit that froze heldout12's definition (and pinned its first keys)
# before any of it was measured; the shipped model was scored on it once.
HELDOUT12_COMMIT = "ec0b013"


def test_shipped_model_records_its_heldout12_check():
    """heldout12, defined and committed alone before any of it was measured
    and measured with the library the model records, scores the shipped
    model warm and cold exactly as recorded in its checks (at least 90%);
    every measured case passed the sampled correctness gate."""
    base = Path(calibrate.__file__).with_name("calibration")
    records = calibrate.load(base / "heldout12.jsonl")
    assert {r["key"] for r in records} == {c.key for c in calibrate.suite("heldout12")}
    assert all(0.0 <= g <= 1.0 for r in records for g in r["gate"].values())
    model = CostModel.load()
    assert {r["library_sha256"] for r in records} == {model.calibration["library_sha256"]}
    recorded = model.calibration["checks"]["heldout12.jsonl"]
    warm, cold = calibrate.evaluate(model, records), calibrate.evaluate(model, records, cold=True)
    assert recorded == {"cases": 150, "within_3pct": warm["share"], "within_3pct_cold": cold["share"]}
    assert warm["share"] >= 0.9 and cold["share"] >= 0.9


def test_transfer_onto_the_shipped_measurements_reproduces_the_shipped_model(tmp_path):
    """`transfer` (reference bench/calibrate.py:229-272) refits on another
    device's train measurements: run on the measurements the shipped model
    was fitted on, its refit equals the shipped model and scores the same
    held-out share; the CLI writes the refit and prints the report."""
    directory = Path(calibrate.__file__).with_name("calibration")
    train = [r for name in TRAIN_SUITES for r in calibrate.load(directory / f"{name}.jsonl")]
    heldout = calibrate.load(directory / f"{HELDOUT}.jsonl")
    shipped = CostModel.load()
    data, report = calibrate.transfer(train, heldout, shipped)
    assert json.loads(calibrate.dump_model(data))["ensembles"] == json.loads(
        Path(calibrate.__file__).with_name("cost_model.json").read_text())["ensembles"]
    assert data["margins"] == shipped.margins
    assert report["heldout_cases"] == 150
    recorded = round(shipped.calibration["heldout_within_3pct"] * 150)
    assert report["shipped"]["within_3pct"] == report["refitted"]["within_3pct"] == recorded
    out = tmp_path / "refit.json"
    pooled = tmp_path / "train_pooled.jsonl"
    pooled.write_text("".join(json.dumps(record) + "\n" for record in train))
    assert calibrate.main(["transfer", str(pooled), str(directory / f"{HELDOUT}.jsonl"), "--out", str(out)]) == 0
    assert json.loads(out.read_text())["ensembles"] == json.loads(calibrate.dump_model(data))["ensembles"]


def test_evaluate_scores_the_short_segment_rule_before_the_model():
    """run(select="auto") takes the one-launch short-segment schedule when
    max_len lets one lane group reduce every segment alone, without the
    model; evaluate scores that choice (measured as "classified"), and fit
    leaves such cases out of the terms."""
    from ragged import native
    spec = native.make_spec("sum", "f32", "i64", 3)
    assert spec.alone_rows == 32 and spec.t_wave > 0
    base = {"op": "sum", "dtype": "f32", "d": 3, "n": 1 << 16, "b": 4096, "distribution": "uniform", "seed": 1,
            "key": "k", "fused": False, "mapping": "row", "us": {"classified": 10.0, "naive": 30.0}}
    always_naive = json.loads(json.dumps(TRUTH))
    for fam in always_naive:
        always_naive[fam]["naive"] = [0.0] * len(TRUTH[fam]["naive"])
    model = CostModel.from_dict({"version": 6, "coefficients": always_naive, "margins": NO_MARGINS,
                                 "l2_mib": 32.0, "mall_mib": 256.0})
    short = {**base, "max_len": 32}
    long = {**base, "max_len": 33}
    assert calibrate.short_segments(short) and not calibrate.short_segments(long)
    assert [c for _, c in calibrate.choices(model, [short, long])] == ["classified", "naive"]
    assert calibrate.evaluate(model, [short, long])["within_3pct"] == 1


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


def test_leaf_table_follows_the_decisions():
    """Depth 4, heap order, bit i set = node i goes right: no bits is the
    leftmost leaf, all bits the rightmost; root right, then left, left, left
    is nodes 0 -> 2 -> 5 -> 11 -> 23, leaf 8. Bits off the path do not matter."""
    from ragged.selection import _leaf_table
    table = _leaf_table(4)
    assert len(table) == 1 << 15
    assert table[0] == 0 and table[(1 << 15) - 1] == 15
    assert table[1] == 8
    assert table[1 | (1 << 1) | (1 << 3)] == 8          # nodes 1 and 3 are not on that path
    assert table[1 | (1 << 2)] == 12                   # 0 -> 2 -> 6 -> 13 -> 27: leaf 12
    for depth in (1, 2, 3):
        t = _leaf_table(depth)
        assert sorted(set(t.tolist())) == list(range(2**depth))


def _hand_ensemble(base=1.0):
    """One depth-2 tree: root splits statistic 3 at 0.5, its children
    statistic 0 at -1 (left) and statistic 8 at 2 (right)."""
    from ragged.selection import Ensemble
    return Ensemble.from_dict({"base": base, "depth": 2, "features": [[3, 0, 8]],
                               "thresholds": [[0.5, -1.0, 2.0]], "leaves": [[0.1, 0.2, 0.3, 0.4]]})


def test_ensemble_prediction_on_a_hand_built_tree():
    e = _hand_ensemble()
    x = [0.0] * 9
    assert e.log_us(x) == pytest.approx(1.2)            # 3 <= 0.5: left; 0 > -1: right -> leaf 1
    x[0] = -2.0
    assert e.log_us(x) == pytest.approx(1.1)            # leaf 0
    x[3], x[8] = 1.0, 5.0
    assert e.log_us(x) == pytest.approx(1.4)            # right, right -> leaf 3
    x[8] = 2.0
    assert e.log_us(x) == pytest.approx(1.3)            # equal to the threshold goes left
    from ragged.selection import Ensemble
    assert Ensemble.pair_log_us(e, _hand_ensemble(2.0), x) == pytest.approx((1.3, 2.3))


def test_paired_and_single_predictions_agree():
    rng = np.random.default_rng(3)
    from ragged.selection import Ensemble
    def random_ensemble(depth, trees):
        inner = 2**depth - 1
        return Ensemble.from_dict({"base": float(rng.normal()), "depth": depth,
                                   "features": rng.integers(0, 9, (trees, inner)).tolist(),
                                   "thresholds": rng.normal(size=(trees, inner)).tolist(),
                                   "leaves": rng.normal(size=(trees, 2**depth)).tolist()})
    for depth in (3, 4, 5):
        a, b = random_ensemble(depth, 20), random_ensemble(depth, 30)
        for _ in range(50):
            x = rng.normal(size=9)
            assert Ensemble.pair_log_us(a, b, x) == pytest.approx((a.log_us(x), b.log_us(x)), abs=1e-12)


def test_boosted_fit_recovers_a_step():
    """log(µs) that steps with the skew statistic (L over the mean length)
    is recovered by the version-7 fit on both sides of the step."""
    from ragged.selection import host_features
    records = synthetic_records(calibrate.suite("train")[::2], TRUTH)
    element = {"f32": 4, "bf16": 2}
    for r in records:
        x = host_features(r["n"], r["b"], r["d"], r["max_len"], element[r["dtype"]], r["op"],
                          flat=r["mapping"] == "flat")
        r["us"] = {"classified": 40.0 if x[3] > 3 else 20.0, "naive": 30.0}
    data = calibrate.fit(records)
    model = CostModel.from_dict(json.loads(calibrate.dump_model(data)))
    assert model.version == 7
    for r in records[:40]:
        predicted = model.predict("classified", r["op"], r["n"], r["b"], r["d"], r["max_len"], element[r["dtype"]],
                                  fused=r["fused"], flat=r["mapping"] == "flat")
        assert predicted == pytest.approx(r["us"]["classified"], rel=0.02)
    assert calibrate.evaluate(model, records)["share"] == 1.0


def test_malformed_version_7_files_are_rejected():
    from ragged.errors import CacheMismatch
    good = _hand_ensemble().to_dict()
    def model(ensemble):
        return {"version": 7, "margins": NO_MARGINS, "l2_mib": 32.0, "mall_mib": 256.0,
                "ensembles": {f: {"classified": ensemble, "naive": good} for f in NO_MARGINS}}
    CostModel.from_dict(model(good))
    for bad in ({**good, "depth": 3}, {**good, "features": [[3, 0, 9]]}, {**good, "leaves": [[0.1, 0.2, 0.3]]},
                {**good, "thresholds": [[0.5, float("nan"), 2.0]]}, {k: v for k, v in good.items() if k != "base"}):
        with pytest.raises(CacheMismatch):
            CostModel.from_dict(model(bad))
    with pytest.raises(CacheMismatch):
        CostModel.from_dict({**model(good), "version": 8})


def test_each_model_predicts_with_its_own_trees():
    """Models created and dropped one after another (as leave-one-suite-out
    does) each choose by their own ensembles: a cache of flattened trees
    keyed by object identity once served a later model a dropped model's
    trees."""
    import gc
    import math
    rng = np.random.default_rng(11)
    from ragged.selection import host_features
    for _ in range(30):
        def ensemble():
            return {"base": float(rng.normal()), "depth": 4, "features": rng.integers(0, 9, (5, 15)).tolist(),
                    "thresholds": rng.normal(size=(5, 15)).tolist(), "leaves": rng.normal(size=(5, 16)).tolist()}
        model = CostModel.from_dict({"version": 7, "margins": NO_MARGINS, "l2_mib": 32.0, "mall_mib": 256.0,
                                     "ensembles": {f: {"classified": ensemble(), "naive": ensemble()}
                                                   for f in NO_MARGINS}})
        x = host_features(1 << 20, 4096, 32, 5000, 4, "sum")
        _, info = model.choose("sum", 1 << 20, 4096, 32, 5000, 4)
        for schedule in ("classified", "naive"):
            expected = math.exp(model.ensembles["reduce"][schedule].log_us(x))
            assert info["predicted_us"][schedule] == pytest.approx(expected, rel=1e-3, abs=0.01)
        del model
        gc.collect()
