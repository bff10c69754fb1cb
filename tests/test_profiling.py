"""CPU tests of the rocprofv3 summariser (ragged/profiling.py; the
reference's bench/profile.py:120-144 restated for rocprofv3) on a committed
database whose rows were copied from real rocprofv3 runs of C1 and of the
1 GiB copy probe on one MI355X (tests/golden/make_rocprof_fixture.py). The
expected values are aggregated here with SQL, independently of the
summariser's own code."""
from __future__ import annotations

import json
from pathlib import Path
import sqlite3

import pytest

from ragged import profiling

DB = Path(__file__).resolve().parent / "golden" / "rocprof_c1_sample.db"
WORKER = "k_worker<0, float, long, 4, true, false>"
COPY_BYTES = 1 << 30


def sql(query, *args):
    connection = sqlite3.connect(f"file:{DB}?mode=ro", uri=True)
    try:
        return connection.execute(query, args).fetchall()
    finally:
        connection.close()


def test_short_names():
    assert profiling.short_name("void rg::k_worker<0, float, long, 4, true, false>(rg::Params)") == WORKER
    assert profiling.short_name("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"


def test_kernel_stats_from_the_trace():
    stats = profiling.kernel_stats(DB)
    (calls, mean, total), = sql("select count(*), avg(duration), sum(duration) from kernels where name like '%k_worker%'")
    assert stats[WORKER]["calls"] == calls == 23
    assert stats[WORKER]["avg_ns"] == pytest.approx(mean)
    grand = sql("select sum(duration) from kernels")[0][0]
    assert stats[WORKER]["pct"] == pytest.approx(100 * total / grand)
    assert set(stats) == {WORKER, "k_classify<long>"}


def test_counters_copy_factor_and_traffic():
    fetch = profiling.counter_per_dispatch(DB, "FETCH_SIZE")
    (dispatches, mean), = sql("select count(*), avg(value) from counters_collection "
                              "where counter_name = 'FETCH_SIZE' and kernel_name like '%k_worker%'")
    assert fetch[WORKER]["dispatches"] == dispatches == 8 and fetch[WORKER]["mean"] == pytest.approx(mean)
    factor = profiling.copy_factor(DB, DB, COPY_BYTES, "copyBuffer")
    (copy_fetch,), = sql("select avg(value) from counters_collection where counter_name = 'FETCH_SIZE' "
                         "and kernel_name like '%copyBuffer%'")
    (copy_write,), = sql("select avg(value) from counters_collection where counter_name = 'WRITE_SIZE' "
                         "and kernel_name like '%copyBuffer%'")
    # The copy reads and writes 1 GiB: WRITE_SIZE counts KiB exactly, FETCH_SIZE half of the bytes.
    assert copy_write == 1 << 20 and factor["write_bytes_per_unit"] == 1024.0
    assert factor["fetch_bytes_per_unit"] == pytest.approx(COPY_BYTES / copy_fetch) == pytest.approx(2048, rel=1e-4)
    traffic = profiling.traffic(DB, DB, "k_worker", factor)
    (worker_write,), = sql("select avg(value) from counters_collection where counter_name = 'WRITE_SIZE' "
                           "and kernel_name like '%k_worker%'")
    assert traffic["read_bytes"] == pytest.approx(mean * COPY_BYTES / copy_fetch)
    assert traffic["write_bytes"] == pytest.approx(worker_write * 1024)
    assert traffic["bytes"] == pytest.approx(traffic["read_bytes"] + traffic["write_bytes"])


def test_resources_and_report(tmp_path, capsys):
    resources = profiling.kernel_resources(DB)
    vgpr, lds, grid, group = sql("select vgpr_count, lds_size, grid_x, workgroup_x from kernels "
                                 "where name like '%k_worker%' limit 1")[0]
    assert resources[WORKER]["vgpr_count"] == vgpr and resources[WORKER]["lds_size"] == lds
    factor = profiling.copy_factor(DB, DB, COPY_BYTES, "copyBuffer")
    roles = {"classify": {"bytes": 80_008}, "worker": {"bytes": 2_600_000}}
    lines = profiling.report(DB, DB, DB, DB, factor, roles, "c1")
    row = next(line for line in lines if line.startswith("| worker |"))
    cells = [c.strip() for c in row.strip("|").split("|")]
    mean_us = profiling.kernel_stats(DB)[WORKER]["avg_ns"] / 1e3
    assert float(cells[3]) == pytest.approx(mean_us, abs=0.005)
    assert cells[5].startswith(f"{2_600_000 / (mean_us * 1e-6) / 1e9:.0f} (")
    traffic = profiling.traffic(DB, DB, "k_worker", factor)
    assert float(cells[8]) == pytest.approx(traffic["bytes"] / 2_600_000, abs=0.0005)
    (occupancy,), = sql("select avg(value) from counters_collection where counter_name = 'OccupancyPercent' "
                        "and kernel_name like '%k_worker%'")
    assert float(cells[9]) == pytest.approx(occupancy, abs=0.05)
    assert int(cells[13]) == 2 * vgpr and int(cells[18]) == grid // group
    # The command line: the same table from a bench.py --details file.
    details = tmp_path / "details.json"
    details.write_text(json.dumps({"records": [{"select": "auto", "op": "sum", "kernels": roles}]}))
    assert profiling.main(["report", "--stats", str(DB), "--fetch", str(DB), "--write", str(DB), "--occupancy",
                           str(DB), "--copy-fetch", str(DB), "--copy-write", str(DB), "--copy-bytes",
                           str(COPY_BYTES), "--copy-kernel", "copyBuffer", "--details", str(details),
                           "--title", "c1"]) == 0
    assert row in capsys.readouterr().out


def test_csv_formats(tmp_path):
    """rocprofv3 --output-format csv: kernel stats and counter collection."""
    stats = tmp_path / "c1_kernel_stats.csv"
    stats.write_text('"Name","Calls","TotalDurationNs","AverageNs","Percentage"\n'
                     f'"void rg::{WORKER}(rg::Params)",4,40000,10000,80.0\n'
                     '"void rg::k_classify<long>(rg::Params)",4,10000,2500,20.0\n')
    table = profiling.kernel_stats(stats)
    assert table[WORKER] == pytest.approx({"calls": 4, "total_ns": 40000.0, "avg_ns": 10000.0, "pct": 80.0})
    counters = tmp_path / "c1_counter_collection.csv"
    counters.write_text('"Dispatch_Id","Kernel_Name","Counter_Name","Counter_Value"\n'
                        f'1,"void rg::{WORKER}(rg::Params)","FETCH_SIZE",10\n'
                        f'1,"void rg::{WORKER}(rg::Params)","FETCH_SIZE",5\n'
                        f'2,"void rg::{WORKER}(rg::Params)","FETCH_SIZE",7\n'
                        f'2,"void rg::{WORKER}(rg::Params)","WRITE_SIZE",99\n')
    # Rows of one dispatch (one per channel on some ROCm versions) add up.
    assert profiling.counter_per_dispatch(counters, "FETCH_SIZE")[WORKER] == {"dispatches": 2, "sum": 22.0,
                                                                              "mean": 11.0}


def test_item_timeline_known_answers():
    """The fused softmax's item trace reduced per class, with the merge time
    of each chunk class split into waiting for the segment's last chunk,
    the chain after it and the later wake-ups (ticks of a 1 MHz clock = µs)."""
    def record(ticket, start, loaded, published, merged, end, kind, rows):
        return [ticket, 100 + start, 100 + loaded, 100 + published, 100 + merged, 100 + end, 0, kind + (rows << 8)]
    trace = [
        record(0, 0, 4, 6, 20, 24, 2, 256),      # tree segment: 3 chunks, last publishes at 9
        record(1, 0, 5, 8, 18, 23, 2, 256),
        record(2, 1, 6, 9, 17, 21, 2, 40),
        record(3, 2, 3, 4, 6, 8, 1, 256),        # direct segment: published 4 and 5, merged 6 and 7
        record(4, 2, 3, 5, 7, 9, 1, 100),
        record(5, 3, 4, 5, 30, 31, 1 + 4, 256),  # deferred: left out of the split
        record(6, 3, 4, 6, 31, 32, 1, 10),
        record(7, 4, 6, 8, 8, 10, 0, 200),       # whole segment
        [0] * 8,                                  # unused record
    ]
    summary = profiling.item_timeline(trace, clock_khz=1000, part_rows=256, bins=4)
    assert summary["items"] == 8 and summary["span_us"] == 32.0
    whole = summary["classes"]["whole"]
    assert whole["items"] == 1 and whole["phases_us"] == {"load_max": 2.0, "exp_sum": 2.0, "merge": 0.0, "store": 2.0}
    tree = summary["classes"]["tree"]["merge_split"]
    # merge time 14 + 10 + 8 = 32; last sibling (9-6) + (9-8) = 4; chain (17-9) x 3 = 24; spread 4
    assert tree == {"segments": 1, "merge_workgroup_us": 32.0, "last_sibling": 0.125, "chain": 0.75,
                    "wake_spread": 0.125, "chain_median_us": 8.0}
    direct = summary["classes"]["direct"]
    assert direct["items"] == 4 and direct["deferred"] == 1
    # merge 2 + 2 = 4; last sibling 1; chain (6-5) x 2 = 2; spread 1
    assert direct["merge_split"] == {"segments": 1, "merge_workgroup_us": 4.0, "last_sibling": 0.25, "chain": 0.5,
                                     "wake_spread": 0.25, "chain_median_us": 1.0}
    # Items live and merging at t = 4, 12, 20, 28.
    assert summary["profile"] == [[8, 1], [5, 5], [5, 2], [2, 2]]
    assert profiling.item_timeline([[0] * 8], clock_khz=1000, part_rows=256) == {"items": 0}


def test_call_passes_known_answers(tmp_path, capsys):
    """Two passes of two calls each after one skipped call, from a database
    in the rocpd layout (dispatch and symbol tables, no kernels view), with a
    foreign kernel in between that is ignored; values in ns, hand-computed."""
    db = tmp_path / "trace.db"
    connection = sqlite3.connect(db)
    connection.execute("create table rocpd_info_kernel_symbol (id integer, kernel_name text)")
    connection.execute("create table rocpd_kernel_dispatch (kernel_id integer, start integer, end integer)")
    connection.executemany("insert into rocpd_info_kernel_symbol values (?, ?)",
                           [(1, "rg::k_classify<long>(rg::Params)"),
                            (2, "void rg::k_softmax_fused<__bf16, long, 8, 16, false, false>(rg::Params)"),
                            (3, "at::native::copy_kernel")])
    dispatches = [(1, 0, 10_000), (2, 10_000, 400_000),                          # skipped call
                  (1, 400_000, 411_000), (2, 411_000, 890_000),                  # pass 1: back to back
                  (1, 890_000, 901_000), (2, 901_000, 1_380_000),
                  (3, 1_380_000, 1_390_000),                                     # foreign kernel
                  (1, 1_400_000, 1_410_000), (2, 1_416_000, 1_876_000),          # pass 2: gaps of 6 and 10 µs
                  (1, 1_886_000, 1_896_000), (2, 1_902_000, 2_362_000)]
    connection.executemany("insert into rocpd_kernel_dispatch values (?, ?, ?)", dispatches)
    connection.commit()
    connection.close()
    rows = profiling.call_passes(profiling.dispatch_times(db), "k_classify", "k_softmax_fused", 1, 2, 2)
    assert rows[0] == {"calls": 2, "per_call_us": 490.0, "first_us": 11.0, "gap_first_last_us": 0.0,
                       "last_us": 479.0, "last_min_us": 479.0, "last_max_us": 479.0, "gap_next_call_us": 0.0}
    assert rows[1] == {"calls": 2, "per_call_us": 481.0, "first_us": 10.0, "gap_first_last_us": 6.0,
                       "last_us": 460.0, "last_min_us": 460.0, "last_max_us": 460.0, "gap_next_call_us": 10.0}
    with pytest.raises(ValueError, match="pass 1"):
        profiling.call_passes(profiling.dispatch_times(db), "k_classify", "k_softmax_fused", 1, 3, 2)
    assert profiling.main(["dispatches", str(db), "--skip", "1", "--steps", "2"]) == 0
    out = capsys.readouterr().out
    assert "| 1 | 2 | 490.0 | 11.00 | 0.00 | 479.00 (479.0-479.0) | 0.00 |" in out
    assert "| 2 | 2 | 481.0 | 10.00 | 6.00 | 460.00 (460.0-460.0) | 10.00 |" in out


def _bench_module():
    import importlib.util
    import sys
    root = Path(__file__).resolve().parents[1]
    spec = importlib.util.spec_from_file_location("bench_under_test", root / "bench.py")
    module = importlib.util.module_from_spec(spec)
    argv = sys.argv
    try:
        sys.argv = ["bench.py"]
        spec.loader.exec_module(module)
    finally:
        sys.argv = argv
    return module


def test_bench_finds_the_committed_traffic_summary(monkeypatch):
    """bench.py's roofline.traffic comes from the committed rocprofv3 summary
    of the dominant kernel (profiles/<role>_<workload>_<shape>_traffic.json)
    when it was measured with the library the process loads, and is null
    otherwise."""
    from ragged import native
    bench = _bench_module()
    root = Path(__file__).resolve().parents[1]
    summary = json.loads((root / "profiles" / "fused_c5_softmax_bf16_d128_longtail_traffic.json").read_text())
    monkeypatch.setattr(native, "library_sha256", lambda: summary["library_sha256"])
    found = bench.measured_traffic("c5", "fused")
    assert found == {"bytes": int(round(summary["bytes"])),
                     "source": "profiles/fused_c5_softmax_bf16_d128_longtail_traffic.json"}
    assert 1.0 < found["bytes"] / summary["algorithmic_bytes"] < 1.1
    monkeypatch.setattr(native, "library_sha256", lambda: "0" * 64)
    assert bench.measured_traffic("c5", "fused") is None
    assert bench.measured_traffic("c5", None) is None


def test_bench_refuses_more_than_one_gpu(capsys):
    """One GPU only: --gpus N>1 exits with status 2 and says so, before
    touching a device."""
    bench = _bench_module()
    assert bench.main(["--gpus", "2"]) == 2
    assert "one GPU only" in capsys.readouterr().err
