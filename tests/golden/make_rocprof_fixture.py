"""Builds tests/golden/rocprof_c1_sample.db: the rows ragged/profiling.py
reads, copied from real rocprofv3 (ROCm 7.2) databases of one MI355X run,

    rocprofv3 --kernel-trace --stats -o c1 -- python3 bench.py --config c1 --seeds 711 --steps 10 --warmup 2 --no-cpu
    rocprofv3 --pmc FETCH_SIZE -o c1 -- python3 bench.py --config c1 --seeds 711 --steps 3 --warmup 1 --no-cpu
    rocprofv3 --pmc WRITE_SIZE ...                  (same command)
    rocprofv3 --pmc OccupancyPercent MeanOccupancyPerCU VALUBusy MemUnitStalled ...   (same command)
    rocprofv3 --pmc FETCH_SIZE -o copy -- python3 bench.py --copy-probe 1024 --steps 3
    rocprofv3 --pmc WRITE_SIZE -o copy -- python3 bench.py --copy-probe 1024 --steps 3

keeping the library's kernels of the c1 runs and torch's copy kernel of the
copy-probe runs: table `kernels` (the
columns of the view of that name) and table `counters_collection`
(dispatch_id, kernel_name, counter_name, value), every counter run in one
table (profiling.py filters by counter name). Usage:

    python tests/golden/make_rocprof_fixture.py PROF_DIR
"""
from __future__ import annotations

from pathlib import Path
import sqlite3
import sys

KERNEL_COLUMNS = ("name", "duration", "grid_x", "workgroup_x", "lds_size", "static_lds_size", "scratch_size",
                  "static_scratch_size", "vgpr_count", "accum_vgpr_count", "sgpr_count")
LIBRARY, COPY = "rg::", "copyBuffer"   # the library's kernels (c1 runs), torch's copy (copy-probe runs)


def main(prof: Path) -> int:
    out = Path(__file__).with_name("rocprof_c1_sample.db")
    out.unlink(missing_ok=True)
    db = sqlite3.connect(out)
    db.execute(f"create table kernels ({', '.join(KERNEL_COLUMNS)})")
    db.execute("create table counters_collection (dispatch_id, kernel_name, counter_name, value)")
    src = sqlite3.connect(f"file:{prof / 'c1_stats' / 'c1_results.db'}?mode=ro", uri=True)
    rows = [r for r in src.execute(f"select {', '.join(KERNEL_COLUMNS)} from kernels order by start")
            if LIBRARY in r[0]]
    db.executemany(f"insert into kernels values ({', '.join('?' * len(KERNEL_COLUMNS))})", rows)
    for run in ("c1_fetch/c1", "c1_write/c1", "c1_occ/c1", "copy_fetch/copy", "copy_write/copy"):
        src = sqlite3.connect(f"file:{prof / (run + '_results.db')}?mode=ro", uri=True)
        keep = COPY if run.startswith("copy") else LIBRARY
        rows = [r for r in src.execute("select dispatch_id, kernel_name, counter_name, value from counters_collection")
                if keep in r[1]]
        db.executemany("insert into counters_collection values (?, ?, ?, ?)", rows)
    db.commit()
    db.execute("vacuum")
    db.close()
    print(f"wrote {out} ({out.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main(Path(sys.argv[1])))
