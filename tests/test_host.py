"""CPU tests of the host layer: the C-ABI library's exported symbols and
host-only entry points, the restated input generators against the
reference's recorded hashes, spec validation, checked-mode status decoding,
the cost model's features, and the loud failure when the HIP library is
missing. No test here launches a kernel."""
from __future__ import annotations

import ctypes
import json
from pathlib import Path
import re

import numpy as np
import pytest


from ragged import ProgramSpec
from ragged import native
from ragged.errors import RuntimeUnavailable, ValidationError
from ragged.optimizations import Optimizations
from ragged.selection import access_bytes, features, lane_utilisation
from ragged.validation import CONDITIONS, I64_MAX, raise_for_status
from ragged.workloads import describe, make_lengths, offsets_from_lengths, reference_values, sha256

REPO = Path(__file__).resolve().parents[1]
HEADER = REPO / "include" / "ragged_hip.h"
GOLDEN = REPO / "tests" / "golden" / "reference_cases.json"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(rg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for required in ("rg_abi_version", "rg_last_error", "rg_device_query", "rg_module_create", "rg_plan_create",
                     "rg_run", "rg_check_offsets", "rg_module_resident"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = native.library()
    missing = [name for name in declared_functions() if not hasattr(lib, name)]
    assert not missing, f"declared in {HEADER.name} but not exported: {missing}"


def test_abi_version_and_build_info():
    lib = native.library()
    version = int(re.search(r"#define\s+RG_ABI_VERSION\s+(\d+)", HEADER.read_text()).group(1))
    assert lib.rg_abi_version() == version == native.ABI_VERSION
    info = lib.rg_build_info().decode()
    assert "target=gfx950" in info and "packed-fp32-ops" in info


@pytest.mark.parametrize("dtype,d,capacity", [("bf16", 128, 256), ("f32", 128, 128), ("bf16", 64, 512),
                                              ("f32", 1024, 16)])
def test_register_resident_defaults(dtype, d, capacity):
    """Softmax specs whose rows fit one workgroup's registers default to the
    register-resident schedule, with one chunk = the workgroup's capacity;
    the wave class keeps the streaming worker's threshold, below the block
    class."""
    spec = native.make_spec("softmax", dtype, "i64", d)
    assert native.uses_fused(spec)
    assert spec.part_rows == capacity and spec.t_block == capacity
    streaming = native.make_spec("sum", dtype, "i64", d)
    assert spec.t_wave == min(streaming.t_wave, capacity - 1) and 0 < spec.t_wave < spec.t_block


@pytest.mark.parametrize("d,dtype,alone", [(1, "f32", 64), (2, "f32", 32), (4, "bf16", 16), (3, "f32", 32),
                                           (128, "f32", 32), (256, "bf16", 32), (192, "f32", 0), (1024, "f32", 0)])
def test_alone_rows(d, dtype, alone):
    """Wave-class segments one lane (flat: kLaneElems elements) or one lane
    group (rows of at most 32 vectors: 32 rows) reduces alone; the wave class
    reaches at least as far, and at least 8 KiB of rows."""
    spec = native.make_spec("sum", dtype, "i64", d)
    assert spec.alone_rows == alone
    row = d * (2 if dtype == "bf16" else 4)
    assert spec.t_wave == max(1, alone, 8192 // row) < spec.t_block


def test_reductions_keep_the_class_pipeline():
    for op in ("sum", "max"):
        spec = native.make_spec(op, "f32", "i64", 128)
        assert not native.uses_fused(spec)
        assert 0 < spec.t_wave < spec.t_block and spec.part_rows > 0


def test_spec_defaults_rejects_bad_input():
    lib = native.library()
    spec = native.Spec(9, 0, 1, 128, 1.0, 0, 1, 0, -1, -1, -1)
    assert lib.rg_module_create(0, ctypes.byref(spec), ctypes.byref(ctypes.c_void_p())) != 0
    assert lib.rg_last_error()


def test_generators_match_reference_hashes():
    """Every recorded reference benchmark input (lengths, offsets and, for
    the smaller cases, values) regenerates bit-identically."""
    cases = json.loads(GOLDEN.read_text())["cases"]
    assert len(cases) >= 100
    values_checked = 0
    for case in cases:
        lengths = make_lengths(case["distribution"], case["segments"], seed=case["seed"],
                               total_elements=case["total_elements"], mean_length=case["mean_length"])
        stats = describe(lengths)
        assert stats["lengths_sha256"] == case["lengths_sha256"], case["source"]
        assert stats["histogram_counts"] == case["histogram_counts"]
        assert stats["max_length"] == case["max_length"]
        assert sha256(offsets_from_lengths(lengths, case["offsets_dtype"])) == case["offsets_sha256"]
        if case["elements"] * case["d"] <= 1 << 20:
            values = reference_values(case["seed"], case["elements"], case["d"])
            assert sha256(values) == case["values_sha256"], case["source"]
            values_checked += 1
    assert values_checked >= 20


@pytest.mark.parametrize("kwargs,message", [
    ({"op": "mean"}, "op must be"),
    ({"op": "sum", "dtype": "f16"}, "dtype"),
    ({"op": "sum", "feature_dim": 0}, "feature_dim"),
    ({"op": "sum", "feature_dim": 1025}, "feature_dim"),
    ({"op": "sum", "offsets_dtype": "u64"}, "offsets_dtype"),
    ({"op": "sum", "mask": True}, "mask"),
    ({"op": "max", "alias": "inplace"}, "in-place"),
    ({"op": "softmax", "scale": float("inf")}, "scale"),
])
def test_program_spec_validation(kwargs, message):
    with pytest.raises(ValidationError, match=message):
        ProgramSpec(**kwargs)


def test_spec_identity_is_stable():
    a = ProgramSpec("softmax", "bf16", 128, "i64")
    b = ProgramSpec("softmax", "bf16", 128, "i64")
    c = ProgramSpec("softmax", "bf16", 64, "i64")
    assert a.ir_hash == b.ir_hash != c.ir_hash
    assert ProgramSpec.from_dict(a.to_dict()) == a


def test_status_decoding_known_answers():
    clean = [I64_MAX] * 7
    raise_for_status(clean, b=4)
    status = list(clean)
    status[CONDITIONS.index("nonmonotone")] = 2
    status[CONDITIONS.index("above_n")] = 3
    with pytest.raises(ValidationError) as info:
        raise_for_status(status, b=4)
    assert info.value.errors == {"above_n": 3, "nonmonotone": 2}
    bad = list(clean)
    bad[0] = 1                     # first_nonzero can only be reported at index 0
    with pytest.raises(ValidationError, match="domain"):
        raise_for_status(bad, b=4)
    with pytest.raises(ValidationError, match="layout"):
        raise_for_status(clean[:6], b=4)


def test_cost_model_features_known_answer():
    # N = 2^20 rows, B = 1024, D = 4 f32 (16-byte rows), L = 2^14: W = 16 MiB of rows read + 1024
    # result rows = 16.015625 MiB; S = 2^14*16/2^20 = 0.25 MiB; B/1000 = 1.024; row mapping (F = 0);
    # R*B/1000 = 1.024 * 16/1024; the working set is under the 32 MiB L2; 16-byte accesses (A = 0);
    # one 16-byte vector per row on one lane (u = 1, U = 0).
    assert features(2**20, 1024, 4, 2**14, 4, "sum") == (1.0, 16.015625, 0.25, 1.024, 0.0, 1.024 * 16 / 1024,
                                                          0.0, 0.0, 0.0, 0.0, 0.0)
    assert features(2**20, 1024, 4, 2**14, 4, "sum", flat=True)[4] == 1.024
    # Softmax writes N rows: 128 MiB of rows at D=32 f32 -> 256 MiB moved.
    f = features(2**20, 1024, 32, 2**14, 4, "softmax")
    assert f[1] == 256.0 and f[6] == pytest.approx(256.0 - 32.0) and f[7] == 0.0 and f[8] == 0.0
    # Access width: D=3 f32 reads 4-byte elements (A = 3), D=6 f32 8 bytes (A = 1), D=10 bf16 4 bytes
    # (A = 3), D=2 f32 and D=4 bf16 the flat 16-byte vector (A = 0).
    assert [access_bytes(d, e) for d, e in ((3, 4), (6, 4), (10, 2), (2, 4), (4, 2), (12, 2))] == [4, 8, 4, 16, 16, 8]
    assert features(1000, 10, 3, 100, 4, "sum")[8] == pytest.approx(3 * features(1000, 10, 3, 100, 4, "sum")[1])
    # Lane utilisation of the row mapping: D=80 f32 is 20 vectors on 32 lanes (u = 0.625, U = 0.6),
    # D=13 f32 13 on 16, D=176 bf16 22 on 32, D=1024 f32 256 vectors in 4 passes of 64 lanes (u = 1);
    # W*U and S*U carry U, zero for the flat mapping.
    assert [lane_utilisation(d, e) for d, e in ((80, 4), (13, 4), (176, 2), (1024, 4), (128, 2))] == [
        0.625, 13 / 16, 22 / 32, 1.0, 1.0]
    f = features(1 << 20, 4096, 80, 1000, 4, "sum")
    assert f[9] == pytest.approx(0.6 * f[1]) and f[10] == pytest.approx(0.6 * f[2])
    assert features(1 << 20, 4096, 2, 1000, 4, "sum", flat=True)[9:] == (0.0, 0.0)
    # The same width as the geometry the programs are built with.
    for dtype, element in (("f32", 4), ("bf16", 2)):
        for d in range(1, 300):
            _, vec, mapping = Optimizations().geometry(d, dtype)
            assert access_bytes(d, element) == (16 if mapping == "flat" else vec * element), (d, dtype)



def test_host_features_known_answers():
    """The version-7 statistics: 2^20 rows of 4 f32 (16 B) in 1024 segments,
    longest 2^14 rows: (16 MiB + 1024 result rows) over the 32 MiB L2, 2^10
    segments, a 0.25 MiB longest segment 16x the mean, 16-byte rows and
    accesses on one lane, a 1/64 MiB mean segment; D=80 f32 idles 3/8 of
    its 32 lanes (1/0.625 - 1)."""
    import math
    from ragged.selection import host_features
    x = host_features(2**20, 1024, 4, 2**14, 4, "sum")
    assert x == pytest.approx((math.log2(16.015625 / 32), 10, -2, 4, 4, 0, 0, 0, -6))
    assert host_features(2**20, 1024, 4, 2**14, 4, "softmax")[0] == pytest.approx(0.0)
    assert host_features(2**20, 1024, 4, 2**14, 4, "sum", l2_mib=8.0)[0] == pytest.approx(math.log2(16.015625 / 8))
    assert host_features(1 << 20, 4096, 80, 1000, 4, "sum")[7] == pytest.approx(0.6)
    assert host_features(1 << 20, 4096, 2, 1000, 4, "sum", flat=True)[5:8] == (1.0, 0.0, 0.0)

def test_product_fails_loudly_without_the_library(monkeypatch, tmp_path):
    monkeypatch.setattr(native, "LIBRARY_PATH", tmp_path / "missing.so")
    with pytest.raises(RuntimeUnavailable, match="missing"):
        native.library_sha256()


def test_oracle_is_test_infrastructure_only():
    """Nothing in the product package imports the oracle."""
    for path in (REPO / "ragged-mlir_amd" / "ragged").glob("*.py"):
        text = path.read_text()
        assert not re.search(r"^\s*(from|import)\s+oracle\b", text, flags=re.M), path.name


def test_deferred_rows_bound_known_answers():
    """Rows the register-resident softmax surely defers (segments longer than
    its limit): the caller's longest segment when it exceeds the limit, or
    the rows B segments of at most the limit cannot hold."""
    from ragged.runtime import STREAM_SHARE, deferred_rows_bound
    limit = 896 * 256
    # Four 2^20-row segments: the three others hold at most 3 x limit rows.
    assert deferred_rows_bound(4 << 20, 4, 1 << 20, limit) == (4 << 20) - 3 * limit
    # Sixteen 2^18-row segments (all beyond the limit, but only just): the bound is weak.
    assert deferred_rows_bound(16 << 18, 16, 1 << 18, limit) == (16 << 18) - 15 * limit
    assert deferred_rows_bound(16 << 18, 16, 1 << 18, limit) < STREAM_SHARE * (16 << 18)
    # max_len within the limit: only what B segments of the limit cannot hold.
    assert deferred_rows_bound(4 << 20, 4, limit, limit) == (4 << 20) - 4 * limit
    # C5: the longest segment (200,000 rows) fits; 8192 segments hold any N.
    assert deferred_rows_bound(4_194_304, 8192, 200_000, limit) == 0
    # One segment of half the rows beyond the limit.
    assert deferred_rows_bound(8_388_608, 8193, 4_194_304, limit) == 4_194_304
    assert deferred_rows_bound(8_388_608, 8193, 4_194_304, limit) >= STREAM_SHARE * 8_388_608
    # A long segment that is a small share stays below the share.
    assert deferred_rows_bound(5_194_304, 8193, 1_000_000, limit) < STREAM_SHARE * 5_194_304
    # The decision on the measured inputs: at least half the rows and 1.5 limits.
    from ragged.runtime import streams_long_segments
    assert streams_long_segments(4 << 20, 4, 1 << 20, limit)                       # 2.2x faster streamed
    assert streams_long_segments(8_388_608, 8193, 4_194_304, limit)                # 1.5x
    assert streams_long_segments(4 << 20, 8, 1 << 19, limit)                       # 2.2x
    assert not streams_long_segments(4_194_304, 8192, 200_000, limit)              # C5
    assert not streams_long_segments(5_194_304, 8193, 1_000_000, limit)            # a 19% segment
    assert not streams_long_segments(131_072, 640, 114_860, 896 * 128)             # one round of the drain: 10% slower streamed
    assert not streams_long_segments(int(1.1 * limit) + 517, 3, int(1.1 * limit), limit)   # within 10% either way
    assert streams_long_segments(2 * limit + 517, 3, 2 * limit, limit)                     # 1.4-1.6x
    # No max_len, an empty call or no limit: nothing is known.
    assert deferred_rows_bound(4 << 20, 4, None, limit) == 0
    assert deferred_rows_bound(0, 0, 5, limit) == 0
    assert deferred_rows_bound(10, 1, 10, 0) == 0


def test_stream_part_rows_known_answers():
    """Streaming split parts of about 2 MiB of rows, at most 16,384 rows, and
    beyond the register path's part."""
    from ragged.runtime import stream_part_rows
    assert stream_part_rows(16 * 4, 1024) == 16384          # f32 D=16: 1 MiB (the row cap)
    assert stream_part_rows(128 * 4, 128) == 4096           # f32 D=128: 2 MiB
    assert stream_part_rows(128 * 2, 256) == 8192           # bf16 D=128: 2 MiB
    assert stream_part_rows(1024 * 2, 32) == 1024           # bf16 D=1024: 2 MiB
    assert stream_part_rows(4096 * 4, 8) == 128             # f32 D=4096: 2 MiB
    assert stream_part_rows(128 * 2, 16384) == 32768        # beyond a (hypothetical) large register part


def test_big_part_rows_known_answers():
    """Sum / max calls split into parts of about N/512 rows, at most 4 MiB,
    at least the library's default, which they keep while N/512 is below
    twice it (about 256 MiB of rows). Segments of up to N/1024 rows (at most
    a part, rounded down to an eighth of it) go to the block class."""
    from ragged.runtime import big_block_rows, big_part_rows
    assert big_part_rows(1 << 22, 512, 512) == 8192          # f32 D=128, 2 GiB: 4 MiB parts
    assert big_part_rows(1 << 22, 256, 1024) == 8192         # bf16 D=128, 1 GiB: 2 MiB parts
    assert big_part_rows(1 << 24, 512, 512) == 8192          # 8 GiB: capped at 4 MiB
    assert big_part_rows(1 << 21, 256, 1024) == 4096         # bf16 D=128, 512 MiB: 1 MiB parts
    assert big_part_rows(1_040_746, 512, 512) == 1024        # C2 (508 MiB): 2032 rows per 512th -> 1024
    assert big_part_rows(524_288, 512, 512) == 1024          # f32 D=128, exactly 256 MiB
    assert big_part_rows(524_287, 512, 512) == 512           # one row less: the default
    assert big_part_rows(1 << 20, 304, 862) == 1724          # the suites' largest (f32 D=76, 304 MiB)
    assert big_part_rows(1 << 18, 512, 512) == 512           # 128 MiB: the default
    assert big_part_rows(1 << 27, 8, 32768) == 262144        # f32 D=2, 1 GiB: N/512 rows (2 MiB)
    assert big_block_rows(1 << 23, 8192, 1024) == 8192        # N/1024 = 8192 rows
    assert big_block_rows(1 << 22, 8192, 1024) == 4096        # N/1024 below the part
    assert big_block_rows(1 << 24, 8192, 1024) == 8192        # at most the part
    assert big_block_rows(1 << 20, 2048, 1024) == 1024        # at least the default
    assert big_block_rows(1_449_545, 2048, 1024) == 1280       # 1,415 rounded down to an eighth of the part
    assert big_block_rows(8_003_578, 8192, 1024) == 7168       # 7,815 -> 7 x 1,024
    # At most BIG_BLOCK_STEPS distinct thresholds (companion modules) per part size.
    assert len({big_block_rows(n, 8192, 1024) for n in range(1 << 22, 1 << 24, 99_991)}) <= 8


def test_splits_segments_known_answers():
    """Larger split parts are taken only by calls that provably hold a
    segment longer than the block class: by max_len, or without it by more
    rows than b block-class segments hold (pigeonhole)."""
    from ragged.runtime import splits_segments
    assert not splits_segments(1_040_746, 4096, None, 1024)   # C2 without max_len: 4096 x 1024 rows would hold it
    assert not splits_segments(1_040_746, 4096, 512, 1024)    # C2 with max_len
    assert splits_segments(786_432, 3, None, 1024)             # three 2^18-row segments
    assert splits_segments(3073, 3, None, 1024)                # one row more than three block segments hold
    assert not splits_segments(3072, 3, None, 1024)            # could be three 1024-row segments
    assert splits_segments(4_194_304, 8192, 200_000, 1024)     # C5 lengths with max_len
    assert not splits_segments(4_194_304, 8192, None, 1024)    # ... and without: not provable
    assert not splits_segments(0, 0, None, 1024)
