"""ctypes binding of libragged_hip.so (include/ragged_hip.h).

This replaces the reference's nanobind module ``ragged._native``
(runtime/bindings.cpp:11-37): ``NativeModule`` plays the role of
``DriverModule``. The library is loaded from this package directory only
(in-tree build); when it is absent every entry point raises
``RuntimeUnavailable`` -- there is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import hashlib
from pathlib import Path
import threading

from .errors import RuntimeUnavailable, ValidationError

LIBRARY_PATH = Path(__file__).with_name("libragged_hip.so")
ABI_VERSION = 3

OPS = {"sum": 0, "max": 1, "softmax": 2}
DTYPES = {"f32": 0, "bf16": 1}
INDEX_DTYPES = {"i32": 0, "i64": 1}
SCHEDULES = {"classified": 0, "naive": 1, "short": 2}
ROLES = ("init", "classify", "wave", "block", "split_partial", "split_combine", "split_normalize", "naive",
         "fused", "deferred", "worker")
BUFFERS = ("class_counts", "segment_ids", "item_segments", "part_begin", "partials", "partial_sums",
           "max_stats", "sum_stats", "visits", "deferred", "arrive", "segment_arrive", "items", "block_items",
           "pairs", "final_pairs")
MAX_LAUNCHES = 8
STATIC_WORKSPACE_BYTES = 64 << 20    # RG_STATIC_WORKSPACE_BYTES

RG_OK, RG_E_INVALID, RG_E_DEVICE, RG_E_UNSUPPORTED, RG_E_WORKSPACE = 0, -1, -2, -3, -4


class Spec(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int32), ("dtype", ctypes.c_int32), ("offsets_dtype", ctypes.c_int32),
                ("feature_dim", ctypes.c_int32), ("scale", ctypes.c_float), ("has_mask", ctypes.c_int32),
                ("vectorize", ctypes.c_int32), ("debug_visits", ctypes.c_int32), ("t_wave", ctypes.c_int64),
                ("t_block", ctypes.c_int64), ("part_rows", ctypes.c_int64), ("alone_rows", ctypes.c_int64)]


class DeviceProps(ctypes.Structure):
    _fields_ = [("ordinal", ctypes.c_int32), ("cu_count", ctypes.c_int32), ("xcd_count", ctypes.c_int32),
                ("wave_size", ctypes.c_int32), ("l2_bytes", ctypes.c_int64), ("mall_bytes", ctypes.c_int64),
                ("lds_per_cu", ctypes.c_int64), ("global_mem_bytes", ctypes.c_int64), ("arch", ctypes.c_char * 64)]


class Plan(ctypes.Structure):
    _fields_ = [("schedule", ctypes.c_int32), ("launches", ctypes.c_int32),
                ("roles", ctypes.c_int32 * MAX_LAUNCHES), ("grid", (ctypes.c_uint32 * 3) * MAX_LAUNCHES),
                ("block", ctypes.c_uint32 * MAX_LAUNCHES), ("lds_bytes", ctypes.c_uint32 * MAX_LAUNCHES),
                ("workspace_bytes", ctypes.c_uint64), ("buffer_offset", ctypes.c_uint64 * len(BUFFERS)),
                ("buffer_bytes", ctypes.c_uint64 * len(BUFFERS)), ("n", ctypes.c_int64), ("b", ctypes.c_int64),
                ("b_split", ctypes.c_int64), ("items_cap", ctypes.c_int64), ("t_wave", ctypes.c_int64),
                ("t_block", ctypes.c_int64), ("part_rows", ctypes.c_int64), ("vec", ctypes.c_int32),
                ("flat", ctypes.c_int32), ("fused", ctypes.c_int32)]

    @property
    def steps(self) -> list[tuple[str, tuple[int, int, int], int, int]]:
        """(role, grid, block threads, static LDS bytes) in submission order."""
        return [(ROLES[self.roles[i]], tuple(int(x) for x in self.grid[i]), int(self.block[i]),
                 int(self.lds_bytes[i])) for i in range(self.launches)]

    @property
    def buffers(self) -> list[tuple[str, int, int]]:
        """(name, offset, bytes) of every workspace buffer with nonzero size."""
        return [(name, int(self.buffer_offset[i]), int(self.buffer_bytes[i]))
                for i, name in enumerate(BUFFERS) if self.buffer_bytes[i]]


_lock = threading.Lock()


def _declare(lib: ctypes.CDLL) -> ctypes.CDLL:
    c_int, c_i64, c_u64, vp = ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_void_p
    signatures = {
        "rg_abi_version": (c_int, []),
        "rg_build_info": (ctypes.c_char_p, []),
        "rg_last_error": (ctypes.c_char_p, []),
        "rg_device_query": (c_int, [c_int, ctypes.POINTER(DeviceProps)]),
        "rg_spec_defaults": (c_int, [ctypes.POINTER(Spec)]),
        "rg_spec_uses_fused": (c_int, [ctypes.POINTER(Spec)]),
        "rg_module_create": (c_int, [c_int, ctypes.POINTER(Spec), ctypes.POINTER(vp)]),
        "rg_module_destroy": (None, [vp]),
        "rg_module_resident": (c_int, [vp, c_int, ctypes.POINTER(c_i64)]),
        "rg_plan_create": (c_int, [vp, c_i64, c_i64, c_int, ctypes.POINTER(Plan)]),
        "rg_run": (c_int, [vp, ctypes.POINTER(Plan), vp, vp, vp, vp, vp, c_u64, vp]),
        "rg_run_static": (c_int, [vp, ctypes.POINTER(Plan), vp, vp, vp, vp, vp]),
        "rg_test_interrupt_static": (c_int, [c_int]),
        "rg_check_offsets": (c_int, [c_int, c_int, vp, c_i64, c_i64, c_i64, c_i64, vp, vp]),
        "rg_profile_start": (c_int, [vp, c_int]),
        "rg_module_set_spin_limit": (c_int, [vp, c_i64]),
        "rg_module_set_trace": (c_int, [vp, vp, c_i64]),
        "rg_device_clock_khz": (c_int, [c_int, ctypes.POINTER(c_i64)]),
        "rg_profile_stop": (c_int, [vp, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_i64),
                                    ctypes.POINTER(ctypes.c_double), ctypes.POINTER(c_i64)]),
    }
    for name, (restype, argtypes) in signatures.items():
        function = getattr(lib, name)
        function.restype = restype
        function.argtypes = argtypes
    return lib


_loaded: dict[Path, ctypes.CDLL] = {}   # LIBRARY_PATH -> declared library


def library() -> ctypes.CDLL:
    """The in-tree HIP library, loaded and declared once per path;
    RuntimeUnavailable if it was not built."""
    lib = _loaded.get(LIBRARY_PATH)
    if lib is not None:
        return lib
    if not LIBRARY_PATH.is_file():
        raise RuntimeUnavailable(f"native HIP library is missing: {LIBRARY_PATH}; run "
                                 "`python ragged-mlir_amd/build.py` (no CPU execution fallback exists)")
    with _lock:
        try:
            lib = _declare(ctypes.CDLL(str(LIBRARY_PATH)))
        except OSError as exc:
            raise RuntimeUnavailable(f"cannot load {LIBRARY_PATH}: {exc}") from exc
        if lib.rg_abi_version() != ABI_VERSION:
            raise RuntimeUnavailable(f"{LIBRARY_PATH.name} ABI {lib.rg_abi_version()} != {ABI_VERSION}")
        _loaded[LIBRARY_PATH] = lib
    return lib


def forget_library() -> None:
    """Drop the declared library of LIBRARY_PATH (after a rebuild, so the
    next ``library()`` opens and checks it again)."""
    with _lock:
        _loaded.pop(LIBRARY_PATH, None)


def plan_ref(plan: "Plan"):
    """The by-reference argument ``rg_run`` takes for ``plan`` (keep ``plan``
    alive while it is used)."""
    return ctypes.byref(plan)


def library_sha256() -> str:
    """sha256 of the library file: the identity artifacts bind to."""
    if not LIBRARY_PATH.is_file():
        raise RuntimeUnavailable(f"native HIP library is missing: {LIBRARY_PATH}")
    return hashlib.sha256(LIBRARY_PATH.read_bytes()).hexdigest()


def build_info() -> str:
    return library().rg_build_info().decode()


def _check(status: int, what: str) -> None:
    if status == RG_OK:
        return
    message = library().rg_last_error().decode(errors="replace")
    if status == RG_E_UNSUPPORTED:
        raise RuntimeUnavailable(f"{what}: {message}")
    if status in (RG_E_INVALID, RG_E_WORKSPACE):
        raise ValidationError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")


def device_props(ordinal: int) -> DeviceProps:
    props = DeviceProps()
    _check(library().rg_device_query(ordinal, ctypes.byref(props)), "rg_device_query")
    return props


def make_spec(op: str, dtype: str, offsets_dtype: str, feature_dim: int, *, scale: float = 1.0,
              mask: bool = False, vectorize: bool = True, debug_visits: bool = False,
              t_wave: int = -1, t_block: int = -1, part_rows: int = -1) -> Spec:
    spec = Spec(OPS[op], DTYPES[dtype], INDEX_DTYPES[offsets_dtype], feature_dim, scale, int(mask),
                int(vectorize), int(debug_visits), t_wave, t_block, part_rows, 0)
    _check(library().rg_spec_defaults(ctypes.byref(spec)), "rg_spec_defaults")
    return spec


def uses_fused(spec: Spec) -> bool:
    """Whether the library runs this softmax spec register-resident."""
    status = library().rg_spec_uses_fused(ctypes.byref(spec))
    if status < 0:
        _check(status, "rg_spec_uses_fused")
    return status == 1


def interrupt_static(launches: int) -> None:
    """Test control (``rg_test_interrupt_static``): the next ``run_static``
    stops after ``launches`` launches of its plan and fails as a launch error
    would; -1 turns it off."""
    _check(library().rg_test_interrupt_static(int(launches)), "rg_test_interrupt_static")


def device_clock_khz(device: int = 0) -> int:
    """Rate of the device wall clock (the timeline records' ticks), in kHz."""
    khz = ctypes.c_int64(0)
    _check(library().rg_device_clock_khz(device, ctypes.byref(khz)), "rg_device_clock_khz")
    return int(khz.value)


class NativeModule:
    """One kernel specialisation on one device (the reference's DriverModule)."""

    def __init__(self, device: int, spec: Spec):
        self.device = device
        self.spec = spec
        handle = ctypes.c_void_p()
        self._lib = library()
        _check(self._lib.rg_module_create(device, ctypes.byref(spec), ctypes.byref(handle)), "rg_module_create")
        self._handle = handle

    def resident_blocks(self, role: str) -> int:
        blocks = ctypes.c_int64()
        _check(library().rg_module_resident(self._handle, ROLES.index(role), ctypes.byref(blocks)),
               "rg_module_resident")
        return int(blocks.value)

    def plan(self, n: int, b: int, schedule: str) -> Plan:
        plan = Plan()
        _check(library().rg_plan_create(self._handle, n, b, SCHEDULES[schedule], ctypes.byref(plan)),
               "rg_plan_create")
        return plan

    def run(self, plan: Plan, values: int, offsets: int, out: int, mask: int | None, workspace: int | None,
            workspace_bytes: int, stream: int) -> None:
        self.run_ref(plan_ref(plan), values, offsets, out, mask, workspace, workspace_bytes, stream)

    def run_ref(self, plan, values: int, offsets: int, out: int, mask: int | None, workspace: int | None,
                workspace_bytes: int, stream: int) -> None:
        """``run`` with ``plan`` already a ctypes reference (``plan_ref``)."""
        status = self._lib.rg_run(self._handle, plan, values, offsets, out, mask, workspace, workspace_bytes,
                                  stream)
        if status:
            _check(status, "rg_run")

    def run_static(self, plan: Plan, values: int, offsets: int, out: int, mask: int | None, stream: int) -> None:
        """``rg_run_static``: the plan on the library's static per-device
        workspace (no allocation; plans up to STATIC_WORKSPACE_BYTES; calls
        that overlap on one device race)."""
        status = self._lib.rg_run_static(self._handle, plan_ref(plan), values, offsets, out, mask, stream)
        if status:
            _check(status, "rg_run_static")

    def set_spin_limit(self, microseconds: int) -> None:
        """Bound of every softmax wait for other workgroups' statistics: a
        register-resident chunk's wait for its segment and a worker split
        part's wait for its segment's statistics (test control; -1 restores
        the defaults)."""
        _check(library().rg_module_set_spin_limit(self._handle, microseconds), "rg_module_set_spin_limit")

    def set_trace(self, buffer: int | None, records: int = 0) -> None:
        """Item timeline of the register-resident softmax into ``buffer``
        (device pointer to ``records`` x 8 int64), or off with None."""
        _check(library().rg_module_set_trace(self._handle, buffer, records if buffer else 0), "rg_module_set_trace")

    def profile_start(self, max_calls: int) -> None:
        """Record per-launch HIP events in the next ``max_calls`` runs."""
        _check(library().rg_profile_start(self._handle, max_calls), "rg_profile_start")

    def profile_stop(self) -> dict:
        """Per-role kernel ms and launch counts, and whole-call ms, of the
        recorded runs (waits for their events)."""
        count = len(ROLES)
        role_ms = (ctypes.c_double * count)()
        role_launches = (ctypes.c_int64 * count)()
        call_ms, calls = ctypes.c_double(), ctypes.c_int64()
        _check(library().rg_profile_stop(self._handle, role_ms, role_launches, ctypes.byref(call_ms),
                                         ctypes.byref(calls)), "rg_profile_stop")
        return {"calls": int(calls.value), "call_ms": float(call_ms.value),
                "roles": {ROLES[i]: {"ms": float(role_ms[i]), "launches": int(role_launches[i])}
                          for i in range(count) if role_launches[i]}}

    def close(self) -> None:
        handle, self._handle = getattr(self, "_handle", None), None
        if handle and handle.value:
            library().rg_module_destroy(handle)

    def __del__(self):
        try:
            self.close()
        except Exception:  # noqa: BLE001 - finalizers must not raise
            pass


def check_offsets(device: int, offsets_dtype: str, offsets: int, n: int, b: int, min_len: int | None,
                  max_len: int | None, status: int, stream: int) -> None:
    _check(library().rg_check_offsets(device, INDEX_DTYPES[offsets_dtype], offsets, n, b,
                                      -1 if min_len is None else min_len, -1 if max_len is None else max_len,
                                      status, stream), "rg_check_offsets")
