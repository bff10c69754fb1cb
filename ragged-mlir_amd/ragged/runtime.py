"""``CompiledProgram``: validate tensors and enqueue on the current HIP stream.

Restates the public behaviour of the reference's ``python/ragged/runtime.py``
(:218-558): ``run(values, offsets, out, stream=None, mode="validated", *,
debug_buffers=None, mask=None, concurrent=True, select="auto", max_len=None)``
validates every tensor before any allocation or launch, chooses a schedule
per call with the cost model (``choose``), allocates one scratch buffer on
the consumer stream, records the caller's tensors on that stream and makes a
single native call that enqueues every kernel. Validated mode never
synchronises; checked mode validates the offsets on the device first
(docs/checked-abi.md). There is no CPU execution path: CPU tensors, a
missing library or a non-gfx950 device raise ``RuntimeUnavailable``.
"""
from __future__ import annotations

import contextlib
import importlib
import json
import threading
import time
from typing import Any

from . import native
from .cache import Artifact
from .errors import CacheMismatch, RuntimeUnavailable, ValidationError
from .model import ExecutionReport, ProgramSpec, canonical_json, runs_on
from .selection import default_model
from .validation import raise_for_status, validate_program

_lock = threading.RLock()
_modules: dict[tuple[int, str], native.NativeModule] = {}   # (device, artifact digest) -> module
_device_arch: dict[int, str] = {}
_device_runs: dict[tuple[int, str], bool] = {}     # (device, chip) -> the chip's code runs there
_device_l2_mib: dict[int, float | None] = {}
# torch.cuda.Stream objects of current streams, keyed by torch's exact
# (stream id, device index, device type) of each: equal keys are one stream.
_current_streams: dict[tuple, Any] = {}
I64_MAX = 2**63 - 1

# The register-resident softmax holds a segment's chunks only while the
# device can hold them all: segments of more chunks than 7/8 of its resident
# workgroups (the library's rule, rg_plan_create's wait_parts) defer every
# chunk to the kernel's drain, a pass per round of the resident workgroups
# that re-reads them about 3-4x slower per chunk than the streaming worker's
# split schedule streams them. A call whose deferred rows are provably at
# least half of N and at least 1.5 such limits runs the streaming schedule
# instead (a program of the same spec whose split parts exceed the register
# capacity). Measured with one long segment: at 1.1 limits the two schedules
# are within 10% either way, from 2 limits streaming is 1.4-2.4x faster.
STREAM_SHARE = 0.5
STREAM_MIN_LIMITS = 1.5
# The streaming schedule's split parts when it takes over: about 2 MiB of rows,
# at most 16,384 rows (measured, µs per call on four long-segment inputs:
# f32 D=16 best at 16,384 rows = 1 MiB, f32 D=128 at 4,096 = 2 MiB, bf16 D=128
# at 8,192 = 2 MiB, bf16 D=1024 at 1,024 = 2 MiB; a fixed 4,096 rows was up to
# 1.9x slower).
STREAM_PART_BYTES = 2 << 20
STREAM_MAX_PART_ROWS = 16384


def stream_part_rows(row_bytes: int, register_part_rows: int) -> int:
    """Rows of a streaming split part for rows of ``row_bytes``: the power of
    two nearest below STREAM_PART_BYTES of rows, at most STREAM_MAX_PART_ROWS,
    and above the register path's part (so that the library runs the
    streaming worker)."""
    rows = 1
    while rows * 2 * row_bytes <= STREAM_PART_BYTES and rows * 2 <= STREAM_MAX_PART_ROWS:
        rows *= 2
    return max(rows, 2 * register_part_rows)


def deferred_rows_bound(n: int, b: int, max_len: int | None, limit: int) -> int:
    """Rows of an (n, b) call that the register-resident softmax surely
    defers: segments longer than ``limit`` rows defer, so at least the rows
    that the segments of at most ``limit`` rows cannot hold -- N - B*limit,
    or, when the caller's longest segment exceeds the limit (it is then one
    of the deferred), the larger of it and N - (B-1)*limit."""
    if max_len is None or n <= 0 or limit <= 0:
        return 0
    if max_len > limit:
        return max(max_len, n - (b - 1) * limit)
    return max(n - b * limit, 0)


# Sum / max calls split long segments into parts of about N/512 rows (at
# most 4 MiB) instead of the library's 256 KiB once N/512 rows reach twice the
# default part (from about 256 MiB of rows): every part is a queue item that
# publishes its partial with a release (an L2 write-back) and counts in at its
# segment, and thousands of small ones cost more than the parallelism they
# add. Measured (µs per call, default -> these parts and block class): f32
# D=128 one 2^22-row segment 2,438 -> 466, 64 segments of 2^16 rows 783 ->
# 420, three 2^18-row segments (384 MiB) 219 -> 133; bf16 D=128 four 2^20-row
# segments 546 -> 233; on the calibration suites' 32 training cases it
# changes, 11% less time warm. Only calls that provably hold a segment longer
# than the block class take them (``splits_segments``), and segments of up to
# about N/1024 rows join the block class (``big_block_rows``). The cost model was
# fitted on measurements taken with these rules.
BIG_PART_SHARE = 512
BIG_PART_BYTES = 4 << 20
BIG_BLOCK_SHARE = 1024
BIG_BLOCK_STEPS = 8


def big_part_rows(n: int, row_bytes: int, default_rows: int) -> int:
    """Split part (rows) of a sum / max call of ``n`` rows of ``row_bytes``:
    the power of two nearest below n / BIG_PART_SHARE, at most BIG_PART_BYTES
    of rows, at least the library's default (which it stays while
    n / BIG_PART_SHARE is below twice the default)."""
    rows = default_rows
    while rows * 2 <= n // BIG_PART_SHARE and rows * 2 * row_bytes <= BIG_PART_BYTES:
        rows *= 2
    return rows


def big_block_rows(n: int, part_rows: int, default_t_block: int) -> int:
    """Longest block-class segment of a call of ``n`` rows that splits into
    ``part_rows`` parts: a segment one part would hold goes to one workgroup
    whole, with no partial to publish (as one split part it costs 1.2-1.3x
    the time), up to n / BIG_BLOCK_SHARE rows (about 1.5 resident
    workgroups' share of the call: block items are taken after the split
    parts, and larger ones finish last), rounded down to a multiple of
    part_rows / BIG_BLOCK_STEPS, so that a program keeps at most that many
    companion modules per part size."""
    step = max(1, part_rows // BIG_BLOCK_STEPS)
    return max(default_t_block, min(part_rows, n // BIG_BLOCK_SHARE // step * step))


def splits_segments(n: int, b: int, max_len: int | None, t_block: int) -> bool:
    """Whether a call of (n, b, max_len) provably holds a segment longer than
    the block class (``t_block`` rows): by max_len, or else by more rows than
    b block-class segments hold."""
    return max_len > t_block if max_len is not None else n > b * t_block


def streams_long_segments(n: int, b: int, max_len: int | None, limit: int) -> bool:
    """Whether a register-resident softmax call of (n, b, max_len) runs the
    streaming schedule instead, given the longest segment ``limit`` (rows)
    the register path holds."""
    deferred = deferred_rows_bound(n, b, max_len, limit)
    return deferred > 0 and deferred >= STREAM_SHARE * n and deferred >= STREAM_MIN_LIMITS * limit


_torch_module = None


def _torch():
    """torch, imported on first use (``import ragged`` never imports it)."""
    global _torch_module
    if _torch_module is None:
        try:
            _torch_module = importlib.import_module("torch")
        except ImportError as exc:
            raise RuntimeUnavailable("PyTorch is not installed; install PyTorch-ROCm to execute") from exc
    return _torch_module


def device_l2_mib(values) -> float | None:
    """Total L2 (all XCDs) of the device holding ``values`` in MiB."""
    device = getattr(values, "device", None)
    if getattr(device, "type", None) != "cuda":
        return None
    index = device.index if device.index is not None else 0
    if index not in _device_l2_mib:
        try:
            props = native.device_props(index)
            _device_l2_mib[index] = props.l2_bytes * max(props.xcd_count, 1) / 2**20 if props.l2_bytes else None
        except Exception:  # noqa: BLE001 - the cost model then uses its calibration value
            _device_l2_mib[index] = None
    return _device_l2_mib[index]


def _span(tensor) -> tuple[int, int]:
    """[first byte, one past the last byte) of a contiguous tensor."""
    start = tensor.data_ptr()
    return start, start + tensor.nbytes


def _spans_overlap(left: tuple[int, int], right: tuple[int, int]) -> bool:
    return left[0] < right[1] and right[0] < left[1]


def _current_stream(torch, device: int):
    """torch.cuda.current_stream(device), without building a new Stream
    object per call."""
    key = torch._C._cuda_getCurrentStream(device)
    stream = _current_streams.get(key)
    if stream is None:
        if len(_current_streams) > 64:
            _current_streams.clear()
        stream = _current_streams[key] = torch.cuda.Stream(stream_id=key[0], device_index=key[1], device_type=key[2])
    return stream


class CompiledProgram:
    """A validated artifact plus, for adaptive programs, its block-per-segment
    companion ``naive`` (reference runtime.py:218-268)."""

    def __init__(self, spec: ProgramSpec, artifact: Artifact, *, cache_hit: bool = False,
                 naive: "CompiledProgram | None" = None):
        validate_program(spec, artifact)
        self.spec, self.artifact, self.cache_hit = spec, artifact, cache_hit
        self._metadata = json.loads(canonical_json(artifact.metadata))
        self._digest = artifact.key.digest
        self._selects = spec.strategy == "auto" and not spec.debug_visits and self._metadata["dispatch_abi"] is not None
        self._schedule = "classified" if self._metadata["dispatch_abi"] is not None else "naive"
        if naive is not None and (not self._selects or naive.spec != _naive_spec(spec)):
            raise CacheMismatch("a block-per-segment companion must be the naive strategy of a classifying program")
        self.naive = naive
        self._choices: dict[tuple, tuple[str, dict[str, Any]]] = {}
        self._plans: dict[tuple[native.NativeModule, int, int, str], native.Plan] = {}
        # Per plan: its kernel names and grids for reports, and the ctypes
        # reference rg_run takes (built once, not per call).
        self._launches: dict[tuple[native.NativeModule, int, int, str], tuple[list, list, Any]] = {}
        # Workspace per (device, stream): calls on one stream run in order,
        # so they can share it; it grows to the largest plan seen.
        self._workspaces: dict[tuple[int, int], Any] = {}
        self._names = {kernel["role"]: kernel["name"] for kernel in self._metadata["kernels"]}
        self._alone: int | None = None
        self._wait_limit: dict[int, int] = {}   # device -> longest segment (rows) the register path holds
        self._torch_dtypes: tuple | None = None    # (values dtype, offsets dtype) as torch dtypes
        self._report_static: tuple | None = None   # (classes, thresholds) of every report

    @property
    def selects(self) -> bool:
        """Whether this program classifies on the device, so that one block per
        segment is an alternative worth choosing per call."""
        return self._selects

    @property
    def metadata(self) -> dict[str, Any]:
        return self._metadata

    def choose(self, n: int, b: int, max_len: int | None, l2_mib: float | None = None) -> tuple[str, dict[str, Any]]:
        """The schedule ``run(select="auto")`` uses for this input, and why."""
        if self.naive is None:
            return self._schedule, {}
        key = (n, b, max_len, l2_mib)
        choice = self._choices.get(key)
        if choice is None:
            if len(self._choices) >= 256:
                self._choices.clear()
            element = 2 if self.spec.dtype == "bf16" else 4
            choice = self._choices[key] = default_model().choose(self.spec.op, n, b, self.spec.feature_dim, max_len,
                                                                 element, l2_mib=l2_mib,
                                                                 fused=bool(self._metadata["fused"]),
                                                                 flat=self._metadata["mapping"] == "flat")
        return choice

    def close(self) -> None:
        """Drop this program's plans and workspaces; the shared native module
        stays loaded."""
        self._plans.clear()
        self._launches.clear()
        self._workspaces.clear()

    def _workspace(self, torch, device, stream, nbytes: int, fresh: bool):
        """Zeroed scratch of at least ``nbytes`` for a call on ``stream``.
        Calls on one stream run in order and each leaves the workspace's
        counters at zero, so they share one allocation (made on that
        stream); ``fresh`` (debug buffers handed to the caller, or a debug
        specialisation, which keeps its counters) allocates a new one."""
        if fresh:
            with torch.cuda.stream(stream):
                return torch.zeros((nbytes,), dtype=torch.uint8, device=device)
        key = (device.index if device.index is not None else 0, stream.cuda_stream)
        workspace = self._workspaces.get(key)
        if workspace is None or workspace.numel() < nbytes:
            if len(self._workspaces) >= 16:
                self._workspaces.clear()
            with torch.cuda.stream(stream):
                workspace = self._workspaces[key] = torch.zeros((nbytes,), dtype=torch.uint8, device=device)
        return workspace

    # ------------------------------------------------------------------
    def _validate_tensors(self, values, offsets, out, torch, *, checked: bool = False, mask=None) -> tuple[int, int]:
        if self.spec.mask != (mask is not None):
            raise ValidationError("mask presence must match the compiled specialization")
        tensors = [("values", values), ("offsets", offsets), ("out", out)]
        if mask is not None:
            tensors.append(("mask", mask))
        for name, tensor in tensors:
            if not isinstance(tensor, torch.Tensor):
                raise ValidationError(f"{name} must be a torch.Tensor")
            if not tensor.is_cuda:
                raise RuntimeUnavailable(f"{name} must be on a ROCm device that runs {self.spec.chip} code; "
                                         "no CPU execution fallback exists")
            if not tensor.is_contiguous():
                raise ValidationError(f"{name} must be row-major contiguous")
            if tensor.requires_grad:
                raise ValidationError("autograd is outside the supported forward-only contract")
        device = values.get_device()
        if offsets.get_device() != device or out.get_device() != device:
            raise ValidationError("values, offsets and out must use the same device")
        if values.ndim != 2 or values.shape[1] != self.spec.feature_dim:
            raise ValidationError("values must have shape [N, static D]")
        if offsets.ndim != 1 or offsets.numel() < 1:
            raise ValidationError("offsets must have shape [B+1], including [0] when B=0")
        dtypes = self._torch_dtypes
        if dtypes is None:
            dtypes = self._torch_dtypes = ({"f32": torch.float32, "bf16": torch.bfloat16}[self.spec.dtype],
                                           {"i32": torch.int32, "i64": torch.int64}[self.spec.offsets_dtype])
        dtype, offset_dtype = dtypes
        if values.dtype != dtype or out.dtype != dtype or offsets.dtype != offset_dtype:
            raise ValidationError("tensor dtype differs from compiled dtype/offsets specialization")
        vector = self._metadata["d_vector"]
        if vector > 1:
            # Flat-mapped reductions store their [B, D] results element-wise.
            scalar_out = self.spec.op != "softmax" and self._metadata["mapping"] == "flat"
            for name, tensor in (("values", values), ("out", None if scalar_out else out), ("mask", mask)):
                if tensor is not None and tensor.numel():
                    need = min(16, vector * tensor.element_size())
                    if tensor.data_ptr() % need:
                        raise ValidationError(f"{name} must be {need}-byte aligned: this specialization accesses "
                                              f"{vector} elements at a time (compile with vectorize=False for "
                                              "unaligned views)")
        n, b = values.shape[0], offsets.numel() - 1
        if b == 0 and n != 0 and not checked:
            raise ValidationError("B=0 requires N=0; values cannot exist without segments")
        if self.spec.offsets_dtype == "i32" and n > 2**31 - 1:
            raise ValidationError("N exceeds the i32 offsets range")
        expected = (n if self.spec.op == "softmax" else b, self.spec.feature_dim)
        if tuple(out.shape) != expected:
            raise ValidationError(f"out shape must be {expected}")
        values_span, offsets_span, out_span = _span(values), _span(offsets), _span(out)
        if mask is not None:
            if mask.dtype != torch.float32 or tuple(mask.shape) != tuple(values.shape):
                raise ValidationError("mask must have f32 dtype and exactly values shape [N,D]; "
                                      "broadcasting is unsupported")
            if mask.get_device() != device:
                raise ValidationError("mask must use the values device")
            mask_span = _span(mask)
            if _spans_overlap(mask_span, out_span) or _spans_overlap(mask_span, offsets_span):
                raise ValidationError("mask must not overlap out or offsets")
        if _spans_overlap(offsets_span, values_span) or _spans_overlap(offsets_span, out_span):
            raise ValidationError("offsets must not alias values or out")
        overlap = values.numel() and out.numel() and _spans_overlap(values_span, out_span)
        exact = values_span[0] == out_span[0] and values.shape == out.shape
        if overlap:
            if not exact or self.spec.alias != "inplace" or not self._metadata["alias_safe"]:
                raise ValidationError("out aliases values without a safe in-place schedule")
        elif self.spec.alias == "inplace" and not (exact or values.numel() == 0):
            raise ValidationError("in-place specialization requires out and values to be the same buffer")
        return n, b

    def _module(self, device: int) -> native.NativeModule:
        key = (device, self._digest)
        module = _modules.get(key)
        if module is not None:
            return module
        with _lock:
            module = _modules.get(key)
            if module is None:
                if self.artifact.key.library_sha256 != native.library_sha256():
                    raise CacheMismatch("artifact was built for a different libragged_hip.so; recompile")
                module = _modules[key] = native.NativeModule(device, self._native_spec())
            return module

    def _native_spec(self) -> native.Spec:
        """The library's specialisation of this program (thresholds from the
        manifest, defaults filled by the library)."""
        metadata = self._metadata
        thresholds = metadata["thresholds"] or [-1, -1]
        return native.make_spec(self.spec.op, self.spec.dtype, self.spec.offsets_dtype, self.spec.feature_dim,
                                scale=self.spec.scale, mask=self.spec.mask,
                                vectorize=self.spec.optimizations.vectorize, debug_visits=self.spec.debug_visits,
                                t_wave=thresholds[0], t_block=thresholds[1], part_rows=metadata["part_rows"] or -1)

    def _alone_rows(self) -> int:
        """Longest segment one lane or lane group reduces alone (0: none)."""
        if self._alone is None:
            self._alone = int(self._native_spec().alone_rows)
        return self._alone

    def _streams(self, values, n: int, b: int, max_len: int | None) -> bool:
        """Whether run(select="auto") takes the streaming schedule for this
        register-resident softmax call (see STREAM_SHARE)."""
        if not self._metadata["fused"] or max_len is None or n <= 0 or self.spec.debug_visits:
            return False
        try:
            device = values.get_device()
        except (AttributeError, RuntimeError):
            return False
        if not isinstance(device, int) or device < 0:
            return False         # not a device tensor: validation reports it
        limit = self._wait_limit.get(device)
        if limit is None:
            resident = self._module(device).resident_blocks("fused")
            limit = self._wait_limit[device] = max(1, resident * 7 // 8) * int(self._metadata["part_rows"])
        return streams_long_segments(n, b, max_len, limit)

    def _stream_module(self, device: int) -> native.NativeModule:
        """The streaming schedule of this softmax: the same spec with split
        parts of about 2 MiB (``stream_part_rows``; doubled while the library
        would still hold them in registers)."""
        key = (device, self._digest + ":stream")
        module = _modules.get(key)
        if module is not None:
            return module
        with _lock:
            module = _modules.get(key)
            if module is None:
                self._module(device)     # the library check of the artifact
                row_bytes = self.spec.feature_dim * (2 if self.spec.dtype == "bf16" else 4)
                part_rows = stream_part_rows(row_bytes, int(self._metadata["part_rows"]))
                metadata = self._metadata
                thresholds = metadata["thresholds"] or [-1, -1]
                while True:
                    spec = native.make_spec(self.spec.op, self.spec.dtype, self.spec.offsets_dtype,
                                            self.spec.feature_dim, scale=self.spec.scale, mask=self.spec.mask,
                                            vectorize=self.spec.optimizations.vectorize, t_wave=thresholds[0],
                                            t_block=thresholds[1], part_rows=part_rows)
                    if not native.uses_fused(spec):
                        break
                    part_rows *= 2
                module = _modules[key] = native.NativeModule(device, spec)
            return module

    def _parts_module(self, device: int, part_rows: int, t_block: int) -> native.NativeModule:
        """This sum / max program with split parts of ``part_rows`` rows and
        block-class segments up to ``t_block`` rows (``big_part_rows``,
        ``big_block_rows``)."""
        key = (device, f"{self._digest}:parts{part_rows}:block{t_block}")
        module = _modules.get(key)
        if module is not None:
            return module
        with _lock:
            module = _modules.get(key)
            if module is None:
                spec = self._native_spec()
                module = _modules[key] = native.NativeModule(device, native.make_spec(
                    self.spec.op, self.spec.dtype, self.spec.offsets_dtype, self.spec.feature_dim,
                    vectorize=self.spec.optimizations.vectorize, t_wave=int(spec.t_wave), t_block=t_block,
                    part_rows=part_rows))
            return module

    def _plan(self, module: native.NativeModule, n: int, b: int, schedule: str) -> native.Plan:
        return self._plan_launches(module, n, b, schedule)[0]

    def _plan_launches(self, module: native.NativeModule, n: int, b: int, schedule: str):
        """(plan, kernel names, grids, ctypes reference) for (N, B, schedule)
        on ``module``: keyed by the module, whose thresholds and part size the
        plan carries."""
        key = (module, n, b, schedule)
        plan = self._plans.get(key)
        if plan is None:
            if len(self._plans) >= 256:
                self._plans.clear()
                self._launches.clear()
            native_schedule = "classified" if schedule == "stream" or schedule.startswith("parts") else schedule
            plan = self._plans[key] = module.plan(n, b, native_schedule)
        launches = self._launches.get(key)
        if launches is None:
            steps = plan.steps
            launches = self._launches[key] = ([self._kernel_name(role) for role, _, _, _ in steps],
                                              [grid for _, grid, _, _ in steps], native.plan_ref(plan))
        return (plan,) + launches

    # ------------------------------------------------------------------
    def run(self, values, offsets, out, stream=None, mode: str = "validated", *,
            debug_buffers: dict[str, Any] | None = None, mask=None, concurrent: bool = True,
            select: str = "auto", max_len: int | None = None) -> ExecutionReport:
        """Enqueue on ``stream`` (default: the current stream of values' device).

        ``select="auto"`` asks the cost model, given the longest segment
        ``max_len`` when the caller knows it (a wrong value costs time, never
        correctness); ``"classified"`` / ``"naive"`` force a schedule.
        ``concurrent`` is accepted for compatibility: every class worker is
        enqueued on the one stream, in a fixed order.
        """
        if select not in ("auto", "classified", "naive"):
            raise ValidationError("select must be auto, classified or naive")
        if max_len is not None and (type(max_len) is not int or max_len < 0):
            raise ValidationError("max_len must be None or a nonnegative int")
        if select == "naive" and self.naive is None:
            raise ValidationError("select=naive requires a program compiled with a block-per-segment companion")
        if self.naive is not None and select != "classified":
            if select == "naive":
                chosen, selection = "naive", {"forced": True}
            elif self._short_segments(max_len):
                # One worker launch reduces every segment alone: cheaper than
                # both modelled schedules, so the model is not consulted.
                chosen, selection = "classified", {"max_len": max_len, "reason": "every segment reduced alone"}
            else:
                try:
                    n, b = int(values.shape[0]), int(offsets.numel()) - 1
                except (AttributeError, IndexError, TypeError):
                    n = b = None
                if n is not None and self._streams(values, n, b, max_len):
                    # Segments too long for the register-resident softmax
                    # hold at least half the rows: the streaming schedule.
                    selection = {"max_len": max_len, "streaming": True,
                                 "reason": "segments too long to hold in registers carry at least half the rows "
                                           "and 1.5 register limits"}
                    return self._run(values, offsets, out, stream, mode, debug_buffers=debug_buffers, mask=mask,
                                     selected="classified", selection=selection, max_len=max_len, streaming=True)
                chosen, selection = (self.choose(n, b, max_len, device_l2_mib(values)) if n is not None
                                     else ("classified", {}))
            if chosen == "naive":
                return self.naive._run(values, offsets, out, stream, mode, debug_buffers=debug_buffers, mask=mask,
                                       selected="naive", selection=selection)
        else:
            selection = {"forced": True} if self.naive is not None else {}
        return self._run(values, offsets, out, stream, mode, debug_buffers=debug_buffers, mask=mask,
                         selected=self._schedule, selection=selection, max_len=max_len)

    def _report(self, started, plan_names=(), grids=(), workspace=0, *, mode, selected, selection,
                validation_bytes=0, validation_ms=None) -> ExecutionReport:
        metadata = self._metadata
        static = self._report_static
        if static is None:
            static = self._report_static = (tuple(metadata["classes"]), tuple(metadata["thresholds"]))
        thresholds = static[1]
        if selection and "t_block" in selection:
            # A companion module's block threshold (big_block_rows).
            thresholds = (thresholds[0], selection["t_block"]) + thresholds[2:]
        return ExecutionReport(
            static[0] if plan_names else (), thresholds, tuple(grids),
            workspace + validation_bytes, self._digest, None, mode, tuple(plan_names),
            (time.perf_counter() - started) * 1000, cache_hit=self.cache_hit,
            validation_workspace_bytes=validation_bytes, validation_host_ms=validation_ms,
            optimizations=metadata["optimizations"], d_tile=metadata["d_tile"], d_vector=metadata["d_vector"],
            resources=None, streams=1, selected=selected, selection=selection)

    def _short_segments(self, max_len: int | None) -> bool:
        """Whether the caller's max_len lets one lane (or lane group) reduce
        every segment alone: then one worker launch takes the segments in
        order (no classify, no workspace). A max_len that is too small only
        costs time."""
        thresholds = self._metadata["thresholds"]
        return (self._schedule == "classified" and max_len is not None
                and not self.spec.debug_visits and bool(thresholds) and 0 < thresholds[0]
                and 0 < self._alone_rows() and max_len <= self._alone_rows())

    def _run(self, values, offsets, out, stream, mode, *, debug_buffers, mask, selected, selection,
             max_len: int | None = None, streaming: bool = False) -> ExecutionReport:
        if mode not in ("validated", "checked"):
            raise ValidationError("mode must be validated or checked")
        if self.spec.mask != (mask is not None):
            raise ValidationError("mask presence must match the compiled specialization")
        if debug_buffers is not None and (type(debug_buffers) is not dict or debug_buffers
                                          or not self.spec.debug_visits):
            raise ValidationError("debug_buffers requires an empty dict and a debug_visits specialization")
        torch = _torch()
        checked = mode == "checked"
        n, b = self._validate_tensors(values, offsets, out, torch, checked=checked, mask=mask)
        started = time.perf_counter()
        if b == 0 and not checked:
            return self._report(started, mode=mode, selected=selected, selection=selection)
        # The tensors' device (validated: all on one ROCm device), and a
        # switch only when it is not the current one.
        device = values.get_device()
        switch = device != torch._C._cuda_getDevice()
        with torch.cuda.device(device) if switch else contextlib.nullcontext():
            runs = _device_runs.get((device, self.spec.chip))
            if runs is None:
                if device not in _device_arch:
                    _device_arch[device] = torch.cuda.get_device_properties(device).gcnArchName
                runs = _device_runs[(device, self.spec.chip)] = runs_on(self.spec.chip, _device_arch[device])
            if not runs:
                raise RuntimeUnavailable(f"compiled target {self.spec.chip} does not run on the current device "
                                         f"({_device_arch[device]})")
            if stream is None:
                active = _current_stream(torch, device)
            else:
                active = stream
                if not isinstance(active, torch.cuda.Stream) or active.device != values.device:
                    raise ValidationError("stream must be a torch.cuda.Stream on the values device")
            module = self._module(device)
            names, grids, validation_bytes, validation_ms = [], [], 0, None
            if checked:
                validation_started = time.perf_counter()
                with torch.cuda.stream(active):
                    status = torch.empty((7,), dtype=torch.int64, device=values.device)
                    host_status = torch.empty((7,), dtype=torch.int64, device="cpu", pin_memory=True)
                    for tensor in (offsets, status):
                        tensor.record_stream(active)
                    native.check_offsets(device, self.spec.offsets_dtype, offsets.data_ptr(), n, b,
                                         self.spec.hints.min_len, self.spec.hints.max_len, status.data_ptr(),
                                         active.cuda_stream)
                    host_status.copy_(status, non_blocking=True)
                active.synchronize()
                raise_for_status(host_status.tolist(), b=b)
                validation_ms = (time.perf_counter() - validation_started) * 1000
                validation_bytes = 56
                names += ["ragged_0_offsets_init", "ragged_0_offsets_check"]
                grids += [(1, 1, 1), (-(-(b + 1) // 256), 1, 1)]
                if b == 0:
                    return self._report(started, names, grids, 0, mode=mode, selected=selected, selection=selection,
                                        validation_bytes=validation_bytes, validation_ms=validation_ms)
            short = not streaming and self._short_segments(max_len)
            if short:
                selection = {**selection, "short_segments": True}
            schedule = "stream" if streaming else "short" if short else self._schedule
            if streaming:
                module = self._stream_module(device)
            elif schedule == "classified" and self.spec.op != "softmax" and not self.spec.debug_visits:
                default_rows = int(self._metadata["part_rows"])
                part_rows = big_part_rows(n, self.spec.feature_dim * (2 if self.spec.dtype == "bf16" else 4),
                                          default_rows)
                # Part size matters only where a segment is longer than the
                # block class.
                default_block = int(self._metadata["thresholds"][1])
                if part_rows != default_rows and splits_segments(n, b, max_len, default_block):
                    t_block = big_block_rows(n, part_rows, default_block)
                    module = self._parts_module(device, part_rows, t_block)
                    schedule = f"parts{part_rows}"
                    selection = {**selection, "part_rows": part_rows, "t_block": t_block}
            plan, plan_names, plan_grids, plan_ref = self._plan_launches(module, n, b, schedule)
            workspace = None
            if plan.workspace_bytes:
                workspace = self._workspace(torch, values.device, active, int(plan.workspace_bytes),
                                            fresh=debug_buffers is not None or self.spec.debug_visits)
            inputs = [values, offsets, out] + ([mask] if mask is not None else [])
            for tensor in inputs:
                tensor.record_stream(active)
            try:
                module.run_ref(plan_ref, values.data_ptr(), offsets.data_ptr(), out.data_ptr(),
                               mask.data_ptr() if mask is not None else None,
                               workspace.data_ptr() if workspace is not None else None, int(plan.workspace_bytes),
                               active.cuda_stream)
            except Exception:
                # A launch that failed part way may leave the counters set:
                # the next call on this stream gets a fresh zeroed workspace.
                self._workspaces.pop((device, active.cuda_stream), None)
                raise
            names += plan_names
            grids += plan_grids
            if debug_buffers is not None and workspace is not None:
                dtypes = {"class_counts": torch.int64, "segment_ids": torch.int64, "item_segments": torch.int64,
                          "part_begin": torch.int64, "partials": torch.float32, "partial_sums": torch.float32,
                          "max_stats": torch.float32, "sum_stats": torch.float32, "visits": torch.int32,
                          "deferred": torch.int64, "arrive": torch.int32, "segment_arrive": torch.int32,
                          "items": torch.int64, "block_items": torch.int64, "pairs": torch.int64,
                          "final_pairs": torch.int64}
                for name, offset, nbytes in plan.buffers:
                    view = workspace[offset:offset + nbytes].view(dtypes[name])
                    if name == "segment_ids":
                        view = view.view(3, b)
                    debug_buffers[name] = view
                # Present the wave class as one count and one run of ids: the
                # library counts the segments reduced alone in slot 0 (slot
                # 7 for a register-resident softmax) and queues them from the
                # front, the others in slot 8 and from the back. The copies
                # are ordered after the launch on its stream; reading the
                # counts makes a debug call synchronise.
                if "class_counts" in debug_buffers:
                    with torch.cuda.stream(active):
                        counts = debug_buffers["class_counts"]
                        alone = counts[7 if plan.fused else 0]
                        coop = counts[8]
                        debug_buffers["class_counts"] = presented = counts[:8].clone()
                        presented[0] = alone + coop
                        if "segment_ids" in debug_buffers:
                            ids = debug_buffers["segment_ids"].clone()
                            n_alone, n_coop = int(alone), int(coop)
                            if n_coop:
                                ids[0, n_alone:n_alone + n_coop] = debug_buffers["segment_ids"][0, b - n_coop:]
                            debug_buffers["segment_ids"] = ids
        return self._report(started, names, grids, int(plan.workspace_bytes), mode=mode, selected=selected,
                            selection=selection, validation_bytes=validation_bytes, validation_ms=validation_ms)

    def _kernel_name(self, role: str) -> str:
        phase = "online" if self.spec.op == "softmax" else self.spec.op
        manifest_role = {"worker": f"worker_{phase}", "naive": phase, "fused": "fused_online",
                         "deferred": "deferred_online"}.get(role, role)
        return self._names.get(manifest_role, f"ragged_0_{manifest_role}")


def _naive_spec(spec: ProgramSpec) -> ProgramSpec:
    from dataclasses import replace
    return replace(spec, strategy="naive")
