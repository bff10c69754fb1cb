"""Immutable program specification and per-call execution evidence.

Restates the reference's ``python/ragged/model.py`` surface: ``Hints``
(:58-70), ``ProgramSpec`` (:73-197) with the same fields, defaults (except
``chip``: gfx950) and validation messages, and ``ExecutionReport``
(:200-237). The cache key is the sha256 of a canonical source text of the
spec (``source_text``), the role MLIR text played in the reference.
"""
from __future__ import annotations

from dataclasses import asdict, dataclass, field
import hashlib
import json
import math
from typing import Any

from .errors import ValidationError
from .optimizations import BOOL_OPTIONS, Optimizations

DIALECT_VERSION = "1"
SOURCE_FORMAT = "ragged-hip-spec-v1"


@dataclass(frozen=True)
class ChipLimits:
    """Per-workgroup limits of a target: LDS bytes, VGPRs per lane and threads.
    gfx950 (CDNA4): 160 KiB LDS per CU (64 KiB per workgroup addressable by
    default), 512 VGPRs per lane, 1024 threads per workgroup."""
    shared_per_cta: int
    registers_per_thread: int
    threads_per_cta: int


DEFAULT_CHIP = "gfx950"
CHIPS = {"gfx950": ChipLimits(65536, 512, 1024)}


def runs_on(chip: str, arch: str) -> bool:
    """Whether code for ``chip`` runs on a device whose gcnArchName is
    ``arch`` (for example "gfx950:sramecc+:xnack-")."""
    if chip not in CHIPS:
        raise ValidationError("chip must be gfx950")
    return arch.split(":")[0] == chip


def canonical_json(value: Any) -> str:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False)


def _nonnegative_int(name: str, value: int | None) -> None:
    if value is not None and (type(value) is not int or value < 0 or value > 2**63 - 1):
        raise ValidationError(f"{name} must be an integer in [0, 2^63-1]")


@dataclass(frozen=True)
class Hints:
    """Caller promises about every segment length (reference model.py:58-70)."""
    max_len: int | None = None
    min_len: int | None = None
    offsets_checked: bool = False

    def __post_init__(self) -> None:
        _nonnegative_int("max_len", self.max_len)
        _nonnegative_int("min_len", self.min_len)
        if type(self.offsets_checked) is not bool:
            raise ValidationError("offsets_checked must be bool")
        if self.max_len is not None and self.min_len is not None and self.min_len > self.max_len:
            raise ValidationError("min_len must not exceed max_len")


@dataclass(frozen=True)
class ProgramSpec:
    """What to compute: op over ``values[N, feature_dim]`` of ``dtype`` with
    ``offsets_dtype`` offsets (reference model.py:73-188)."""
    op: str
    dtype: str = "f32"
    feature_dim: int = 128
    offsets_dtype: str = "i64"
    hints: Hints = field(default_factory=Hints)
    strategy: str = "auto"
    alias: str = "none"
    chip: str = DEFAULT_CHIP
    force_fusion: bool = False
    scale: float = 1.0
    debug_visits: bool = False
    mask: bool = False
    optimizations: Optimizations = field(default_factory=Optimizations)
    smem_per_cta: int = 65536
    regs_budget: int = 65536

    def __post_init__(self) -> None:
        if self.op not in ("sum", "max", "softmax"):
            raise ValidationError("op must be sum, max or softmax")
        if self.dtype not in ("f32", "bf16"):
            raise ValidationError("dtype must be f32 or bf16; accumulation is always f32")
        if type(self.feature_dim) is not int or not 1 <= self.feature_dim <= 1024:
            raise ValidationError("feature_dim must be a static integer in [1, 1024]")
        if self.offsets_dtype not in ("i32", "i64"):
            raise ValidationError("offsets_dtype must be i32 or i64")
        if not isinstance(self.hints, Hints):
            raise ValidationError("hints must be Hints")
        if self.strategy not in ("auto", "naive"):
            raise ValidationError("strategy must be auto or naive")
        if self.alias not in ("none", "inplace"):
            raise ValidationError("alias must be none or inplace")
        if self.alias == "inplace" and self.op != "softmax":
            raise ValidationError("in-place output is only defined for softmax")
        if self.chip not in CHIPS:
            raise ValidationError("chip must be gfx950")
        if type(self.force_fusion) is not bool:
            raise ValidationError("force_fusion must be bool")
        if type(self.debug_visits) is not bool:
            raise ValidationError("debug_visits must be bool")
        if type(self.mask) is not bool:
            raise ValidationError("mask must be bool")
        if self.mask and self.op != "softmax":
            raise ValidationError("additive mask is only defined for softmax")
        if not isinstance(self.optimizations, Optimizations):
            raise ValidationError("optimizations must be Optimizations")
        if self.debug_visits and not self.optimizations.classification:
            raise ValidationError("debug_visits requires classification")
        if self.force_fusion and not self.optimizations.online_fusion:
            raise ValidationError("force_fusion conflicts with online_fusion disabled")
        if self.force_fusion and self.op != "softmax":
            raise ValidationError("force_fusion is only defined for softmax")
        if (type(self.scale) not in (int, float) or abs(self.scale) > 3.402823466e38
                or not math.isfinite(self.scale)):
            raise ValidationError("scale must be a finite f32 value")
        for name in ("smem_per_cta", "regs_budget"):
            value = getattr(self, name)
            if type(value) is not int or not 1 <= value <= 2**63 - 1:
                raise ValidationError(f"{name} must be a positive signed i64 integer")

    @property
    def signature(self) -> str:
        """Semantic tensor signature that hints and mapping policy specialise."""
        return f"{self.op}:{self.dtype}:D{self.feature_dim}:{self.offsets_dtype}:{self.chip}"

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @classmethod
    def from_dict(cls, data: dict[str, Any]) -> "ProgramSpec":
        data = dict(data)
        data["hints"] = Hints(**data.get("hints", {}))
        data["optimizations"] = Optimizations(**data.get("optimizations", {}))
        return cls(**data)

    def source_text(self) -> str:
        """Canonical text of everything that selects device code or its
        launch: stable key order, the f32 value of scale, final newline."""
        body = self.to_dict()
        body["scale"] = float.hex(float(_f32(self.scale)))
        body["optimizations"] = {name: getattr(self.optimizations, name) for name in BOOL_OPTIONS} | {
            "feature_tile": self.optimizations.feature_tile}
        return f"{SOURCE_FORMAT} dialect={DIALECT_VERSION}\n{canonical_json(body)}\n"

    @property
    def ir_hash(self) -> str:
        return hashlib.sha256(self.source_text().encode()).hexdigest()


def _f32(value: float) -> float:
    import struct
    return struct.unpack("f", struct.pack("f", value))[0]


@dataclass(frozen=True)
class ExecutionReport:
    """What one call launched (reference model.py:200-237)."""
    classes: tuple[str, ...]
    thresholds: tuple[int, ...]
    grids: tuple[tuple[int, int, int], ...]
    workspace_bytes: int
    cache_key: str
    fallback_reason: str | None = None
    mode: str = "validated"
    kernel_names: tuple[str, ...] = ()
    host_enqueue_ms: float | None = None
    device_elapsed_ms: float | None = None
    cache_hit: bool = False
    validation_workspace_bytes: int = 0
    validation_host_ms: float | None = None
    optimizations: dict[str, Any] | None = None
    d_tile: int | None = None
    d_vector: int = 1
    pointwise_materialized: bool = False
    resources: dict[str, Any] | None = None
    streams: int = 1
    selected: str | None = None
    selection: dict[str, Any] | None = None

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    def to_json(self) -> str:
        return json.dumps(self.to_dict(), sort_keys=True, indent=2, allow_nan=False)
