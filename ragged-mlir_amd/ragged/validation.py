"""Kernel manifests: construction from a spec, validation, and the checked
mode's status decoding.

The reference validates the JSON sidecar its compiler writes
(python/ragged/validation.py:97-354) and binds it to the spec and cache key.
Here the "compiler" is the ahead-of-time HIP library, so ``build_manifest``
derives the launch sequence, classes, thresholds and workspace of a spec
from the library's own defaults, and ``validate_manifest`` /
``validate_program`` re-check every field fail-closed before any launch.
``raise_for_status`` restates validation.py:76-94 (checked-abi.md).
"""
from __future__ import annotations

import re
from typing import TYPE_CHECKING, Any

from .errors import CacheMismatch, ValidationError
from .model import DEFAULT_CHIP, ProgramSpec, _f32

if TYPE_CHECKING:
    from .cache import Artifact

ABI = "ragged-hip-v1"
DISPATCH_ABI = "classified-wave64-v1"
CONDITIONS = ("first_nonzero", "final_mismatch", "negative", "above_n",
              "nonmonotone", "below_min_len", "above_max_len")
I64_MAX = 2**63 - 1
STATUS_WORKSPACE = [{"name": "validation_status", "dtype": "i64", "shape": [7]}]
NO_SPLIT = 2**62          # t_block when the split class is disabled


def _phase(op: str) -> str:
    return "online" if op == "softmax" else op


def kernel_roles(spec: ProgramSpec, classes: list[str], fused: bool = False) -> list[str]:
    """Role names in launch order. The classified schedule runs classify
    (which also initialises the per-segment state of the call) and one
    worker over the wave, block and split classes (a softmax's worker also
    normalises its split parts); with ``fused`` a softmax runs classify and
    its register-resident worker, which also takes the wave class and
    re-reads the chunks that stopped waiting. The last kernel's last
    workgroup returns the workspace's counters to zero."""
    phase = _phase(spec.op)
    if classes == ["block"] and spec.strategy == "naive":
        return [phase]
    if fused:
        return ["classify", "fused_online"]
    roles = ["classify"]
    # One persistent worker drains every class; the reference's per-class
    # chains, split combine and (softmax) split normalisation run inside it.
    roles.append(f"worker_{phase}")
    return roles


def workspace_layout(spec: ProgramSpec, classified: bool, fused: bool = False) -> list[dict[str, Any]]:
    """Symbolic workspace list; byte sizes are resolved per call by the
    library (rg_plan_create) from N and B."""
    if not classified:
        return []
    d = spec.feature_dim
    workspace = [{"name": "class_counts", "dtype": "i64", "shape": [8]},
                 {"name": "segment_ids", "dtype": "i64", "shape": [3, "B"]}]
    if fused:
        workspace += [{"name": "deferred", "dtype": "i64", "shape": ["items"]},
                      {"name": "arrive", "dtype": "i32", "shape": ["items"]},
                      {"name": "items", "dtype": "i64", "shape": ["items", 4]},
                      {"name": "block_items", "dtype": "i64", "shape": ["B", 4]},
                      {"name": "pairs", "dtype": "i64", "shape": ["items", d]},
                      {"name": "final_pairs", "dtype": "i64", "shape": ["B_split", d]}]
        if spec.debug_visits:
            workspace.append({"name": "visits", "dtype": "i32", "shape": ["B"]})
        return workspace
    workspace += [{"name": "item_segments", "dtype": "i64", "shape": ["items"]},
                  {"name": "part_begin", "dtype": "i64", "shape": ["B_split"]},
                  {"name": "partials", "dtype": "f32", "shape": ["items", d]}]
    if spec.op == "softmax":
        workspace += [{"name": "partial_sums", "dtype": "f32", "shape": ["items", d]},
                      {"name": "max_stats", "dtype": "f32", "shape": ["B_split", d]},
                      {"name": "sum_stats", "dtype": "f32", "shape": ["B_split", d]},
                      {"name": "deferred", "dtype": "i64", "shape": ["items", "tiles"]}]
    if spec.debug_visits:
        workspace.append({"name": "visits", "dtype": "i32", "shape": ["B"]})
    return workspace


def build_manifest(spec: ProgramSpec, *, thresholds: tuple[int, int], part_rows: int, library_sha256: str,
                   build_info: str, fused: bool = False) -> dict[str, Any]:
    """The manifest of ``spec`` for the library build ``library_sha256``."""
    options = spec.optimizations
    classified = spec.strategy == "auto" and options.classification
    t_wave, t_block = thresholds
    if classified:
        classes = ["wave", "block", "split"]
        if not options.warp_mapping:
            t_wave = 0
        if not options.split_mapping:
            t_block = NO_SPLIT
            classes = ["wave", "block"]
    else:
        classes = ["block"]
    strategy_spec = spec if classified or spec.strategy == "naive" else _as_naive(spec)
    fused = bool(fused and classified and spec.op == "softmax")
    roles = kernel_roles(strategy_spec, classes, fused)
    lpr, vec, mapping = options.geometry(spec.feature_dim, spec.dtype)
    effective = options.effective()
    effective["classification"] = classified
    effective["warp_mapping"] = classified and options.warp_mapping
    effective["split_mapping"] = classified and options.split_mapping
    effective["vectorize"] = vec > 1
    return {
        "schema": 1,
        "abi": ABI,
        "chip": spec.chip,
        "op": spec.op,
        "dtype": spec.dtype,
        "feature_dim": spec.feature_dim,
        "offsets_dtype": spec.offsets_dtype,
        "mask": spec.mask,
        "scale": float(_f32(spec.scale)),
        "dispatch_abi": DISPATCH_ABI if classified else None,
        "backend": "persistent-wave64" if classified else "block-per-segment",
        "classes": classes,
        "thresholds": [int(t_wave), int(t_block)] if classified else [],
        "part_rows": int(part_rows) if classified else None,
        "fusion": "online" if spec.op == "softmax" else "not_applicable",
        "alias_safe": spec.op == "softmax",
        "d_tile": lpr,
        "d_vector": vec,
        "mapping": mapping,
        "debug_visits": spec.debug_visits,
        "kernels": [{"role": role, "name": f"ragged_0_{role}", "block": [256, 1, 1]} for role in roles],
        "workspace": workspace_layout(spec, classified, fused),
        "fused": fused,
        "library_sha256": library_sha256,
        "build_info": build_info,
        "optimizations": {"requested": options.to_dict(), "effective": effective},
        "validation": {"abi": "offsets-check-v1", "workspace": STATUS_WORKSPACE, "conditions": list(CONDITIONS),
                       "sentinel": I64_MAX, "min_len": spec.hints.min_len, "max_len": spec.hints.max_len},
    }


def _as_naive(spec: ProgramSpec) -> ProgramSpec:
    from dataclasses import replace
    return replace(spec, strategy="naive")


def validate_manifest(metadata: dict[str, Any]) -> None:
    """Structural checks that hold for any manifest this package writes."""
    if not isinstance(metadata, dict) or type(metadata.get("schema")) is not int or metadata["schema"] != 1:
        raise CacheMismatch("unsupported kernel manifest schema")
    if metadata.get("abi") != ABI:
        raise CacheMismatch(f"unsupported kernel ABI; expected {ABI}")
    if metadata.get("chip") != DEFAULT_CHIP:
        raise CacheMismatch("kernel manifest chip must be gfx950")
    for name in ("mask", "debug_visits", "alias_safe"):
        if type(metadata.get(name)) is not bool:
            raise CacheMismatch(f"{name} must be boolean")
    if metadata.get("op") not in ("sum", "max", "softmax"):
        raise CacheMismatch("manifest op must be sum, max or softmax")
    if metadata["mask"] and metadata["op"] != "softmax":
        raise CacheMismatch("additive mask is only supported by softmax")
    dispatch = metadata.get("dispatch_abi")
    if dispatch not in (None, DISPATCH_ABI):
        raise CacheMismatch("unsupported dispatch ABI")
    classes = metadata.get("classes")
    if dispatch is None:
        if classes != ["block"] or metadata.get("thresholds") != []:
            raise CacheMismatch("block-per-segment manifests have exactly the block class and no thresholds")
    else:
        if classes not in (["wave", "block", "split"], ["wave", "block"]):
            raise CacheMismatch("classified classes must be wave, block[, split]")
        thresholds = metadata.get("thresholds")
        if (not isinstance(thresholds, list) or len(thresholds) != 2
                or any(type(value) is not int or not 0 <= value <= I64_MAX for value in thresholds)
                or thresholds[0] >= thresholds[1]):
            raise CacheMismatch("thresholds must be two ascending nonnegative i64 row counts")
        if type(metadata.get("part_rows")) is not int or metadata["part_rows"] < 1:
            raise CacheMismatch("part_rows must be a positive integer")
    if metadata.get("d_vector") not in (1, 2, 4, 8) or metadata.get("mapping") not in ("row", "flat"):
        raise CacheMismatch("d_vector must be 1, 2, 4 or 8 with a row or flat mapping")
    kernels = metadata.get("kernels")
    if not isinstance(kernels, list) or not kernels:
        raise CacheMismatch("kernel manifest has no launch sequence")
    names = set()
    for kernel in kernels:
        if (not isinstance(kernel, dict) or set(kernel) != {"role", "name", "block"}
                or not isinstance(kernel["name"], str) or not re.fullmatch(r"[A-Za-z_][A-Za-z0-9_]*", kernel["name"])
                or kernel["block"] != [256, 1, 1]):
            raise CacheMismatch("invalid kernel entry")
        if kernel["name"] in names:
            raise CacheMismatch("kernel symbols must be unique in the launch sequence")
        names.add(kernel["name"])
    workspace = metadata.get("workspace")
    if not isinstance(workspace, list):
        raise CacheMismatch("workspace must be an array")
    for buffer in workspace:
        if (not isinstance(buffer, dict) or set(buffer) != {"name", "dtype", "shape"}
                or buffer["dtype"] not in ("i32", "i64", "f32")):
            raise CacheMismatch("invalid workspace entry")
    validation = metadata.get("validation")
    if (not isinstance(validation, dict) or validation.get("abi") != "offsets-check-v1"
            or validation.get("conditions") != list(CONDITIONS) or validation.get("sentinel") != I64_MAX
            or validation.get("workspace") != STATUS_WORKSPACE):
        raise CacheMismatch("offsets validation metadata differs from offsets-check-v1")


def validate_program(spec: ProgramSpec, artifact: "Artifact", *, library_sha256: str | None = None) -> None:
    """Bind an artifact to ``spec``: key, manifest fields, and (when given)
    the library build that will run it."""
    key = artifact.key
    if key.ir_hash != spec.ir_hash:
        raise CacheMismatch("compiled program source does not match cached IR hash")
    for name in ("op", "dtype", "feature_dim", "offsets_dtype", "strategy", "chip"):
        if getattr(key, name) != getattr(spec, name):
            raise CacheMismatch(f"compiled program {name} differs from artifact key")
    metadata = artifact.metadata
    validate_manifest(metadata)
    for name in ("op", "dtype", "feature_dim", "offsets_dtype", "mask", "debug_visits"):
        if metadata.get(name) != getattr(spec, name):
            raise CacheMismatch(f"kernel manifest {name} differs from the source specialization")
    if metadata.get("library_sha256") != key.library_sha256 or metadata.get("build_info") != key.build_info:
        raise CacheMismatch("kernel manifest is not bound to the library build of its cache key")
    if library_sha256 is not None and key.library_sha256 != library_sha256:
        raise CacheMismatch("artifact was built for a different libragged_hip.so; recompile")
    if type(metadata.get("fused")) is not bool:
        raise CacheMismatch("fused must be boolean")
    expected = build_manifest(spec, thresholds=tuple(metadata["thresholds"]) if metadata["thresholds"] else (0, 1),
                              part_rows=metadata["part_rows"] or 1, library_sha256=key.library_sha256,
                              build_info=key.build_info, fused=metadata["fused"])
    for name in ("kernels", "workspace", "classes", "d_vector", "mapping", "dispatch_abi", "fusion", "scale", "fused"):
        if metadata.get(name) != expected[name]:
            raise CacheMismatch(f"kernel manifest {name} differs from the source specialization")
    validation = metadata["validation"]
    if validation.get("min_len") != spec.hints.min_len or validation.get("max_len") != spec.hints.max_len:
        raise CacheMismatch("offsets validation bounds differ from source hints")


def raise_for_status(status: list[int], *, b: int) -> None:
    """Decode the seven status slots after the stream synchronised
    (checked-abi.md; reference validation.py:76-94)."""
    if not isinstance(status, list) or len(status) != len(CONDITIONS):
        raise ValidationError("invalid offsets validation status layout")
    errors = {}
    for slot, (condition, index) in enumerate(zip(CONDITIONS, status)):
        if type(index) is not int or not 0 <= index <= I64_MAX:
            raise ValidationError("invalid offsets validation status index")
        if index == I64_MAX:
            continue
        limit = b if slot < 4 else b - 1
        if index > limit or (slot == 0 and index != 0) or (slot == 1 and index != b):
            raise ValidationError("offsets validation status index exceeds its condition domain")
        errors[condition] = index
    if errors:
        first = next(iter(errors))
        detail = "; ".join(f"{condition} at index {index}" for condition, index in errors.items())
        raise ValidationError("offsets validation failed: " + detail, condition=first, index=errors[first],
                              errors=errors)
