"""``Compiler``: bind a ProgramSpec to the ahead-of-time gfx950 library.

Same surface as the reference's ``python/ragged/compiler.py`` (:42-247):
``Compiler(executable=None, *, timeout=300, toolchain_record=None)`` and
``compile(spec, cache, *, adaptive=True)`` returning a ``CompiledProgram``
that, when it classifies, carries its block-per-segment companion as
``.naive``. No code is generated at run time: "compiling" resolves the
spec's kernel specialisation, class thresholds and workspace from the HIP
library, writes the manifest, and publishes it in the artifact cache keyed by
the spec's source hash and the library's sha256. A library rebuilt with
different code therefore misses the cache instead of reusing stale metadata.
"""
from __future__ import annotations

from dataclasses import dataclass, replace
import json
import os
from pathlib import Path
from typing import Any

from . import native
from .cache import Artifact, ArtifactCache, CacheKey, parse_strict_json
from .errors import CacheMismatch, CacheMiss, CompilationError, RuntimeUnavailable, ToolchainUnavailable
from .model import DIALECT_VERSION, ProgramSpec, canonical_json
from .validation import build_manifest, validate_manifest

TOOLCHAIN_FIELDS = ("library_sha256", "build_info", "abi_version", "dialect_version", "chip")
EMITS = ("legal", "plan", "gpu", "nvvm", "ptx", "cubin")


@dataclass(frozen=True)
class CompilationResult:
    """One lowering stage of a spec (reference compiler.py:24-28): its bytes,
    diagnostics, the stage name and the command that produced it."""
    output: bytes
    diagnostics: str
    emit: str
    command: tuple[str, ...]


class Compiler:
    """The HIP library this process loads, or, with ``toolchain_record``, a
    recorded identity under which only precompiled artifacts are served."""

    def __init__(self, executable: str | os.PathLike[str] | None = None, *, timeout: float = 300,
                 toolchain_record: str | os.PathLike[str] | None = None):
        # ``executable`` and ``timeout`` are accepted for the reference's
        # signature; no compiler process is started.
        self.executable = str(executable) if executable is not None else None
        self.timeout = timeout
        self.record = None if toolchain_record is None else self._load_record(Path(toolchain_record))

    @staticmethod
    def _load_record(path: Path) -> dict[str, Any]:
        try:
            data = parse_strict_json(path.read_text(encoding="utf-8"))
        except (OSError, ValueError, UnicodeError) as exc:
            raise ToolchainUnavailable(f"cannot read toolchain record {path}: {exc}") from exc
        if (not isinstance(data, dict) or set(data) != {"schema", "toolchain"} or data["schema"] != 2
                or not isinstance(data["toolchain"], dict)
                or any(field not in data["toolchain"] for field in TOOLCHAIN_FIELDS)):
            raise ToolchainUnavailable(f"toolchain record {path} is malformed")
        return data

    def toolchain(self) -> dict[str, Any]:
        """Identity of the code artifacts bind to."""
        if self.record is not None:
            return dict(self.record["toolchain"])
        try:
            lib = native.library()
            identity = {"library_sha256": native.library_sha256(), "build_info": native.build_info(),
                        "abi_version": int(lib.rg_abi_version()), "dialect_version": DIALECT_VERSION,
                        "chip": "gfx950"}
        except RuntimeUnavailable as exc:
            raise ToolchainUnavailable(str(exc)) from exc
        return identity

    def record_toolchain(self, path: str | os.PathLike[str]) -> dict[str, Any]:
        """Write the identity a toolchain-record Compiler serves artifacts under."""
        if self.record is not None:
            raise ToolchainUnavailable("a toolchain record is written from the real library")
        data = {"schema": 2, "toolchain": self.toolchain()}
        Path(path).write_text(json.dumps(data, indent=2, sort_keys=True) + "\n", encoding="utf-8")
        return data

    @staticmethod
    def _manifest(spec: ProgramSpec, toolchain: dict[str, Any]) -> dict[str, Any]:
        """The manifest an artifact of ``spec`` records: the library's class
        thresholds and part size for it, and whether softmax runs
        register-resident with those effective thresholds."""
        defaults = native.make_spec(spec.op, spec.dtype, spec.offsets_dtype, spec.feature_dim, scale=spec.scale,
                                    mask=spec.mask, vectorize=spec.optimizations.vectorize,
                                    debug_visits=spec.debug_visits)
        metadata = build_manifest(spec, thresholds=(int(defaults.t_wave), int(defaults.t_block)),
                                  part_rows=int(defaults.part_rows), library_sha256=toolchain["library_sha256"],
                                  build_info=toolchain["build_info"])
        if metadata["thresholds"]:
            # Optimizations can move the thresholds; the register-resident
            # softmax depends on the effective ones.
            effective = native.make_spec(spec.op, spec.dtype, spec.offsets_dtype, spec.feature_dim,
                                         scale=spec.scale, mask=spec.mask, vectorize=spec.optimizations.vectorize,
                                         debug_visits=spec.debug_visits, t_wave=metadata["thresholds"][0],
                                         t_block=metadata["thresholds"][1], part_rows=metadata["part_rows"])
            if native.uses_fused(effective):
                metadata = build_manifest(spec, thresholds=tuple(metadata["thresholds"]),
                                          part_rows=metadata["part_rows"], library_sha256=toolchain["library_sha256"],
                                          build_info=toolchain["build_info"], fused=True)
        return metadata

    def lower(self, spec: ProgramSpec, *, emit: str = "gpu", explain: bool = False,
              features: str = "gfx950") -> CompilationResult:
        """The reference's staged lowering (compiler.py:114-144). Its stages
        that exist here: ``legal`` is the spec's canonical source text (what
        its ir_hash covers) and ``plan`` the manifest ``compile`` publishes
        (kernels, classes, thresholds, workspace layout rule). The MLIR/NVVM
        stages (gpu, nvvm, ptx, cubin) have no counterpart: the gfx950
        kernels are compiled ahead of time into libragged_hip.so, so they
        raise CompilationError. ``explain`` adds the stage's rationale to the
        diagnostics; ``features`` is recorded in the command."""
        if emit not in EMITS:
            raise ValueError("emit must be legal, plan, gpu, nvvm, ptx or cubin")
        command = (native.LIBRARY_PATH.name, f"--emit={emit}", f"--chip={spec.chip}", f"--features={features}") + \
            (("--explain",) if explain else ())
        if emit == "legal":
            text = spec.source_text()
            notes = "canonical source text of the specialisation (sha256 = ir_hash)" if explain else ""
            return CompilationResult(text.encode(), notes, emit, command)
        if emit == "plan":
            metadata = self._manifest(spec, self.toolchain())
            notes = "kernels, classes and thresholds the published artifact records" if explain else ""
            return CompilationResult((canonical_json(metadata) + "\n").encode(), notes, emit, command)
        raise CompilationError(f"--emit={emit} has no counterpart in this build: there is no MLIR/NVVM lowering, "
                               "the gfx950 kernels are compiled ahead of time into libragged_hip.so")

    def compile(self, spec: ProgramSpec, cache: ArtifactCache, *, adaptive: bool = True):
        """Resolve (or load) the artifact of ``spec``; with ``adaptive`` a
        classifying program also gets its block-per-segment companion."""
        program = self._compile(spec, cache)
        if not adaptive or not program.selects:
            return program
        naive = self._compile(replace(spec, strategy="naive"), cache)
        from .runtime import CompiledProgram
        return CompiledProgram(spec, program.artifact, cache_hit=program.cache_hit and naive.cache_hit, naive=naive)

    def _compile(self, spec: ProgramSpec, cache: ArtifactCache):
        from .runtime import CompiledProgram
        toolchain = self.toolchain()
        if toolchain.get("dialect_version") != DIALECT_VERSION:
            raise CompilationError("recorded dialect version differs from the frontend")
        key = CacheKey.from_spec(spec, library_sha256=toolchain["library_sha256"],
                                 build_info=toolchain["build_info"])
        try:
            return CompiledProgram(spec, cache.load(key), cache_hit=True)
        except CacheMiss:
            if self.record is not None:
                raise CacheMiss(f"{spec.signature} {spec.strategy} ({spec.ir_hash[:16]}) was not precompiled into "
                                f"{cache.root}; a toolchain-record Compiler builds nothing") from None
        metadata = self._manifest(spec, toolchain)
        validate_manifest(metadata)
        code = (canonical_json({"library": native.LIBRARY_PATH.name, **toolchain}) + "\n").encode()
        # Bind the manifest to its source before publication.
        CompiledProgram(spec, Artifact(cache.entry_path(key), key, code, metadata))
        artifact = cache.publish(key, code, metadata)
        if artifact.metadata != json.loads(canonical_json(metadata)):
            raise CacheMismatch("published metadata differs from the manifest")
        return CompiledProgram(spec, artifact, cache_hit=False)
