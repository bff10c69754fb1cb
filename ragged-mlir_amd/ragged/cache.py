"""Content-addressed artifact cache with fail-closed loads and atomic publish.

Behaviour of the reference's ``python/ragged/cache.py`` (:32-192): entries
live under ``<root>/<sha256(signature)>/<key digest>/`` as a payload file plus
``manifest.json``; an entry becomes visible only after both files are
fsynced and its temporary directory renamed; anything incomplete, mismatched
or symlinked raises ``CacheMismatch``; an existing entry is immutable; at most
``MAX_SPECIALIZATIONS`` entries per signature. The payload here is the code
object binding (the HIP library's identity), not a cubin.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import asdict, dataclass
import fcntl
import hashlib
import json
import os
from pathlib import Path
import shutil
import tempfile
from typing import Any, Iterator

from .errors import CacheError, CacheMismatch, CacheMiss, SpecializationLimit, ValidationError
from .model import ProgramSpec, canonical_json

PAYLOAD = "code_object.json"


def _sha(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def _unique_object(pairs):
    result = {}
    for key, value in pairs:
        if key in result:
            raise ValueError(f"duplicate manifest field: {key}")
        result[key] = value
    return result


def _hex64(value: Any) -> bool:
    return isinstance(value, str) and len(value) == 64 and all(c in "0123456789abcdef" for c in value)


@dataclass(frozen=True)
class CacheKey:
    """Everything that identifies compiled code: the spec's source hash, the
    toolchain (library build) and the tensor signature (reference cache.py:32-76)."""
    ir_hash: str
    dialect_version: str
    library_sha256: str
    build_info: str
    chip: str
    strategy: str
    dtype: str
    feature_dim: int
    offsets_dtype: str
    op: str

    def __post_init__(self) -> None:
        if not _hex64(self.ir_hash):
            raise ValidationError("ir_hash must be a SHA256 hex digest")
        if not _hex64(self.library_sha256):
            raise ValidationError("library_sha256 must be a SHA256 hex digest")
        for name in ("dialect_version", "build_info"):
            value = getattr(self, name)
            if not isinstance(value, str) or not value.strip():
                raise ValidationError(f"cache key requires a nonempty {name}")
        ProgramSpec(self.op, self.dtype, self.feature_dim, self.offsets_dtype, strategy=self.strategy, chip=self.chip)

    @classmethod
    def from_spec(cls, spec: ProgramSpec, *, library_sha256: str, build_info: str,
                  dialect_version: str = "1") -> "CacheKey":
        return cls(spec.ir_hash, dialect_version, library_sha256, build_info, spec.chip, spec.strategy,
                   spec.dtype, spec.feature_dim, spec.offsets_dtype, spec.op)

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @property
    def digest(self) -> str:
        return _sha(canonical_json(self.to_dict()).encode())

    @property
    def signature(self) -> str:
        return f"{self.op}:{self.dtype}:D{self.feature_dim}:{self.offsets_dtype}:{self.chip}"


@dataclass(frozen=True)
class Artifact:
    path: Path
    key: CacheKey
    code_object: bytes
    metadata: dict[str, Any]


class ArtifactCache:
    """Per-signature ``flock`` guards the specialisation budget; readers never
    treat partial files as hits; corrupt entries are reported, not replaced."""

    SCHEMA = 1
    MAX_SPECIALIZATIONS = 16

    def __init__(self, root: str | os.PathLike[str], *, max_specializations: int | None = None):
        self.root = Path(root).expanduser()
        if max_specializations is not None:
            if type(max_specializations) is not int or max_specializations < 1:
                raise ValidationError("max_specializations must be a positive integer")
            self.MAX_SPECIALIZATIONS = max_specializations

    def _signature_dir(self, key: CacheKey) -> Path:
        return self.root / _sha(key.signature.encode())

    def entry_path(self, key: CacheKey) -> Path:
        return self._signature_dir(key) / key.digest

    @contextmanager
    def _locked(self, key: CacheKey) -> Iterator[Path]:
        directory = self._signature_dir(key)
        directory.mkdir(parents=True, exist_ok=True)
        with (directory / ".publish.lock").open("a+b") as lock:
            fcntl.flock(lock, fcntl.LOCK_EX)
            try:
                yield directory
            finally:
                fcntl.flock(lock, fcntl.LOCK_UN)

    def load(self, key: CacheKey) -> Artifact:
        path = self.entry_path(key)
        if not path.exists() and not path.is_symlink():
            raise CacheMiss(f"no compiled artifact for {key.digest}")
        try:
            if path.is_symlink() or not path.is_dir():
                raise CacheMismatch(f"cache entry must be a directory: {path}")
            for name in ("manifest.json", PAYLOAD):
                if (path / name).is_symlink():
                    raise CacheMismatch(f"cache artifact must not be a symbolic link: {name}")
            manifest = json.loads((path / "manifest.json").read_text(encoding="utf-8"),
                                  object_pairs_hook=_unique_object)
            fields = {"schema", "key", "cache_key", "signature", "code_sha256", "metadata", "metadata_sha256"}
            if not isinstance(manifest, dict) or set(manifest) != fields:
                raise CacheMismatch("cache manifest schema fields differ")
            if type(manifest["schema"]) is not int or manifest["schema"] != self.SCHEMA:
                raise CacheMismatch("cache manifest schema version differs")
            if canonical_json(manifest["key"]) != canonical_json(key.to_dict()):
                raise CacheMismatch("cache manifest key differs from the requested key")
            if manifest["cache_key"] != key.digest or manifest["signature"] != key.signature:
                raise CacheMismatch("cache manifest digest or signature differs")
            if not isinstance(manifest["metadata"], dict):
                raise CacheMismatch("cache metadata must be an object")
            if _sha(canonical_json(manifest["metadata"]).encode()) != manifest["metadata_sha256"]:
                raise CacheMismatch("kernel metadata does not match manifest SHA256")
            code = (path / PAYLOAD).read_bytes()
            if not code or _sha(code) != manifest["code_sha256"]:
                raise CacheMismatch("code object is empty or does not match manifest SHA256")
            return Artifact(path, key, code, manifest["metadata"])
        except CacheError:
            raise
        except (OSError, ValueError, TypeError, KeyError) as exc:
            raise CacheMismatch(f"incomplete or invalid cache entry {path}: {exc}") from exc

    def publish(self, key: CacheKey, code_object: bytes, metadata: dict[str, Any]) -> Artifact:
        if not isinstance(code_object, bytes) or not code_object:
            raise ValidationError("code object must be nonempty bytes")
        if not isinstance(metadata, dict):
            raise ValidationError("artifact metadata must be a dictionary")
        metadata = json.loads(canonical_json(metadata))
        manifest = {"schema": self.SCHEMA, "key": key.to_dict(), "cache_key": key.digest,
                    "signature": key.signature, "code_sha256": _sha(code_object), "metadata": metadata,
                    "metadata_sha256": _sha(canonical_json(metadata).encode())}
        with self._locked(key) as directory:
            destination = self.entry_path(key)
            if destination.exists() or destination.is_symlink():
                artifact = self.load(key)
                if artifact.code_object != code_object or artifact.metadata != metadata:
                    raise CacheMismatch("refusing to replace immutable artifact with different content")
                return artifact
            entries = [entry for entry in directory.iterdir() if not entry.name.startswith(".")]
            if len(entries) >= self.MAX_SPECIALIZATIONS:
                raise SpecializationLimit(
                    f"signature {key.signature} already has {self.MAX_SPECIALIZATIONS} specializations")
            temporary = Path(tempfile.mkdtemp(prefix=".pending-", dir=directory))
            try:
                for name, data in ((PAYLOAD, code_object),
                                   ("manifest.json", (canonical_json(manifest) + "\n").encode())):
                    with (temporary / name).open("xb") as stream:
                        stream.write(data)
                        stream.flush()
                        os.fsync(stream.fileno())
                self._fsync_dir(temporary)
                os.rename(temporary, destination)
                self._fsync_dir(directory)
            finally:
                if temporary.exists():
                    shutil.rmtree(temporary)
        return self.load(key)

    @staticmethod
    def _fsync_dir(path: Path) -> None:
        fd = os.open(path, os.O_RDONLY | os.O_DIRECTORY)
        try:
            os.fsync(fd)
        finally:
            os.close(fd)
