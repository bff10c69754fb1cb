"""Artifact store: one self-describing file per compiled specialisation.

Public surface of the reference's ``python/ragged/cache.py`` (:32-192):
``CacheKey`` (``from_spec``, ``to_dict``, ``digest``, ``signature``),
``Artifact`` and ``ArtifactCache(root, *, max_specializations=None)`` with
``load``, ``publish`` and ``entry_path``; the guarantees are the same --
content addressing, fail-closed loads, atomic publication that never replaces
an entry, and a per-signature budget of specialisations. The storage is this
package's own:

* ``<root>/sig-<sha256(signature)[:32]>/<key digest>.rgart``, one file per
  artifact: the line ``RGART1``, one line of canonical JSON (the header: the
  key, its digest and signature, the payload's byte count and sha256, the
  metadata and its sha256), then the payload bytes.
* ``load`` opens the file without following symbolic links and accepts it
  only if every header field is present, of its type and consistent with the
  requested key, the payload and the metadata; anything else raises
  ``CacheMismatch`` (a missing file is ``CacheMiss``).
* ``publish`` writes a hidden temporary file (exclusive create, fsync) and
  links it to the entry name, which fails if the name exists, so a published
  entry is never overwritten or seen half-written; an interrupted publication
  leaves only a hidden file that no load or budget count ever reads. A
  per-signature ``flock`` serialises publishers for the budget.

The payload here is the binding to the HIP library (its identity), not a
cubin: kernels are compiled ahead of time.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import asdict, dataclass, fields
import errno
import fcntl
import hashlib
import json
import os
from pathlib import Path
import secrets
from typing import Any, Iterator

from .errors import CacheError, CacheMismatch, CacheMiss, SpecializationLimit, ValidationError
from .model import ProgramSpec, canonical_json

MAGIC = b"RGART1\n"
SUFFIX = ".rgart"
HEADER_FIELDS = ("digest", "key", "metadata", "metadata_sha256", "payload_bytes", "payload_sha256", "signature")


def sha256_hex(data: bytes) -> str:
    return hashlib.sha256(data).hexdigest()


def strict_json_object(pairs: list[tuple[str, Any]]) -> dict[str, Any]:
    """``object_pairs_hook`` that refuses a repeated key (json would keep the
    last one silently)."""
    seen: dict[str, Any] = {}
    for name, value in pairs:
        if name in seen:
            raise ValueError(f"repeated JSON field {name!r}")
        seen[name] = value
    return seen


def _refuse_constant(name: str):
    raise ValueError(f"non-finite JSON number {name}")


def parse_strict_json(text: str) -> Any:
    """JSON with unique keys and finite numbers only."""
    return json.loads(text, object_pairs_hook=strict_json_object, parse_constant=_refuse_constant)


def _is_sha256(value: Any) -> bool:
    return isinstance(value, str) and len(value) == 64 and set(value) <= set("0123456789abcdef")


def _nonempty_text(value: Any) -> bool:
    return isinstance(value, str) and bool(value.strip())


@dataclass(frozen=True)
class CacheKey:
    """What identifies compiled code: the spec's source hash, the identity of
    the HIP library it binds to, and the tensor signature it specialises."""
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

    # (field, predicate, message) checked in order by __post_init__.
    _CHECKS = (
        ("ir_hash", _is_sha256, "ir_hash must be a SHA256 hex digest"),
        ("library_sha256", _is_sha256, "library_sha256 must be a SHA256 hex digest"),
        ("dialect_version", _nonempty_text, "cache key requires a nonempty dialect_version"),
        ("build_info", _nonempty_text, "cache key requires a nonempty build_info"),
    )

    def __post_init__(self) -> None:
        for name, accept, message in self._CHECKS:
            if not accept(getattr(self, name)):
                raise ValidationError(message)
        # The signature fields must describe a valid program.
        ProgramSpec(self.op, self.dtype, self.feature_dim, self.offsets_dtype, strategy=self.strategy, chip=self.chip)

    @classmethod
    def from_spec(cls, spec: ProgramSpec, *, library_sha256: str, build_info: str,
                  dialect_version: str = "1") -> "CacheKey":
        return cls(ir_hash=spec.ir_hash, dialect_version=dialect_version, library_sha256=library_sha256,
                   build_info=build_info, chip=spec.chip, strategy=spec.strategy, dtype=spec.dtype,
                   feature_dim=spec.feature_dim, offsets_dtype=spec.offsets_dtype, op=spec.op)

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)

    @property
    def digest(self) -> str:
        return sha256_hex(canonical_json(self.to_dict()).encode())

    @property
    def signature(self) -> str:
        return f"{self.op}:{self.dtype}:D{self.feature_dim}:{self.offsets_dtype}:{self.chip}"


KEY_FIELDS = tuple(f.name for f in fields(CacheKey))


@dataclass(frozen=True)
class Artifact:
    path: Path
    key: CacheKey
    code_object: bytes
    metadata: dict[str, Any]


def encode_artifact(key: CacheKey, code_object: bytes, metadata: dict[str, Any]) -> bytes:
    """The file image of one artifact (``metadata`` already canonical)."""
    header = {"digest": key.digest, "key": key.to_dict(), "metadata": metadata,
              "metadata_sha256": sha256_hex(canonical_json(metadata).encode()),
              "payload_bytes": len(code_object), "payload_sha256": sha256_hex(code_object),
              "signature": key.signature}
    return MAGIC + canonical_json(header).encode() + b"\n" + code_object


def decode_artifact(image: bytes, key: CacheKey) -> tuple[bytes, dict[str, Any]]:
    """(payload, metadata) of a file image, which must describe exactly
    ``key``; CacheMismatch otherwise."""
    if not image.startswith(MAGIC):
        raise CacheMismatch("artifact file lacks the RGART1 magic line")
    end = image.find(b"\n", len(MAGIC))
    if end < 0:
        raise CacheMismatch("artifact header is not terminated")
    try:
        header = parse_strict_json(image[len(MAGIC):end].decode("utf-8"))
    except (UnicodeDecodeError, ValueError) as exc:
        raise CacheMismatch(f"artifact header is not valid JSON: {exc}") from exc
    if not isinstance(header, dict) or tuple(sorted(header)) != HEADER_FIELDS:
        raise CacheMismatch("artifact header fields differ from the format's")
    stored = header["key"]
    if not isinstance(stored, dict) or tuple(sorted(stored)) != tuple(sorted(KEY_FIELDS)):
        raise CacheMismatch("artifact key fields differ from the format's")
    wanted = key.to_dict()
    for name in KEY_FIELDS:
        if type(stored[name]) is not type(wanted[name]) or stored[name] != wanted[name]:
            raise CacheMismatch(f"artifact key differs from the requested key in {name}")
    if header["digest"] != key.digest:
        raise CacheMismatch("artifact digest differs from the requested key's")
    if header["signature"] != key.signature:
        raise CacheMismatch("artifact signature differs from the requested key's")
    metadata = header["metadata"]
    if not isinstance(metadata, dict):
        raise CacheMismatch("artifact metadata must be an object")
    if header["metadata_sha256"] != sha256_hex(canonical_json(metadata).encode()):
        raise CacheMismatch("artifact metadata does not match its sha256")
    payload = image[end + 1:]
    size = header["payload_bytes"]
    if type(size) is not int or size != len(payload) or size == 0:
        raise CacheMismatch("artifact payload is empty or its length differs from the header")
    if header["payload_sha256"] != sha256_hex(payload):
        raise CacheMismatch("artifact payload does not match its sha256")
    return payload, metadata


def _canonical_metadata(metadata: Any) -> dict[str, Any]:
    if not isinstance(metadata, dict):
        raise ValidationError("artifact metadata must be a dictionary")
    try:
        return parse_strict_json(canonical_json(metadata))
    except (TypeError, ValueError) as exc:
        raise ValidationError(f"artifact metadata must be finite JSON: {exc}") from exc


def _fsync_directory(path: Path) -> None:
    handle = os.open(path, os.O_RDONLY | os.O_DIRECTORY)
    try:
        os.fsync(handle)
    finally:
        os.close(handle)


class ArtifactCache:
    """Artifacts under ``root`` (see the module docstring for the format);
    at most ``max_specializations`` per tensor signature."""

    MAX_SPECIALIZATIONS = 16

    def __init__(self, root: str | os.PathLike[str], *, max_specializations: int | None = None):
        self.root = Path(root).expanduser()
        if max_specializations is not None:
            if type(max_specializations) is not int or max_specializations < 1:
                raise ValidationError("max_specializations must be a positive integer")
            self.MAX_SPECIALIZATIONS = max_specializations

    def signature_dir(self, key: CacheKey) -> Path:
        return self.root / f"sig-{sha256_hex(key.signature.encode())[:32]}"

    def entry_path(self, key: CacheKey) -> Path:
        return self.signature_dir(key) / f"{key.digest}{SUFFIX}"

    def entries(self, key: CacheKey) -> list[Path]:
        """Published artifacts of ``key``'s signature (hidden files excluded)."""
        directory = self.signature_dir(key)
        if not directory.is_dir():
            return []
        return sorted(p for p in directory.iterdir() if p.name.endswith(SUFFIX) and not p.name.startswith("."))

    # ------------------------------------------------------------------
    def load(self, key: CacheKey) -> Artifact:
        path = self.entry_path(key)
        directory = path.parent
        if directory.is_symlink():
            raise CacheMismatch(f"signature directory must not be a symbolic link: {directory}")
        try:
            handle = os.open(path, os.O_RDONLY | os.O_NOFOLLOW)
        except FileNotFoundError:
            raise CacheMiss(f"no compiled artifact for {key.digest}") from None
        except OSError as exc:
            if exc.errno == errno.ELOOP:
                raise CacheMismatch(f"artifact must not be a symbolic link: {path}") from exc
            raise CacheMismatch(f"cannot open artifact {path}: {exc}") from exc
        try:
            with os.fdopen(handle, "rb") as stream:
                image = stream.read()
        except OSError as exc:
            raise CacheMismatch(f"cannot read artifact {path}: {exc}") from exc
        payload, metadata = decode_artifact(image, key)
        return Artifact(path, key, payload, metadata)

    @contextmanager
    def _publishing(self, key: CacheKey) -> Iterator[Path]:
        directory = self.signature_dir(key)
        directory.mkdir(parents=True, exist_ok=True)
        with open(directory / ".publish-lock", "a+b") as lock:
            fcntl.flock(lock.fileno(), fcntl.LOCK_EX)
            try:
                yield directory
            finally:
                fcntl.flock(lock.fileno(), fcntl.LOCK_UN)

    def publish(self, key: CacheKey, code_object: bytes, metadata: dict[str, Any]) -> Artifact:
        """Store an artifact, or return the identical one already stored.
        A different artifact under the same key raises CacheMismatch; a new
        one past the signature's budget raises SpecializationLimit."""
        if not isinstance(code_object, bytes) or not code_object:
            raise ValidationError("code object must be nonempty bytes")
        metadata = _canonical_metadata(metadata)
        image = encode_artifact(key, code_object, metadata)
        with self._publishing(key) as directory:
            destination = self.entry_path(key)
            if os.path.lexists(destination):
                existing = self.load(key)
                if existing.code_object != code_object or existing.metadata != metadata:
                    raise CacheMismatch("refusing to replace an immutable artifact with different content")
                return existing
            if len(self.entries(key)) >= self.MAX_SPECIALIZATIONS:
                raise SpecializationLimit(f"signature {key.signature} already holds "
                                          f"{self.MAX_SPECIALIZATIONS} specializations")
            pending = directory / f".pending-{secrets.token_hex(8)}{SUFFIX}"
            handle = os.open(pending, os.O_WRONLY | os.O_CREAT | os.O_EXCL, 0o644)
            try:
                with os.fdopen(handle, "wb") as stream:
                    stream.write(image)
                    stream.flush()
                    os.fsync(stream.fileno())
                os.link(pending, destination)      # fails if the entry exists: never replaces
                _fsync_directory(directory)
            except FileExistsError as exc:
                raise CacheError(f"artifact {destination} appeared during publication") from exc
            finally:
                try:
                    os.unlink(pending)
                except FileNotFoundError:
                    pass
        return self.load(key)
