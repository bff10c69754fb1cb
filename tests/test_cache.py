"""Artifact store faults (CPU): the behaviour of the reference's
test/python/test_cache_adversarial.py:27-150, restated for this build's
one-file-per-artifact format. Synthetic payloads never reach a GPU.
"""
from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
from dataclasses import fields
import hashlib
import json
import os

import pytest

from ragged.cache import MAGIC, ArtifactCache, CacheKey, decode_artifact
from ragged.errors import CacheMismatch, CacheMiss, SpecializationLimit, ValidationError
from ragged.model import Hints, ProgramSpec

PAYLOAD = b"synthetic-artifact-payload"


def make_key(max_len: int = 16) -> CacheKey:
    return CacheKey.from_spec(ProgramSpec("softmax", "f32", 16, "i64", hints=Hints(max_len=max_len)),
                              library_sha256="ab" * 32, build_info="target=gfx950;test")


def publish(cache, key, metadata=None):
    return cache.publish(key, PAYLOAD, {"kernel": "test_kernel"} if metadata is None else metadata)


def split(image: bytes):
    end = image.index(b"\n", len(MAGIC))
    return json.loads(image[len(MAGIC):end]), image[end + 1:]


def join(header, payload: bytes) -> bytes:
    return MAGIC + json.dumps(header).encode() + b"\n" + payload


def test_round_trip_and_identity(tmp_path):
    cache, key = ArtifactCache(tmp_path), make_key()
    artifact = publish(cache, key)
    assert artifact.path == cache.entry_path(key) and artifact.path.name == f"{key.digest}.rgart"
    loaded = cache.load(key)
    assert loaded.code_object == PAYLOAD and loaded.metadata == {"kernel": "test_kernel"} and loaded.key == key
    assert key.digest == hashlib.sha256(json.dumps(key.to_dict(), sort_keys=True, separators=(",", ":"))
                                        .encode()).hexdigest()
    with pytest.raises(CacheMiss):
        cache.load(make_key(17))


@pytest.mark.parametrize("field", [field.name for field in fields(CacheKey)])
def test_each_key_field_is_checked_before_a_hit(tmp_path, field):
    cache, key = ArtifactCache(tmp_path), make_key()
    artifact = publish(cache, key)
    header, payload = split(artifact.path.read_bytes())
    value = header["key"][field]
    header["key"][field] = value + 1 if type(value) is int else value + "-corrupt"
    artifact.path.write_bytes(join(header, payload))
    with pytest.raises(CacheMismatch, match="key differs"):
        cache.load(key)


DAMAGE = ["no_magic", "unterminated_header", "truncated_json", "altered_payload", "empty_payload",
          "extra_field", "missing_field", "wrong_signature", "wrong_digest", "nan_metadata", "repeated_field",
          "altered_metadata", "payload_length", "bool_for_int"]


@pytest.mark.parametrize("damage", DAMAGE)
def test_partial_and_corrupt_entries_fail_closed(tmp_path, damage):
    cache, key = ArtifactCache(tmp_path), make_key()
    path = publish(cache, key).path
    image = path.read_bytes()
    header, payload = split(image)
    if damage == "no_magic":
        image = image[len(MAGIC):]
    elif damage == "unterminated_header":
        image = MAGIC + json.dumps(header).encode()
    elif damage == "truncated_json":
        image = MAGIC + b'{"digest":' + b"\n" + payload
    elif damage == "altered_payload":
        image = join(header, payload[:-1] + b"X")
    elif damage == "empty_payload":
        image = join(header, b"")
    elif damage == "extra_field":
        image = join({**header, "extra": 1}, payload)
    elif damage == "missing_field":
        header.pop("metadata_sha256")
        image = join(header, payload)
    elif damage == "wrong_signature":
        image = join({**header, "signature": "sum:f32:D16:i64:gfx950"}, payload)
    elif damage == "wrong_digest":
        image = join({**header, "digest": "0" * 64}, payload)
    elif damage == "nan_metadata":
        image = MAGIC + json.dumps({**header, "metadata": {"x": float("nan")}}).encode() + b"\n" + payload
    elif damage == "repeated_field":
        text = json.dumps(header)
        image = MAGIC + (text[:-1] + ', "digest": "' + header["digest"] + '"}').encode() + b"\n" + payload
    elif damage == "altered_metadata":
        image = join({**header, "metadata": {"kernel": "other_kernel"}}, payload)
    elif damage == "payload_length":
        image = join({**header, "payload_bytes": len(payload) + 1}, payload)
    elif damage == "bool_for_int":
        header["key"]["feature_dim"] = True
        image = join(header, payload)
    path.write_bytes(image)
    with pytest.raises(CacheMismatch):
        cache.load(key)


def test_missing_file_is_a_miss_not_a_mismatch(tmp_path):
    cache, key = ArtifactCache(tmp_path), make_key()
    publish(cache, key).path.unlink()
    with pytest.raises(CacheMiss):
        cache.load(key)


@pytest.mark.parametrize("part", ["file", "directory"])
def test_symbolic_links_are_rejected(tmp_path, part):
    cache, key = ArtifactCache(tmp_path / "cache"), make_key()
    real = ArtifactCache(tmp_path / "real")
    source = publish(real, key).path
    if part == "file":
        target = cache.entry_path(key)
        target.parent.mkdir(parents=True)
        target.symlink_to(source)
    else:
        cache.root.mkdir()
        cache.signature_dir(key).symlink_to(source.parent, target_is_directory=True)
    with pytest.raises(CacheMismatch, match="symbolic link"):
        cache.load(key)


def test_interrupted_publication_never_creates_a_hit(tmp_path, monkeypatch):
    cache, key = ArtifactCache(tmp_path), make_key()

    def crash(*args, **kwargs):
        raise OSError("simulated crash before the entry is linked")

    monkeypatch.setattr(os, "link", crash)
    with pytest.raises(OSError, match="simulated crash"):
        publish(cache, key)
    monkeypatch.undo()
    with pytest.raises(CacheMiss):
        cache.load(key)
    assert cache.entries(key) == []
    # A pending file left by a crash is hidden: not loaded, not counted.
    (cache.signature_dir(key) / ".pending-deadbeef.rgart").write_bytes(b"partial")
    assert cache.entries(key) == []
    assert publish(cache, key).code_object == PAYLOAD


def test_parallel_publication_enforces_the_signature_budget(tmp_path):
    cache = ArtifactCache(tmp_path, max_specializations=3)
    keys = [make_key(max_len) for max_len in range(10, 18)]

    def attempt(key):
        try:
            publish(cache, key)
            return "ok"
        except SpecializationLimit:
            return "limit"

    with ThreadPoolExecutor(8) as pool:
        results = list(pool.map(attempt, keys))
    assert results.count("ok") == 3 and results.count("limit") == 5
    assert len(cache.entries(keys[0])) == 3


def test_parallel_identical_publication_is_idempotent(tmp_path):
    cache, key = ArtifactCache(tmp_path), make_key()
    with ThreadPoolExecutor(8) as pool:
        artifacts = list(pool.map(lambda _: publish(cache, key), range(16)))
    assert {a.path for a in artifacts} == {cache.entry_path(key)}
    assert len(cache.entries(key)) == 1


def test_publication_copies_metadata_and_refuses_replacement(tmp_path):
    cache, key = ArtifactCache(tmp_path), make_key()
    metadata = {"kernel": "test_kernel", "grid": [1, 2]}
    artifact = publish(cache, key, metadata)
    metadata["grid"].append(3)
    assert cache.load(key).metadata == {"kernel": "test_kernel", "grid": [1, 2]} == artifact.metadata
    with pytest.raises(CacheMismatch, match="refusing to replace"):
        cache.publish(key, b"other payload", {"kernel": "test_kernel", "grid": [1, 2]})
    with pytest.raises(CacheMismatch, match="refusing to replace"):
        cache.publish(key, PAYLOAD, {"kernel": "other"})


def test_metadata_edit_on_disk_is_detected(tmp_path):
    """A changed schedule in the stored metadata cannot pass as the
    published one (its sha256 is in the header)."""
    cache, key = ArtifactCache(tmp_path), make_key()
    path = publish(cache, key, {"kernels": [{"name": "worker", "grid": [1, 1, 1]}]}).path
    header, payload = split(path.read_bytes())
    header["metadata"]["kernels"][0]["grid"] = [4096, 1, 1]
    path.write_bytes(join(header, payload))
    with pytest.raises(CacheMismatch, match="metadata"):
        cache.load(key)


@pytest.mark.parametrize("kwargs,message", [
    ({"library_sha256": "xyz"}, "library_sha256"),
    ({"build_info": "  "}, "build_info"),
])
def test_key_validation(kwargs, message):
    spec = ProgramSpec("sum", "f32", 4, "i64")
    arguments = {"library_sha256": "ab" * 32, "build_info": "b", **kwargs}
    with pytest.raises(ValidationError, match=message):
        CacheKey.from_spec(spec, **arguments)


def test_publication_input_validation(tmp_path):
    cache, key = ArtifactCache(tmp_path), make_key()
    with pytest.raises(ValidationError, match="nonempty bytes"):
        cache.publish(key, b"", {})
    with pytest.raises(ValidationError, match="finite JSON"):
        cache.publish(key, PAYLOAD, {"x": float("inf")})
    with pytest.raises(ValidationError, match="positive integer"):
        ArtifactCache(tmp_path, max_specializations=0)
    assert decode_artifact(publish(cache, key).path.read_bytes(), key)[0] == PAYLOAD


def test_compiler_hits_its_own_publication(tmp_path):
    """Compiling a spec twice publishes once and then hits (the artifact binds
    the spec to the built library's identity)."""
    from ragged import Compiler, native
    try:
        native.library()
    except Exception:  # noqa: BLE001 - library not built in this checkout
        pytest.skip("libragged_hip.so is not built")
    cache = ArtifactCache(tmp_path)
    first = Compiler().compile(ProgramSpec("max", "bf16", 8, "i32"), cache)
    second = Compiler().compile(ProgramSpec("max", "bf16", 8, "i32"), cache)
    assert not first.cache_hit and second.cache_hit
    assert second.naive is not None and second.naive.cache_hit
