"""GPU tests of the custom ops, ``bind`` (inside ``torch.compile``) and the
NJT helpers: the same exact results as ``program.run`` against the oracle."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from gpu_helpers import check, quantized

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU containers
    pytest.skip("no ROCm device", allow_module_level=True)

from ragged import Compiler, ProgramSpec, ValidationError  # noqa: E402
from ragged import torch_adapter as ta  # noqa: E402
from ragged.workloads import make_lengths, offsets_from_lengths  # noqa: E402

DEVICE = torch.device("cuda", 0)
_programs = {}


def program(cache, op, dtype, d, offsets_dtype="i64", **kwargs):
    key = (op, dtype, d, offsets_dtype, tuple(sorted(kwargs.items())))
    if key not in _programs:
        _programs[key] = Compiler().compile(ProgramSpec(op, dtype, d, offsets_dtype, **kwargs), cache)
    return _programs[key]


def inputs(d, dtype, offsets_dtype="i64", seed=3, segments=257):
    lengths = make_lengths("long_tail", segments, seed=seed, total_elements=max(3000, 300_000 // d))
    lengths[::11] = 0
    offsets = offsets_from_lengths(lengths, offsets_dtype)
    values = np.random.default_rng(seed + 1).normal(size=(int(offsets[-1]), d)).astype(np.float32)
    tdtype = torch.bfloat16 if dtype == "bf16" else torch.float32
    x = torch.from_numpy(values).to(DEVICE).to(tdtype).contiguous()
    off = torch.from_numpy(offsets).to(DEVICE)
    return values, offsets, x, off


def host(t):
    return t.float().cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("op,dtype,d", [("sum", "f32", 1), ("max", "bf16", 128), ("sum", "bf16", 32),
                                        ("max", "f32", 3)])
def test_segment_reduce_op(artifact_cache, op, dtype, d):
    prog = program(artifact_cache, op, dtype, d)
    values, offsets, x, off = inputs(d, dtype)
    for mode in ("validated", "checked"):
        out = ta.segment_reduce(x, off, op, program=prog, mode=mode, max_len=int(np.diff(offsets).max()))
        torch.cuda.synchronize()
        assert out.shape == (len(offsets) - 1, d) and out.dtype == x.dtype
        check(host(out), values, offsets, op=op, dtype=dtype)


@pytest.mark.parametrize("dtype,d", [("bf16", 128), ("f32", 1), ("f32", 64)])
def test_segment_softmax_op(artifact_cache, dtype, d):
    prog = program(artifact_cache, "softmax", dtype, d)
    values, offsets, x, off = inputs(d, dtype)
    out = ta.segment_softmax(x, off, program=prog)
    torch.cuda.synchronize()
    check(host(out), values, offsets, op="softmax", dtype=dtype)


def test_masked_softmax_op(artifact_cache):
    d = 16
    prog = program(artifact_cache, "softmax", "f32", d, mask=True, scale=0.5)
    values, offsets, x, off = inputs(d, "f32")
    mask = np.random.default_rng(8).normal(size=values.shape).astype(np.float32)
    mask[::5, 3] = -np.inf
    out = ta.segment_softmax(x, off, program=prog, mask=torch.from_numpy(mask).to(DEVICE))
    torch.cuda.synchronize()
    check(host(out), values, offsets, op="softmax", dtype="f32", mask=mask, scale=0.5)


def test_checked_mode_rejects_through_the_op(artifact_cache):
    prog = program(artifact_cache, "sum", "f32", 4)
    x = torch.zeros((8, 4), device=DEVICE)
    off = torch.tensor([0, 5, 3, 8], device=DEVICE)
    with pytest.raises(ValidationError) as caught:
        ta.segment_reduce(x, off, "sum", program=prog, mode="checked")
    assert caught.value.errors == oracle.offsets_errors([0, 5, 3, 8], 8)


@pytest.mark.parametrize("op", ["sum", "softmax"])
def test_bind_inside_torch_compile(artifact_cache, op):
    """``bind`` outside, the opaque op inside a full graph; eager backend so
    the test measures the capture, not a code generator."""
    d = 8
    prog = program(artifact_cache, op, "f32", d)
    call = ta.bind(prog)
    values, offsets, x, off = inputs(d, "f32", seed=21)

    def f(v, o):
        return call(v * 2.0, o)

    compiled = torch.compile(f, backend="eager", fullgraph=True)
    out = compiled(x, off)
    torch.cuda.synchronize()
    check(host(out), values * 2.0, offsets, op=op, dtype="f32")


@pytest.mark.parametrize("kind", ["sum", "max"])
def test_njt_reduce(artifact_cache, kind):
    d = 32
    prog = program(artifact_cache, kind, "bf16", d)
    values, offsets, x, off = inputs(d, "bf16", seed=31)
    longest = int(np.diff(offsets).max())
    nt = torch.nested.nested_tensor_from_jagged(x, offsets=off, max_seqlen=longest)
    out = ta.njt_reduce(nt, kind, program=prog)
    torch.cuda.synchronize()
    check(host(out), values, offsets, op=kind, dtype="bf16")


def test_njt_softmax(artifact_cache):
    d = 128
    prog = program(artifact_cache, "softmax", "bf16", d)
    values, offsets, x, off = inputs(d, "bf16", seed=41)
    nt = torch.nested.nested_tensor_from_jagged(x, offsets=off)
    out = ta.njt_softmax(nt, program=prog)
    torch.cuda.synchronize()
    assert out.is_nested and out.offsets().data_ptr() == off.data_ptr()
    check(host(out.values()), values, offsets, op="softmax", dtype="bf16")
