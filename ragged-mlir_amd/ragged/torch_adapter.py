"""PyTorch custom ops and contiguous-NJT helpers over ``CompiledProgram``.

Same public surface as the reference's ``python/ragged/torch_adapter.py``
(:19-180): ``register_program``, ``register_torch_ops``, ``segment_reduce``,
``segment_softmax``, ``bind``, ``jagged_components``, ``njt_reduce`` and
``njt_softmax``, and the reference's two custom-op schemas exactly
(:57-58, :72-73):

    ragged_mlir::segment_reduce(Tensor values, Tensor offsets, str kind, str program,
                                str mode="validated") -> Tensor
    ragged_mlir::segment_softmax(Tensor values, Tensor offsets, str program,
                                 str mode="validated", Tensor? mask=None) -> Tensor

``program`` is the token ``register_program`` returns (the artifact digest).
The ops are opaque and forward-only; their fake implementations check shapes
and dtypes only, so they trace under ``torch.compile`` without reading
offsets. A caller that knows its longest segment (an NJT's cached
``max_seqlen``) passes it to the cost model through two further ops of this
build, with ``int max_len`` after ``program``:

    ragged_mlir::segment_reduce_bounded(Tensor values, Tensor offsets, str kind, str program,
                                        int max_len, str mode="validated") -> Tensor
    ragged_mlir::segment_softmax_bounded(Tensor values, Tensor offsets, str program, int max_len,
                                         str mode="validated", Tensor? mask=None) -> Tensor

The helpers below pick the bounded op whenever ``max_len`` is given.
Importing ``ragged`` does not import torch: call ``register_torch_ops()``
(the helpers do) to register.
"""
from __future__ import annotations

import threading
from typing import Any

from .errors import ValidationError
from .runtime import CompiledProgram, _torch

MODES = ("validated", "checked")

_lock = threading.RLock()
_registry: dict[str, CompiledProgram] = {}     # token -> program
_ops: dict[str, Any] = {}


def register_program(program: CompiledProgram) -> str:
    """Make ``program`` callable through the custom ops; returns its token.
    The ops return a new tensor, so an in-place specialisation is refused."""
    if program.spec.alias != "none":
        raise ValidationError("functional custom ops require an out-of-place specialization")
    token = program.artifact.key.digest
    with _lock:
        _registry[token] = program
    return token


def _mode(mode: str) -> str:
    if mode not in MODES:
        raise ValidationError("mode must be validated or checked")
    return mode


def _mask_matches(program_has_mask: bool, mask) -> None:
    if program_has_mask != (mask is not None):
        raise ValidationError("mask presence must match the compiled specialization")


def _program(token: str, op: str) -> CompiledProgram:
    with _lock:
        program = _registry.get(token)
    if program is None:
        raise ValidationError("compiled program token is not registered in this process")
    if program.spec.op != op:
        raise ValidationError("custom op does not match compiled program semantics")
    return program


def _run(values, offsets, token: str, op: str, mode: str, mask=None, max_len=None):
    _mode(mode)
    program = _program(token, op)
    _mask_matches(program.spec.mask, mask)
    rows = values.shape[0] if op == "softmax" else offsets.shape[0] - 1
    out = values.new_empty((rows, values.shape[1]))
    program.run(values, offsets, out, mode=mode, mask=mask, max_len=max_len)
    return out


def _check_shapes(values, offsets, torch) -> None:
    """What a fake (shape-only) call can check: ranks, dtypes, layout, device."""
    if values.ndim != 2 or offsets.ndim != 1:
        raise ValidationError("expected values[N,D] and offsets[B+1]")
    if values.dtype not in (torch.float32, torch.bfloat16):
        raise ValidationError("values must be f32 or bf16")
    if offsets.dtype not in (torch.int32, torch.int64):
        raise ValidationError("offsets must be i32 or i64")
    if not values.is_contiguous() or not offsets.is_contiguous():
        raise ValidationError("values and offsets must be contiguous")
    if values.device != offsets.device:
        raise ValidationError("values and offsets must use the same device")
    torch._check(offsets.shape[0] >= 1)
    torch._check(values.shape[1] >= 1)
    torch._check(values.shape[1] <= 1024)


def _check_mask_shape(values, mask, torch) -> None:
    if mask.ndim != 2 or mask.dtype != torch.float32:
        raise ValidationError("mask must be a rank-two f32 tensor")
    if not mask.is_contiguous() or mask.device != values.device:
        raise ValidationError("mask must be contiguous and use the values device")
    if mask.requires_grad:
        raise ValidationError("autograd is outside the supported forward-only mask contract")
    torch._check(mask.shape[0] == values.shape[0])
    torch._check(mask.shape[1] == values.shape[1])


def _reduce_kind(kind: str) -> str:
    if kind not in ("sum", "max"):
        raise ValidationError("segment_reduce kind must be sum or max")
    return kind


def _bound(max_len) -> int:
    if type(max_len) is not int or max_len < 0:
        raise ValidationError("max_len must be a nonnegative int")
    return max_len


def _reduce_fake(values, offsets, kind, mode, torch):
    _mode(mode)
    _reduce_kind(kind)
    _check_shapes(values, offsets, torch)
    return values.new_empty((offsets.shape[0] - 1, values.shape[1]))


def _softmax_fake(values, offsets, mode, mask, torch):
    _mode(mode)
    _check_shapes(values, offsets, torch)
    if mask is not None:
        _check_mask_shape(values, mask, torch)
    return values.new_empty(values.shape)


def register_torch_ops() -> dict[str, Any]:
    """Register both custom ops once per process; returns them by name."""
    with _lock:
        if _ops:
            return dict(_ops)
        torch = _torch()

        @torch.library.custom_op("ragged_mlir::segment_reduce", mutates_args=(),
                                 schema="(Tensor values, Tensor offsets, str kind, str program, "
                                        "str mode=\"validated\") -> Tensor")
        def segment_reduce_op(values, offsets, kind, program, mode="validated"):
            return _run(values, offsets, program, _reduce_kind(kind), mode)

        @segment_reduce_op.register_fake
        def _(values, offsets, kind, program, mode="validated"):
            return _reduce_fake(values, offsets, kind, mode, torch)

        @torch.library.custom_op("ragged_mlir::segment_softmax", mutates_args=(),
                                 schema="(Tensor values, Tensor offsets, str program, str mode=\"validated\", "
                                        "Tensor? mask=None) -> Tensor")
        def segment_softmax_op(values, offsets, program, mode="validated", mask=None):
            return _run(values, offsets, program, "softmax", mode, mask)

        @segment_softmax_op.register_fake
        def _(values, offsets, program, mode="validated", mask=None):
            return _softmax_fake(values, offsets, mode, mask, torch)

        @torch.library.custom_op("ragged_mlir::segment_reduce_bounded", mutates_args=(),
                                 schema="(Tensor values, Tensor offsets, str kind, str program, int max_len, "
                                        "str mode=\"validated\") -> Tensor")
        def segment_reduce_bounded_op(values, offsets, kind, program, max_len, mode="validated"):
            return _run(values, offsets, program, _reduce_kind(kind), mode, max_len=_bound(max_len))

        @segment_reduce_bounded_op.register_fake
        def _(values, offsets, kind, program, max_len, mode="validated"):
            _bound(max_len)
            return _reduce_fake(values, offsets, kind, mode, torch)

        @torch.library.custom_op("ragged_mlir::segment_softmax_bounded", mutates_args=(),
                                 schema="(Tensor values, Tensor offsets, str program, int max_len, "
                                        "str mode=\"validated\", Tensor? mask=None) -> Tensor")
        def segment_softmax_bounded_op(values, offsets, program, max_len, mode="validated", mask=None):
            return _run(values, offsets, program, "softmax", mode, mask, _bound(max_len))

        @segment_softmax_bounded_op.register_fake
        def _(values, offsets, program, max_len, mode="validated", mask=None):
            _bound(max_len)
            return _softmax_fake(values, offsets, mode, mask, torch)

        _ops["segment_reduce"] = segment_reduce_op
        _ops["segment_softmax"] = segment_softmax_op
        _ops["segment_reduce_bounded"] = segment_reduce_bounded_op
        _ops["segment_softmax_bounded"] = segment_softmax_bounded_op
        return dict(_ops)


def segment_reduce(values, offsets, kind: str, *, program: CompiledProgram, mode: str = "validated",
                   max_len: int | None = None):
    """``kind`` ("sum" / "max") of every segment through the custom op (the
    bounded one when ``max_len`` is given)."""
    ops = register_torch_ops()
    token = register_program(program)
    if max_len is None:
        return ops["segment_reduce"](values, offsets, kind, token, mode)
    return ops["segment_reduce_bounded"](values, offsets, kind, token, max_len, mode)


def segment_softmax(values, offsets, *, program: CompiledProgram, mode: str = "validated", mask=None,
                    max_len: int | None = None):
    """Softmax of every segment through the custom op (the bounded one when
    ``max_len`` is given)."""
    _mask_matches(program.spec.mask, mask)
    ops = register_torch_ops()
    token = register_program(program)
    if max_len is None:
        return ops["segment_softmax"](values, offsets, token, mode, mask)
    return ops["segment_softmax_bounded"](values, offsets, token, max_len, mode, mask)


def bind(program: CompiledProgram, *, mode: str = "validated"):
    """Register once and return a callable that only invokes the opaque
    custom op, so it can sit inside a ``torch.compile`` graph. Call ``bind``
    outside the compiled function: it mutates the registry."""
    _mode(mode)
    ops = register_torch_ops()
    token = register_program(program)
    if program.spec.op == "softmax":
        softmax, softmax_bounded = ops["segment_softmax"], ops["segment_softmax_bounded"]
        has_mask = program.spec.mask

        def run_softmax(values, offsets, mask=None, max_len=None):
            _mask_matches(has_mask, mask)
            if max_len is None:
                return softmax(values, offsets, token, mode, mask)
            return softmax_bounded(values, offsets, token, max_len, mode, mask)
        return run_softmax
    reduce_, reduce_bounded = ops["segment_reduce"], ops["segment_reduce_bounded"]
    kind = program.spec.op

    def run_reduce(values, offsets, max_len=None):
        if max_len is None:
            return reduce_(values, offsets, kind, token, mode)
        return reduce_bounded(values, offsets, kind, token, max_len, mode)
    return run_reduce


def jagged_components(nt):
    """``(values[N, D], offsets[B+1])`` of a contiguous ``torch.jagged``
    nested tensor of shape ``[B, jagged, D]`` (no holes, no explicit lengths)."""
    torch = _torch()
    if not getattr(nt, "is_nested", False) or nt.layout != torch.jagged:
        raise ValidationError("expected a torch.jagged nested tensor")
    if nt.dim() != 3:
        raise ValidationError("expected NJT shape [B, jagged, D]")
    if nt.lengths() is not None:
        raise ValidationError("NJT with explicit lengths/holes is outside the contiguous offsets contract")
    values, offsets = nt.values(), nt.offsets()
    if values.ndim != 2 or not values.is_contiguous() or not offsets.is_contiguous():
        raise ValidationError("NJT values[N,D] and offsets must be contiguous")
    if nt.shape[-1] != values.shape[-1]:
        raise ValidationError("only the first non-batch NJT dimension may be ragged")
    return values, offsets


def _cached_max_seqlen(nt) -> int | None:
    """The NJT's cached longest segment, if it holds one (never computed
    here: that would read the offsets back to the host)."""
    cached = getattr(nt, "_maybe_max_seqlen", None)
    if cached is None:
        return None
    try:
        return int(cached)
    except (TypeError, ValueError, RuntimeError):
        return None


def njt_reduce(nt, kind: str, *, program: CompiledProgram, mode: str = "validated"):
    """``kind`` of every row run of an NJT: a dense ``[B, D]`` tensor."""
    values, offsets = jagged_components(nt)
    return segment_reduce(values, offsets, kind, program=program, mode=mode, max_len=_cached_max_seqlen(nt))


def njt_softmax(nt, *, program: CompiledProgram, mode: str = "validated", mask=None):
    """Softmax over each NJT component, as an NJT with the same offsets."""
    torch = _torch()
    values, offsets = jagged_components(nt)
    out = segment_softmax(values, offsets, program=program, mode=mode, mask=mask, max_len=_cached_max_seqlen(nt))
    return torch.nested.nested_tensor_from_jagged(out, offsets=offsets)
