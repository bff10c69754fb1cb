"""CPU tests of the PyTorch custom ops and NJT helpers: registration, the
shape-only fake implementations (meta tensors), graph capture and the NJT
contract. No kernel runs here (reference test/python/test_torch_adapter.py)."""
from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")

from ragged import Compiler, ProgramSpec, ValidationError  # noqa: E402
from ragged.torch_adapter import (jagged_components, register_program, register_torch_ops,  # noqa: E402
                                  segment_softmax)


@pytest.fixture(scope="module")
def ops():
    return register_torch_ops()


def meta(shape, dtype=torch.float32):
    return torch.empty(shape, dtype=dtype, device="meta")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("offsets_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("kind", ["sum", "max"])
def test_reduce_fake_shape(ops, dtype, offsets_dtype, kind):
    out = ops["segment_reduce"](meta((17, 13), dtype), meta((5,), offsets_dtype), kind, "no-program")
    assert out.shape == (4, 13) and out.dtype == dtype and out.device.type == "meta"


def test_softmax_fake_shape_and_idempotent_registration(ops):
    out = ops["segment_softmax"](meta((0, 1024), torch.bfloat16), meta((1,), torch.int64), "no-program")
    assert out.shape == (0, 1024)
    assert register_torch_ops() == ops
    masked = ops["segment_softmax"](meta((9, 4)), meta((3,), torch.int64), "no-program", "checked", meta((9, 4)))
    assert masked.shape == (9, 4)


def test_fake_rejections(ops):
    with pytest.raises(ValidationError, match="kind"):
        ops["segment_reduce"](meta((3, 4)), meta((3,), torch.int64), "mean", "token")
    with pytest.raises(ValidationError, match="mode"):
        ops["segment_reduce"](meta((3, 4)), meta((3,), torch.int64), "sum", "token", "fast")
    with pytest.raises(ValidationError, match="f32 or bf16"):
        ops["segment_reduce"](meta((3, 4), torch.float16), meta((3,), torch.int64), "sum", "token")
    with pytest.raises(ValidationError, match="i32 or i64"):
        ops["segment_reduce"](meta((3, 4)), meta((3,), torch.int16), "sum", "token")
    with pytest.raises(ValidationError, match="values\\[N,D\\]"):
        ops["segment_reduce"](meta((3,)), meta((3,), torch.int64), "sum", "token")
    with pytest.raises(ValidationError, match="mask must be a rank-two f32"):
        ops["segment_softmax"](meta((3, 4)), meta((3,), torch.int64), "token", "validated", meta((3, 4), torch.bfloat16))


def test_fullgraph_capture_of_the_opaque_op(ops):
    graphs = []

    def backend(graph, example_inputs):
        graphs.append(graph)
        return graph.forward

    def f(values, offsets):
        return torch.ops.ragged_mlir.segment_reduce(values, offsets, "sum", "no-program")

    compiled = torch.compile(f, backend=backend, fullgraph=True)
    assert compiled(meta((17, 13)), meta((5,), torch.int64)).shape == (4, 13)
    assert len(graphs) == 1
    assert any(node.op == "call_function" and "ragged_mlir.segment_reduce" in str(node.target)
               for node in graphs[0].graph.nodes)


def test_unregistered_token_and_wrong_op(ops, artifact_cache):
    values, offsets = torch.zeros((4, 2)), torch.tensor([0, 4])
    with pytest.raises(ValidationError, match="not registered"):
        ops["segment_reduce"](values, offsets, "sum", "no-such-token")
    softmax = Compiler().compile(ProgramSpec("softmax", "f32", 2, "i64"), artifact_cache)
    token = register_program(softmax)
    with pytest.raises(ValidationError, match="semantics"):
        ops["segment_reduce"](values, offsets, "sum", token)


def test_inplace_and_mask_mismatch_refused(artifact_cache):
    inplace = Compiler().compile(ProgramSpec("softmax", "f32", 2, "i64", alias="inplace"), artifact_cache)
    with pytest.raises(ValidationError, match="out-of-place"):
        register_program(inplace)
    plain = Compiler().compile(ProgramSpec("softmax", "f32", 2, "i64"), artifact_cache)
    with pytest.raises(ValidationError, match="mask presence"):
        segment_softmax(torch.zeros((4, 2)), torch.tensor([0, 4]), program=plain, mask=torch.zeros((4, 2)))


def test_njt_components_are_zero_copy():
    values = torch.randn(6, 4)
    offsets = torch.tensor([0, 2, 2, 6])
    nt = torch.nested.nested_tensor_from_jagged(values, offsets=offsets)
    got_values, got_offsets = jagged_components(nt)
    assert got_values.data_ptr() == values.data_ptr() and got_offsets.data_ptr() == offsets.data_ptr()


def test_njt_contract_rejections():
    with pytest.raises(ValidationError, match="jagged"):
        jagged_components(torch.zeros((2, 3, 4)))
    values = torch.randn(6, 4)
    holes = torch.nested.nested_tensor_from_jagged(values, offsets=torch.tensor([0, 2, 4, 6]),
                                                   lengths=torch.tensor([1, 2, 2]))
    with pytest.raises(ValidationError, match="holes"):
        jagged_components(holes)
    with pytest.raises(ValidationError, match="\\[B, jagged, D\\]"):
        jagged_components(torch.nested.nested_tensor_from_jagged(torch.randn(6), offsets=torch.tensor([0, 2, 6])))


def test_reference_schemas_are_exact(ops):
    """The reference's two schemas (torch_adapter.py:57-58, 72-73) unchanged;
    max_len travels through the bounded ops of this build."""
    assert str(ops["segment_reduce"]._opoverload._schema) == (
        'ragged_mlir::segment_reduce(Tensor values, Tensor offsets, str kind, str program, '
        'str mode="validated") -> Tensor')
    assert str(ops["segment_softmax"]._opoverload._schema) == (
        'ragged_mlir::segment_softmax(Tensor values, Tensor offsets, str program, str mode="validated", '
        'Tensor? mask=None) -> Tensor')
    out = ops["segment_reduce_bounded"](meta((17, 13)), meta((5,), torch.int64), "sum", "no-program", 9)
    assert out.shape == (4, 13)
    out = ops["segment_softmax_bounded"](meta((9, 4)), meta((3,), torch.int64), "no-program", 9, "checked",
                                         meta((9, 4)))
    assert out.shape == (9, 4)
    with pytest.raises(ValidationError, match="max_len"):
        ops["segment_reduce_bounded"](meta((17, 13)), meta((5,), torch.int64), "sum", "no-program", -1)
