"""ragged on MI355X: segmented sum, max and softmax over packed [N, D] values.

Drop-in for the reference's Python surface (simon-jd/ragged-mlir
python/ragged/__init__.py): ``ProgramSpec``, ``Compiler``/``ArtifactCache`` and
``CompiledProgram.run(values, offsets, out, max_len=...)`` on PyTorch-ROCm
tensors and the current HIP stream, executed by hand-written gfx950 kernels
in ``libragged_hip.so`` (C ABI: include/ragged_hip.h). Torch and the native
library load lazily; nothing here falls back to the CPU.
"""
from .cache import Artifact, ArtifactCache, CacheKey
from .compiler import CompilationResult, Compiler
from .errors import (CacheError, CacheMismatch, CacheMiss, CompilationError, RaggedError, RuntimeUnavailable,
                     SpecializationLimit, ToolchainUnavailable, ValidationError)
from .model import DIALECT_VERSION, ExecutionReport, Hints, Optimizations, ProgramSpec
from .runtime import CompiledProgram

__all__ = ["Artifact", "ArtifactCache", "CacheKey", "CompilationResult", "Compiler", "CompiledProgram", "DIALECT_VERSION",
           "ExecutionReport", "Hints", "Optimizations", "ProgramSpec", "RaggedError", "ValidationError",
           "CacheError", "CacheMismatch", "CacheMiss", "CompilationError", "RuntimeUnavailable",
           "SpecializationLimit", "ToolchainUnavailable"]

__version__ = "0.1.0"
