"""Error taxonomy of the public API (reference: python/ragged/errors.py:4-41).

Invalid programs and tensors, corrupt artifacts, missing tools and a missing
device/library are distinct types, with the same names and bases as the
reference so callers' ``except`` clauses keep working.
"""


class RaggedError(RuntimeError):
    pass


class ValidationError(RaggedError, ValueError):
    """Bad spec, tensor or argument, raised before any allocation or launch.
    ``condition``/``index``/``errors`` carry checked-mode offsets failures."""

    def __init__(self, message, *, condition=None, index=None, errors=None):
        super().__init__(message)
        self.condition = condition
        self.index = index
        self.errors = dict(errors or {})


class CacheError(RaggedError):
    pass


class CacheMiss(CacheError):
    pass


class CacheMismatch(CacheError):
    pass


class SpecializationLimit(CacheError):
    pass


class ToolchainUnavailable(RaggedError):
    pass


class CompilationError(RaggedError):
    pass


class RuntimeUnavailable(RaggedError):
    """No GPU, the wrong architecture, CPU tensors or a missing HIP library."""
