"""tessery_amd: tessery's prefill-attention path, native on AMD Instinct MI355X (gfx950).

Drop-in surface (the names tessery's callers use):
    MetalRuntime / HipRuntime   native bridge with _attention, _linear4, _dispatch, command, read
    length_batches, execution_batches   bucket / execution-width plan
    errors                      tessery's stable error classes

Importing this package loads nothing native; HipRuntime() opens libtessery_hip.so.
"""

from . import errors
from .batching import execution_batches, length_batches
from .errors import (
    ClosedError,
    EmbeddingError,
    HipUnavailableError,
    InferenceError,
    MetalUnavailableError,
    NativeBuildError,
)
from .runtime import Buffer, HipRuntime, MetalRuntime, library_path

__version__ = "0.1.0"

__all__ = [
    "Buffer",
    "ClosedError",
    "EmbeddingError",
    "HipRuntime",
    "HipUnavailableError",
    "InferenceError",
    "MetalRuntime",
    "MetalUnavailableError",
    "NativeBuildError",
    "errors",
    "execution_batches",
    "length_batches",
    "library_path",
]
