"""Stable error types of the drop-in boundary.

The classes raised by this path keep the class names, `code` strings and base class of tessery's
errors (src/metal_inference/errors.py:1-59, re-exported by src/tessery/errors.py:1-33), so a
caller that catches them keeps working. Messages carry only the stable code, never payloads.
HipUnavailableError is the HIP-side reason for the reference's MetalUnavailableError and
subclasses it. Only the classes something in this package raises are defined here; the
reference's API/HTTP-layer classes (overload, deadline, cancellation, ...) belong to its service
layer, which this package does not include.
"""


class EmbeddingError(Exception):
    code = "embedding_error"
    http_status = 500

    def __init__(self) -> None:
        super().__init__(self.code)


class ManifestError(EmbeddingError):
    """A weight pack or its metadata failed verification (weights.py, backends.py)."""

    code = "invalid_manifest"


class UnsupportedProfileError(EmbeddingError):
    """A model config outside the shapes a backend serves."""

    code = "unsupported_profile"


class InferenceError(EmbeddingError):
    """A native call failed or the runtime was used outside its contract."""

    code = "inference_failed"


class ClosedError(EmbeddingError):
    """The runtime or backend was already closed."""

    code = "closed"


class MetalUnavailableError(EmbeddingError):
    code = "metal_unavailable"


class HipUnavailableError(MetalUnavailableError):
    """No gfx950 device is visible to the HIP runtime."""

    code = "hip_unavailable"


class NativeBuildError(EmbeddingError):
    """libtessery_hip.so is missing, unreadable or built for another ABI version."""

    code = "native_engine_not_built"


__all__ = [
    "EmbeddingError",
    "ManifestError",
    "UnsupportedProfileError",
    "InferenceError",
    "ClosedError",
    "MetalUnavailableError",
    "HipUnavailableError",
    "NativeBuildError",
]
