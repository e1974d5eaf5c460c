"""Stable error types of the drop-in boundary.

Same class names, codes and base class as tessery's errors (src/metal_inference/errors.py:1-59;
re-exported by src/tessery/errors.py:1-33), so callers that catch them keep working. Messages
carry only the stable code, never payloads. HipUnavailableError is the HIP-side reason for the
reference's MetalUnavailableError and subclasses it.
"""


class EmbeddingError(Exception):
    code = "embedding_error"
    http_status = 500

    def __init__(self) -> None:
        super().__init__(self.code)


class ConfigurationError(EmbeddingError):
    code = "configuration_error"


class InvalidInputError(EmbeddingError):
    code = "invalid_input"
    http_status = 400


class ManifestError(EmbeddingError):
    code = "invalid_manifest"


class UnsupportedProfileError(EmbeddingError):
    code = "unsupported_profile"


class OverloadError(EmbeddingError):
    code = "overloaded"
    http_status = 429


class CanceledError(EmbeddingError):
    code = "canceled"


class DeadlineExceededError(EmbeddingError):
    code = "deadline_exceeded"


class InferenceError(EmbeddingError):
    code = "inference_failed"


class ClosedError(EmbeddingError):
    code = "closed"


class PrerequisiteError(EmbeddingError):
    code = "baseline_required"


class MetalUnavailableError(EmbeddingError):
    code = "metal_unavailable"


class HipUnavailableError(MetalUnavailableError):
    """No gfx950 device is visible to the HIP runtime."""

    code = "hip_unavailable"


class NativeBuildError(EmbeddingError):
    code = "native_engine_not_built"


__all__ = [
    "EmbeddingError",
    "ConfigurationError",
    "InvalidInputError",
    "ManifestError",
    "UnsupportedProfileError",
    "OverloadError",
    "CanceledError",
    "DeadlineExceededError",
    "InferenceError",
    "ClosedError",
    "PrerequisiteError",
    "MetalUnavailableError",
    "HipUnavailableError",
    "NativeBuildError",
]
