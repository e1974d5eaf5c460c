"""tessery's public names for the parts this package provides (src/tessery/__init__.py:1-42).

A caller of tessery's prefill-attention path imports from here as it would from tessery:
`from tessery import MetalRuntime`, `from tessery.metal import MetalRuntime`, ... The names are
the MI355X implementation in `tessery_amd` (HIP kernels behind the C ABI of
include/tessery_hip.h). The rest of tessery's public API (EmbeddingModel, DocumentIndex,
retrieval, tokenizers, the HTTP service) is outside this package and is not exported.
"""

from tessery_amd import HipRuntime, MetalRuntime, __version__
from tessery_amd.packs import ModelProfile
from tessery_amd.weights import Artifact

from . import batching, bert, errors, metal, qwen3, weights  # noqa: F401

__all__ = ["Artifact", "HipRuntime", "MetalRuntime", "ModelProfile"]
