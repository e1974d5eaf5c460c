"""The Qwen3 embedding backend (src/metal_inference/qwen3.py)."""

from tessery_amd.backends import Qwen3Backend

__all__ = ["Qwen3Backend"]
