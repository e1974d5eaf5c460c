"""The BERT / BGE embedding backend (src/metal_inference/bert.py)."""

from tessery_amd.backends import BertBackend

__all__ = ["BertBackend"]
