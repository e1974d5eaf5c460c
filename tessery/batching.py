"""Length bucketing and execution widths (src/metal_inference/batching.py)."""

from tessery_amd.batching import execution_batches, length_batches

__all__ = ["execution_batches", "length_batches"]
