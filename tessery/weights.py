"""Verified weight artifacts and the SafeTensors reader (src/metal_inference/weights.py)."""

from tessery_amd.weights import Artifact, SafeTensors, read_artifact, read_json

__all__ = ["Artifact", "SafeTensors", "read_artifact", "read_json"]
