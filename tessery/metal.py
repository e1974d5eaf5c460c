"""The native bridge (src/metal_inference/metal.py): MetalRuntime and its buffers."""

from tessery_amd.runtime import SIGNATURES, Buffer, HipRuntime, MetalRuntime, pack_params

__all__ = ["Buffer", "HipRuntime", "MetalRuntime", "SIGNATURES", "pack_params"]
