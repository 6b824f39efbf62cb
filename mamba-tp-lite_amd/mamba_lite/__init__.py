"""MI355X-native Mamba mixer hot path with the mamba-tp-lite Python API.

    from mamba_lite.model import MambaConfig, MambaLM, MambaMixer, MambaCache
    from mamba_lite.cuda_graph import GraphedStepper
    from mamba_lite import ops, tp_utils

The compute runs in libmtl.so (hand-written gfx950 HIP kernels, C ABI in
include/mtl.h) and in torch's GEMMs; nothing here runs on the CPU.
"""
from .model import LayerCache, MambaBlock, MambaCache, MambaConfig, MambaLM, MambaMixer, RMSNorm  # noqa: F401

__all__ = ["MambaConfig", "LayerCache", "MambaCache", "RMSNorm", "MambaMixer", "MambaBlock", "MambaLM"]
