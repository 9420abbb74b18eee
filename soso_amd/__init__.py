"""soso_amd -- MI355X-native (gfx950) decode hot path of soso-llm-core.

Hand-written HIP kernels and a C ABI (include/soso_hip.h) behind soso's
GpuDispatch boundary.  `soso_amd.dispatch.HipGpu` is a Python view of that ABI
for tests, benchmarks and Python callers.
"""
from . import abi  # noqa: F401

__all__ = ["abi"]
