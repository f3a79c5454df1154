"""vireo_amd: MI355X (gfx950) HIP kernels for vireo's quantized MoE-FFN path.

The product is the C-ABI shared library libvireo_hip.so (include/*.h); this
package builds it (vireo_amd.build), binds it (vireo_amd._lib), describes the
benchmark workloads (vireo_amd.workloads) and mirrors the reference's MoE
interface on top of it (vireo_amd.moe).
"""
from ._lib import VireoError, load  # noqa: F401

__all__ = ["load", "VireoError"]
