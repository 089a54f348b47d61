"""MI355X (gfx950) Soft-DTW engine with the public API of BGU-CS-VIL/sdtw-cuda-torch.

    from softdtw_cuda import SoftDTW, softdtw, softdtw_barycenter, softdtw_barycenter_cpu

Same names, arguments, defaults and error messages as the reference package
(softdtw_cuda/__init__.py:1-5).  All numerics run in hand-written HIP kernels
(libsdtw_hip.so, C ABI in include/sdtw.h); CPU tensors are staged through the GPU.
"""
from .functional import softdtw
from .module import SoftDTW
from .barycenters import softdtw_barycenter, softdtw_barycenter_cpu
from ._engine import get_numerics, set_numerics

__all__ = ["softdtw", "SoftDTW", "softdtw_barycenter", "softdtw_barycenter_cpu",
           "set_numerics", "get_numerics"]
