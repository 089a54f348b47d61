"""CPU parity oracle for the Soft-DTW hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import this package, and only as the checker / the timed CPU baseline.  The shipped
package (``sdtw-cuda-torch_amd/softdtw_cuda``) never imports it and has no CPU fallback.
"""
from .oracle import (  # noqa: F401
    load_library,
    sqeuclidean,
    forward,
    backward,
    OracleSoftDTWFunction,
    softdtw,
    barycenter,
)
