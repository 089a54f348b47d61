"""Where the engine computes, and how tensors get there.

The engine has one implementation: HIP kernels on a ROCm GPU.  GPU tensors are used in
place; CPU tensors are staged to the current GPU and results are returned on the caller's
device (autograd follows the copies).  Without a visible GPU this raises: there is no CPU
implementation behind the API.  float64 inputs run the float64 kernels (double
throughout, as the reference computes them); float32 the float32 engine; float16 and
bfloat16 are converted to float32 on entry.  Results are returned in the caller's dtype.
"""
from __future__ import annotations

import torch


def compute_device(t: torch.Tensor) -> torch.device:
    if t.is_cuda:
        return t.device
    if not torch.cuda.is_available():
        raise RuntimeError(
            "softdtw_cuda: this engine computes on a ROCm GPU (MI355X/gfx950) and no GPU is "
            "visible; CPU tensors are staged through the GPU, so they cannot be processed here."
        )
    return torch.device("cuda", torch.cuda.current_device())


def engine_dtype(*ts: torch.Tensor) -> torch.dtype:
    """float64 if any operand is float64 (torch's type promotion), else float32."""
    return torch.float64 if any(t.dtype == torch.float64 for t in ts) else torch.float32


def to_engine(t: torch.Tensor, device: torch.device, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """`dtype` (float32 or float64), contiguous, on `device` (a no-op view when already so)."""
    return t.to(device=device, dtype=dtype).contiguous()
