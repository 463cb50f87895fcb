"""Host plumbing: move NumPy / torch inputs to the GPU and results back.

The reference ops take NumPy arrays (float32, or ml_dtypes.bfloat16) and
return NumPy arrays synchronously.  Here the same calls also accept torch
tensors: CPU tensors come back as CPU tensors, GPU tensors stay on the GPU and
the call is asynchronous on torch's current HIP stream.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib

try:  # bfloat16 NumPy arrays exist only when ml_dtypes is installed
    import ml_dtypes

    NP_BF16 = np.dtype(ml_dtypes.bfloat16)
except ImportError:  # pragma: no cover - depends on the environment
    NP_BF16 = None

NUMPY, TORCH_CPU, TORCH_GPU = "numpy", "torch_cpu", "torch_gpu"


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("nkilab runs its kernels on a ROCm GPU and none is visible (torch.cuda.is_available() is False)")
    return torch.device("cuda", torch.cuda.current_device())


def dtype_code(dt: torch.dtype) -> int:
    """The C ABI's dtype code (float16 is an operand format of the GEMM, the
    RMSNorm output, the gate/up SwiGLU GEMM and the flash attention only)."""
    if dt == torch.float32:
        return _lib.F32
    if dt == torch.bfloat16:
        return _lib.BF16
    if dt == torch.float16:
        return _lib.F16
    raise TypeError(f"unsupported dtype {dt}: float32, bfloat16 or float16 expected")


def to_device(x) -> tuple[torch.Tensor, str]:
    """Return (GPU tensor, kind of the input)."""
    if isinstance(x, torch.Tensor):
        dtype_code(x.dtype)
        if x.is_cuda:
            return x, TORCH_GPU
        return x.to(device()), TORCH_CPU
    arr = np.asarray(x)
    if arr.dtype == np.float32:
        t = torch.from_numpy(np.ascontiguousarray(arr))
    elif NP_BF16 is not None and arr.dtype == NP_BF16:
        t = torch.from_numpy(np.ascontiguousarray(arr).view(np.int16)).view(torch.bfloat16)
    else:
        raise TypeError(f"unsupported dtype {arr.dtype}: float32 or bfloat16 expected")
    return t.to(device()), NUMPY


def from_device(t: torch.Tensor, kind: str):
    """Convert a GPU result back to the kind of the caller's input."""
    if kind == TORCH_GPU:
        return t
    if kind == TORCH_CPU:
        return t.cpu()
    if t.dtype == torch.bfloat16:
        if NP_BF16 is None:
            raise TypeError("a bfloat16 result cannot be returned as NumPy without ml_dtypes")
        return t.cpu().view(torch.int16).numpy().view(NP_BF16)
    return t.cpu().numpy()


def stream_handle() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)
