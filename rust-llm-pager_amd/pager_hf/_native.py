"""Torch-side helpers over the ctypes binding: dtype codes, device/stream plumbing."""
from __future__ import annotations

import os
import sys

import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
import _pgr_native as nat  # noqa: E402,F401

DTYPE_CODES = {torch.float16: nat.DTYPE_F16, torch.bfloat16: nat.DTYPE_BF16}


def lib():
    return nat.load()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise NotImplementedError(
            f"the HIP decode-attention kernels take float16 or bfloat16 q/k/v, got {dtype}"
        ) from None


# torch's own accessor of the current raw stream (what torch.cuda.current_stream(d).cuda_stream
# returns, without building a Stream object: ~0.3 against ~1.9 us per call).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on `device`."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def require_cuda(*tensors: torch.Tensor) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("streaming attention expects CUDA (HIP) tensors")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError(f"tensors on different devices: {device} and {t.device}")
    return device
