"""Device-memory plumbing: torch tensors on the HIP device, their raw
pointers and the current stream, for the ctypes calls into libbfp.so."""
from __future__ import annotations

import numpy as np

_DTYPES = {}


def _torch():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("the BFP datapath needs a HIP GPU (torch.cuda.is_available() is False);"
                           " there is no CPU fallback")
    if not _DTYPES:
        _DTYPES.update(int16=torch.int16, int8=torch.int8, int32=torch.int32,
                       int64=torch.int64, float32=torch.float32, float64=torch.float64,
                       uint8=torch.uint8)
    return torch


def to_dev(a: np.ndarray):
    torch = _torch()
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def empty(n, dtype: str):
    torch = _torch()
    return torch.empty(int(n), dtype=_DTYPES[dtype], device="cuda")


def zeros(n, dtype: str):
    torch = _torch()
    return torch.zeros(int(n), dtype=_DTYPES[dtype], device="cuda")


def ptr(t) -> int:
    return t.data_ptr()


def stream():
    return _torch().cuda.current_stream().cuda_stream


def to_host(t) -> np.ndarray:
    return t.cpu().numpy()


def sync():
    _torch().cuda.synchronize()
