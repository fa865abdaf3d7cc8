"""Torch-side plumbing for the HIP ops: device checks, dtype codes, streams,
status words.  torch only provides device memory and the current stream."""
from __future__ import annotations

import torch

from . import _lib
from .errors import IntegrityError

DTYPE_CODE = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16, torch.float32: _lib.DTYPE_F32}


def dtype_code(dt):
    if dt not in DTYPE_CODE:
        raise IntegrityError(f"unsupported dtype {dt}")
    return DTYPE_CODE[dt]


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise IntegrityError("NSN HIP ops require GPU tensors; there is no CPU fallback")


def stream():
    """The current stream of the current device as a raw hipStream_t (an int).
    torch's raw accessor costs ~1 µs; ``torch.cuda.current_stream()`` builds a
    Stream object and resolves the device index (~11 µs per call)."""
    return torch._C._cuda_getCurrentRawStream(torch.cuda.current_device())


def ptr(t):
    return None if t is None else t.data_ptr()


def new_status(device):
    return torch.zeros(1, dtype=torch.int32, device=device)


def read_status(status):
    """Synchronising read of a device status word."""
    return int(status.item())


def norm_order(x):
    """Order of torch-CPU's vector_norm on ``x.float()`` (see include/nsn_hip.h).

    ``x.float()`` keeps ``x``'s strides when ``x`` is non-overlapping and
    dense (and is ``x`` itself for fp32); its last-dim stride decides between
    the 8-lane contiguous reduction and the sequential one.
    """
    if x.dtype == torch.float32:
        st = x.stride(-1)
    else:
        st = torch.empty_like(x, dtype=torch.float32, device="meta").stride(-1)
    return _lib.NORM_LANES8 if (st == 1 or x.shape[-1] == 1) else _lib.NORM_SEQUENTIAL
