"""Device-memory plumbing: torch tensors carry device pointers and streams.

torch is used only to allocate HBM and to name the current HIP stream; every
computation goes through libklearu_hip.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

_NP2T = {np.float32: torch.float32, np.int32: torch.int32, np.int64: torch.int64,
         np.uint16: torch.int16, np.uint32: torch.int32, np.int8: torch.int8}


def require_gpu() -> None:
    if not torch.cuda.is_available():
        raise RuntimeError("klearu_amd needs an MI355X (gfx950) GPU; none is visible")
    from . import _lib

    _lib.load()


def stream_ptr(stream=None) -> C.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return C.c_void_p(s.cuda_stream)


def ptr(t: torch.Tensor | None) -> C.c_void_p:
    if t is None:
        return C.c_void_p(0)
    if not t.is_cuda:
        raise ValueError("expected a device tensor")
    if not t.is_contiguous():
        raise ValueError("expected a contiguous tensor")
    return C.c_void_p(t.data_ptr())


def hptr(a: np.ndarray | None) -> C.c_void_p:
    if a is None:
        return C.c_void_p(0)
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("expected a C-contiguous host array")
    return C.c_void_p(a.ctypes.data)


def to_device(a, dtype=None) -> torch.Tensor:
    """numpy / list / tensor -> contiguous cuda tensor (uint16 / uint32 reinterpreted)."""
    if isinstance(a, torch.Tensor):
        t = a if a.is_cuda else a.cuda()
        return t.contiguous()
    arr = np.ascontiguousarray(a, dtype=dtype)
    if arr.dtype == np.uint16:
        return torch.from_numpy(arr.view(np.int16)).cuda()
    if arr.dtype == np.uint32:
        return torch.from_numpy(arr.view(np.int32)).cuda()
    return torch.from_numpy(arr).cuda()


def to_host_u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)
