"""klearu-accel entry points on device tensors.

Mirrors crates/klearu-accel/src/simd/mod.rs:19-109 (dense_dot_dense_simd,
sparse_dot_dense_simd, scatter_add_simd) and bf16/mod.rs:22-134 (Bf16Weights,
Bf16FullMode).  Results are bit-identical to the reference's x86_64 AVX2 path.
"""
from __future__ import annotations

import numpy as np
import torch

from . import _lib
from ._dev import ptr, stream_ptr, to_device


def _chk(cond, msg):
    if not cond:
        raise ValueError(msg)


def dense_dot_dense_simd(a, b, stream=None) -> torch.Tensor:
    """dot(a, b); a may be [rows, n] for a batch of row dots against b [n]."""
    a, b = to_device(a, np.float32), to_device(b, np.float32)
    _chk(a.shape[-1] == b.numel(), "dense_dot_dense: length mismatch")
    rows = 1 if a.dim() == 1 else a.shape[0]
    out = torch.empty(rows, dtype=torch.float32, device=a.device)
    _lib.call("kh_dense_dot_dense", ptr(a), rows, b.numel(), ptr(b), b.numel(), ptr(out),
              stream_ptr(stream))
    return out[0] if a.dim() == 1 else out


def sparse_dot_dense_simd(indices, values, dense, stream=None) -> torch.Tensor:
    idx, val, d = to_device(indices, np.uint32), to_device(values, np.float32), to_device(dense, np.float32)
    _chk(idx.numel() == val.numel(), "sparse_dot_dense: indices/values length mismatch")
    out = torch.empty(1, dtype=torch.float32, device=d.device)
    _lib.call("kh_sparse_dot_dense", ptr(idx), ptr(val), idx.numel(), ptr(d), d.numel(), ptr(out),
              stream_ptr(stream))
    return out[0]


def scatter_add_simd(indices, values, dense: torch.Tensor, scale: float, stream=None) -> torch.Tensor:
    """In place: dense[indices[i]] += values[i] * scale (duplicates in order)."""
    idx, val = to_device(indices, np.uint32), to_device(values, np.float32)
    _chk(idx.numel() == val.numel(), "scatter_add: indices/values length mismatch")
    _lib.call("kh_scatter_add", ptr(idx), ptr(val), idx.numel(), ptr(dense), dense.numel(), float(scale),
              stream_ptr(stream))
    return dense


def exp_f32(x, stream=None) -> torch.Tensor:
    """f32::exp of every element, bit-identical to glibc expf (the exponential
    of every sigmoid, SiLU and softmax kernel in this library)."""
    x = to_device(x, np.float32).contiguous()
    y = torch.empty_like(x)
    _lib.call("kh_expf", ptr(x), ptr(y), x.numel(), stream_ptr(stream))
    return y


class Bf16Weights:
    """BF16 storage with f32 arithmetic (bf16/mod.rs:22-107); data is int16 bits on device."""

    def __init__(self, data: torch.Tensor):
        self.data = data

    @classmethod
    def from_f32(cls, x, stream=None):
        x = to_device(x, np.float32)
        out = torch.empty(x.numel(), dtype=torch.int16, device=x.device)
        _lib.call("kh_bf16_from_f32", ptr(x), ptr(out), x.numel(), stream_ptr(stream))
        return cls(out)

    def to_f32(self, stream=None) -> torch.Tensor:
        out = torch.empty(self.data.numel(), dtype=torch.float32, device=self.data.device)
        _lib.call("kh_bf16_to_f32", ptr(self.data), ptr(out), self.data.numel(), stream_ptr(stream))
        return out

    def __len__(self):
        return self.data.numel()

    def dot_f32(self, other, stream=None) -> torch.Tensor:
        x = to_device(other, np.float32)
        _chk(x.numel() == len(self), f"Bf16Weights::dot_f32: length mismatch ({len(self)} vs {x.numel()})")
        out = torch.empty(1, dtype=torch.float32, device=x.device)
        _lib.call("kh_bf16_dot_f32", ptr(self.data), 1, len(self), ptr(x), len(self), ptr(out),
                  stream_ptr(stream))
        return out[0]

    def update_from_f32(self, delta, stream=None):
        d = to_device(delta, np.float32)
        _chk(d.numel() == len(self), "update_from_f32: length mismatch")
        _lib.call("kh_bf16_update_from_f32", ptr(self.data), ptr(d), len(self), stream_ptr(stream))


def bf16_full_dot(a: torch.Tensor, b: torch.Tensor, stream=None) -> torch.Tensor:
    """Bf16FullMode::dot (bf16/mod.rs:122-134) on int16 bit tensors."""
    _chk(a.numel() == b.numel(), "Bf16FullMode::dot: length mismatch")
    out = torch.empty(1, dtype=torch.float32, device=a.device)
    _lib.call("kh_bf16_full_dot", ptr(a), ptr(b), a.numel(), ptr(out), stream_ptr(stream))
    return out[0]
