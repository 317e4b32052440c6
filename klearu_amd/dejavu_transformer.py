"""klearu-dejavu transformer layer host mirror: Linear, SparseMlp, SparseAttention.

Mirrors crates/klearu-dejavu/src/transformer/mod.rs:79-134 (Linear with f32
weight [out][in] and bias), mlp.rs:5-64 (SparseMlp) and attention.rs:4-80
(SparseAttention).  Outputs are bit-identical to the reference; every
computation runs in libklearu_hip.so.  Index lists are host sequences, as the
reference's &[usize].
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from ._dev import hptr, ptr, stream_ptr, to_device


def _indices(idx) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(idx, dtype=np.int64).reshape(-1))
    return a


class Linear:
    """Linear{weight, bias, in_features, out_features} on the GPU."""

    def __init__(self, weight, bias=None):
        w = np.ascontiguousarray(weight, np.float32)
        self.out_features, self.in_features = w.shape
        b = np.zeros(self.out_features, np.float32) if bias is None else np.ascontiguousarray(bias, np.float32)
        if b.size != self.out_features:
            raise ValueError("bias must have out_features entries")
        h = C.c_void_p()
        _lib.call("kh_dejavu_linear_create", self.in_features, self.out_features, hptr(w), hptr(b), C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_dejavu_linear_destroy(h)
            except Exception:
                pass

    def forward(self, x, stream=None) -> torch.Tensor:
        """output = weight * input + bias for x [in] or [batch, in]."""
        x = to_device(x, np.float32)
        xb = x.reshape(-1, self.in_features)
        y = torch.empty(xb.shape[0], self.out_features, dtype=torch.float32, device=x.device)
        _lib.call("kh_dejavu_linear_forward", self._h, ptr(xb), xb.shape[0], ptr(y), stream_ptr(stream))
        return y.reshape(*x.shape[:-1], self.out_features)

    def forward_sparse(self, x, indices, stream=None) -> torch.Tensor:
        """Values of rows `indices` (in that order); the reference returns (index, value) pairs."""
        idx = _indices(indices)
        x = to_device(x, np.float32)
        xb = x.reshape(-1, self.in_features)
        y = torch.empty(xb.shape[0], idx.size, dtype=torch.float32, device=x.device)
        _lib.call("kh_dejavu_linear_forward_sparse", self._h, ptr(xb), xb.shape[0], hptr(idx), idx.size, ptr(y),
                  stream_ptr(stream))
        return y.reshape(*x.shape[:-1], idx.size)


class SparseMlp:
    """SparseMlp::new(hidden_size, intermediate_size) / forward."""

    def __init__(self, hidden_size: int, intermediate_size: int):
        self.hidden_size, self.intermediate_size = hidden_size, intermediate_size
        h = C.c_void_p()
        _lib.call("kh_dejavu_sparse_mlp_create", hidden_size, intermediate_size, C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_dejavu_sparse_mlp_destroy(h)
            except Exception:
                pass

    def forward(self, x, gate_proj: Linear, up_proj: Linear, down_proj: Linear, selected_neurons,
                stream=None) -> torch.Tensor:
        sel = _indices(selected_neurons)
        x = to_device(x, np.float32)
        xb = x.reshape(-1, self.hidden_size)
        y = torch.empty_like(xb)
        _lib.call("kh_dejavu_sparse_mlp_forward", self._h, ptr(xb), xb.shape[0], gate_proj._h, up_proj._h,
                  down_proj._h, hptr(sel), sel.size, ptr(y), stream_ptr(stream))
        return y.reshape(x.shape)

    def flops_savings(self, num_selected: int) -> float:
        return float(np.float32(1.0) - np.float32(num_selected) / np.float32(self.intermediate_size))


class SparseAttention:
    """SparseAttention::new(config) / forward over the selected heads."""

    def __init__(self, hidden_size: int, num_heads: int, head_dim: int):
        self.hidden_size, self.num_heads, self.head_dim = hidden_size, num_heads, head_dim
        h = C.c_void_p()
        _lib.call("kh_dejavu_sparse_attention_create", hidden_size, num_heads, head_dim, C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_dejavu_sparse_attention_destroy(h)
            except Exception:
                pass

    def forward(self, x, q_proj: Linear, k_proj: Linear, v_proj: Linear, o_proj: Linear, selected_heads,
                stream=None) -> torch.Tensor:
        heads = _indices(selected_heads)
        x = to_device(x, np.float32)
        xb = x.reshape(-1, self.hidden_size)
        y = torch.empty_like(xb)
        _lib.call("kh_dejavu_sparse_attention_forward", self._h, ptr(xb), xb.shape[0], q_proj._h, k_proj._h,
                  v_proj._h, o_proj._h, hptr(heads), heads.size, ptr(y), stream_ptr(stream))
        return y.reshape(x.shape)

    def flops_savings(self, num_selected: int) -> float:
        return float(np.float32(1.0) - np.float32(num_selected) / np.float32(self.num_heads))
