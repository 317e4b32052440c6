"""SLIDE layer host mirror.

Mirrors Layer / LayerConfig / LayerOutput (crates/klearu-core/src/network/layer.rs:10-120,
crates/klearu-core/src/config.rs:67-105).  Weights are explicit (the reference's
Xavier init draws from rand_distr and is not on the inference path); the LSH
index is built like Layer::new (layer.rs:40-44): create_lsh_index with seed
+ 1_000_000, then insert neurons 0..n-1 in order.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from ._dev import hptr, ptr, stream_ptr, to_device
from .lsh import LshConfig, create_lsh_index, csr_batch

SAMPLING = {"Vanilla": 0, "TopK": 1, "Threshold": 2}
ACTIVATION = {"Relu": 0, "Sigmoid": 1, "Tanh": 2, "Softmax": 3, "Identity": 4}


@dataclass
class LayerConfig:
    input_dim: int
    num_neurons: int
    activation: str = "Relu"
    lsh: LshConfig = field(default_factory=LshConfig)
    sampling: str = "TopK"
    sampling_threshold: int = 2
    top_k: int = 0
    is_output: bool = False

    @classmethod
    def hidden(cls, input_dim, num_neurons):
        return cls(input_dim, num_neurons, "Relu", LshConfig(), "TopK", 2, num_neurons // 10, False)

    @classmethod
    def output(cls, input_dim, num_neurons):
        return cls(input_dim, num_neurons, "Softmax", LshConfig(), "TopK", 2, num_neurons // 10, True)


@dataclass
class LayerOutput:
    activations: np.ndarray      # dense [num_neurons], zeros for inactive neurons
    active_neurons: np.ndarray   # ascending ids
    pre_activations: np.ndarray  # in active_neurons order


class Layer:
    def __init__(self, config: LayerConfig, weights, bias, seed: int, index=None):
        w = np.ascontiguousarray(weights, np.float32)
        b = np.ascontiguousarray(bias, np.float32)
        if w.shape != (config.num_neurons, config.input_dim) or b.size != config.num_neurons:
            raise ValueError("weights must be [num_neurons, input_dim] and bias [num_neurons]")
        self.config = config
        self.index = index or create_lsh_index(config.lsh, config.input_dim, seed + 1_000_000)
        h = C.c_void_p()
        _lib.call("kh_slide_layer_create", config.input_dim, config.num_neurons, hptr(w), hptr(b), self.index._h,
                  SAMPLING[config.sampling], config.top_k, config.sampling_threshold,
                  ACTIVATION[config.activation], C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_slide_layer_destroy(h)
            except Exception:
                pass

    def _cap(self, B):
        L = self.index.num_tables()
        return B * max(self.config.num_neurons, L * self.index.cap)

    def forward_batch(self, X, capacity=None, stream=None):
        """Dense X [B, input_dim] -> device CSR (off, ids, pre, act)."""
        X = to_device(X, np.float32).reshape(-1, self.config.input_dim)
        B = X.shape[0]
        cap = capacity or self._cap(B)
        off = torch.empty(B + 1, dtype=torch.int64, device=X.device)
        ids = torch.empty(cap, dtype=torch.int32, device=X.device)
        pre = torch.empty(cap, dtype=torch.float32, device=X.device)
        act = torch.empty(cap, dtype=torch.float32, device=X.device)
        _lib.call("kh_slide_layer_forward", self._h, ptr(X), B, ptr(off), ptr(ids), ptr(pre), ptr(act), cap,
                  stream_ptr(stream))
        return off, ids, pre, act

    def forward_sparse_batch(self, vectors, capacity=None, stream=None):
        xo, xi, xv = csr_batch(vectors)
        B = len(vectors)
        cap = capacity or self._cap(B)
        off = torch.empty(B + 1, dtype=torch.int64, device="cuda")
        ids = torch.empty(cap, dtype=torch.int32, device="cuda")
        pre = torch.empty(cap, dtype=torch.float32, device="cuda")
        act = torch.empty(cap, dtype=torch.float32, device="cuda")
        _lib.call("kh_slide_layer_forward_sparse", self._h, ptr(xo), ptr(xi), ptr(xv), B, ptr(off), ptr(ids),
                  ptr(pre), ptr(act), cap, stream_ptr(stream))
        return off, ids, pre, act

    def forward(self, x) -> LayerOutput:
        """Layer::forward for one dense input."""
        off, ids, pre, act = self.forward_batch(np.asarray(x, np.float32)[None, :])
        n = int(off[1].item())
        a = ids[:n].cpu().numpy().astype(np.int64)
        dense = np.zeros(self.config.num_neurons, np.float32)
        dense[a] = act[:n].cpu().numpy()
        return LayerOutput(dense, a, pre[:n].cpu().numpy())


class DenseLayer:
    """Every neuron over CSR inputs (the 128-d hidden layer of the XC net)."""

    def __init__(self, weights, bias, activation="Relu"):
        w = np.ascontiguousarray(weights, np.float32)
        b = np.ascontiguousarray(bias, np.float32)
        self.num_neurons, self.input_dim = w.shape
        h = C.c_void_p()
        _lib.call("kh_dense_layer_create", self.input_dim, self.num_neurons, hptr(w), hptr(b),
                  ACTIVATION[activation], C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_dense_layer_destroy(h)
            except Exception:
                pass

    def forward_sparse_csr(self, off, idx, val, batch, stream=None) -> torch.Tensor:
        y = torch.empty(batch, self.num_neurons, dtype=torch.float32, device="cuda")
        _lib.call("kh_dense_layer_forward_sparse", self._h, ptr(off), ptr(idx), ptr(val), batch, ptr(y),
                  stream_ptr(stream))
        return y

    def forward_sparse(self, vectors, stream=None) -> torch.Tensor:
        off, idx, val = csr_batch(vectors)
        return self.forward_sparse_csr(off, idx, val, len(vectors), stream)
