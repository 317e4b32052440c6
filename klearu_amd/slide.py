"""SLIDE layer and network host mirror.

Mirrors Layer / LayerConfig / LayerOutput (crates/klearu-core/src/network/layer.rs:10-233,
crates/klearu-core/src/config.rs:67-105), Network (network/net.rs:10-174) and
RebuildScheduler (lsh/maintenance.rs:20-98).  Weights are explicit (the
reference's Xavier init draws from rand_distr); the LSH index is built like
Layer::new (layer.rs:40-44): create_lsh_index with seed + 1_000_000, then
insert neurons 0..n-1 in order.
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

    # ------------------------------------------------------------ training side
    def init_optimizer(self, optimizer="Sgd", momentum=0.9, beta1=0.9, beta2=0.999, eps=1e-8):
        """Optimizer::create_state for every neuron (zeroed)."""
        _lib.call("kh_slide_layer_init_optimizer", self._h, OPTIMIZER[optimizer], momentum, beta1, beta2, eps)

    def backward(self, x, output: LayerOutput, grad_output, lr, step, want_grad_input=True, stream=None):
        """Layer::backward (layer.rs:124-226) for one sample.  output.active_neurons
        gives the order of the sums over active neurons.  Returns grad_input
        (numpy) or None."""
        ids = to_device(np.asarray(output.active_neurons, np.uint32))
        n_act = to_device(np.array([ids.numel()], np.int32))
        pre = to_device(np.asarray(output.pre_activations, np.float32))
        dense = to_device(np.asarray(output.activations, np.float32))
        g = to_device(np.asarray(grad_output, np.float32))
        xd = to_device(np.asarray(x, np.float32))
        gi = torch.empty(self.config.input_dim, dtype=torch.float32, device="cuda") if want_grad_input else None
        _lib.call("kh_slide_layer_backward", self._h, ptr(xd), ptr(ids), ptr(n_act), ptr(pre), ptr(dense), ptr(g),
                  g.numel(), float(lr), int(step), ptr(gi), stream_ptr(stream))
        return gi.cpu().numpy() if gi is not None else None

    def rebuild_index(self, stream=None):
        """Layer::rebuild_index (layer.rs:228-233)."""
        _lib.call("kh_slide_layer_rebuild_index", self._h, stream_ptr(stream))

    def weights(self):
        w = np.empty((self.config.num_neurons, self.config.input_dim), np.float32)
        b = np.empty(self.config.num_neurons, np.float32)
        _lib.call("kh_slide_layer_weights", self._h, hptr(w), hptr(b))
        return w, b


OPTIMIZER = {"Sgd": 0, "Adam": 1}


class RebuildScheduler(C.Structure):
    """RebuildScheduler (lsh/maintenance.rs:20-98); state lives in this struct."""

    _fields_ = [("base_interval", C.c_uint64), ("decay", C.c_double), ("rebuild_count", C.c_uint64),
                ("next_rebuild_step", C.c_uint64), ("current_step", C.c_uint64)]

    def __init__(self, base_interval=100, decay=0.1):
        super().__init__()
        _lib.load().kh_rebuild_scheduler_init(C.byref(self), int(base_interval), float(decay))

    def step(self) -> bool:
        return bool(_lib.load().kh_rebuild_scheduler_step(C.byref(self)))

    def should_rebuild(self, step) -> bool:
        return bool(_lib.load().kh_rebuild_scheduler_should_rebuild(C.byref(self), int(step)))

    def next_rebuild(self) -> int:
        return int(self.next_rebuild_step)


class Network:
    """Network (net.rs:10-174) over Layer objects (kept alive here).

    optimizer "Sgd" (Sgd::new(momentum), the reference config uses 0.9) or
    "Adam" (Adam::new(beta1, beta2, eps), default 0.9 / 0.999 / 1e-8); the
    scheduler takes the first layer's rebuild settings (net.rs:32-38)."""

    def __init__(self, layers, optimizer="Sgd", momentum=0.9, beta1=0.9, beta2=0.999, eps=1e-8,
                 rebuild_base=None, rebuild_decay=None):
        self.layers = list(layers)
        lsh = self.layers[0].config.lsh
        base = getattr(lsh, "rebuild_interval_base", 100) if rebuild_base is None else rebuild_base
        decay = getattr(lsh, "rebuild_decay", 0.1) if rebuild_decay is None else rebuild_decay
        arr = (C.c_void_p * len(self.layers))(*[l._h.value for l in self.layers])
        h = C.c_void_p()
        _lib.call("kh_slide_network_create", arr, len(self.layers), OPTIMIZER[optimizer], momentum, beta1, beta2,
                  eps, int(base), float(decay), C.byref(h))
        self._h = h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_slide_network_destroy(h)
            except Exception:
                pass

    def train_step(self, X, labels, lr, stream=None) -> float:
        """Network::train_step (net.rs:81-120): X [B, input_dim] dense
        (features.to_dense()), labels one id list per example."""
        X = to_device(X, np.float32).reshape(-1, self.layers[0].config.input_dim)
        B = X.shape[0]
        off = np.zeros(B + 1, np.int64)
        for i, lab in enumerate(labels[:B]):
            off[i + 1] = off[i] + len(lab)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(l, np.uint32) for l in labels[:B]] or
                                                   [np.zeros(0, np.uint32)]), np.uint32)
        loss = C.c_float()
        _lib.call("kh_slide_network_train_step", self._h, ptr(X), B, hptr(off), hptr(flat) if flat.size else None,
                  float(lr), C.byref(loss), stream_ptr(stream))
        return float(loss.value)

    def train_step_sparse(self, vectors, labels, lr, csr=None, stream=None) -> float:
        """train_step with each example's features as a SparseVector (densified
        as SparseVector::to_dense does); csr=(off, idx, val) device arrays
        instead of `vectors` skips the host conversion."""
        off, idx, val = csr if csr is not None else csr_batch(vectors)
        B = off.numel() - 1
        loff = np.zeros(B + 1, np.int64)
        for i, lab in enumerate(labels[:B]):
            loff[i + 1] = loff[i] + len(lab)
        flat = np.ascontiguousarray(np.concatenate([np.asarray(l, np.uint32) for l in labels[:B]] or
                                                   [np.zeros(0, np.uint32)]), np.uint32)
        loss = C.c_float()
        _lib.call("kh_slide_network_train_step_sparse", self._h, ptr(off), ptr(idx), ptr(val), B, hptr(loff),
                  hptr(flat) if flat.size else None, float(lr), C.byref(loss), stream_ptr(stream))
        return float(loss.value)

    def predict_sparse(self, vectors, stream=None) -> torch.Tensor:
        off, idx, val = csr_batch(vectors)
        out = torch.empty(len(vectors), self.layers[-1].config.num_neurons, dtype=torch.float32, device="cuda")
        _lib.call("kh_slide_network_predict_sparse", self._h, ptr(off), ptr(idx), ptr(val), len(vectors), ptr(out),
                  stream_ptr(stream))
        return out

    def predict_batch(self, X, stream=None) -> torch.Tensor:
        """Network::predict (net.rs:151-154) per row: the last layer's dense activations."""
        X = to_device(X, np.float32).reshape(-1, self.layers[0].config.input_dim)
        out = torch.empty(X.shape[0], self.layers[-1].config.num_neurons, dtype=torch.float32, device=X.device)
        _lib.call("kh_slide_network_predict", self._h, ptr(X), X.shape[0], ptr(out), stream_ptr(stream))
        return out

    def predict(self, x) -> np.ndarray:
        return self.predict_batch(np.asarray(x, np.float32)[None, :])[0].cpu().numpy()

    def predict_top_k(self, x, k):
        """Network::predict_top_k (net.rs:159-174): (label, score) by score
        descending; a stable sort, so ties keep ascending labels."""
        out = self.predict(x)
        order = sorted(range(out.size), key=lambda i: -out[i])[:k]
        return [(i, float(out[i])) for i in order]

    @property
    def step(self) -> int:
        s = C.c_uint64()
        _lib.call("kh_slide_network_state", self._h, C.byref(s), None)
        return int(s.value)

    def scheduler(self) -> RebuildScheduler:
        r = RebuildScheduler.__new__(RebuildScheduler)
        C.Structure.__init__(r)
        _lib.call("kh_slide_network_state", self._h, None, C.byref(r))
        return r


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


class SparseInferenceEngine:
    """SparseInferenceEngine (crates/klearu-bolt/src/sparse_inference.rs:8-111)
    over a Layer's index and weights."""

    def __init__(self, sparsity_multiplier: float):
        self._m = float(np.float32(sparsity_multiplier))

    def sparsity_multiplier(self) -> float:
        return self._m

    def _run(self, layer: Layer, X, base_top_k, relu, stream=None):
        X = to_device(X, np.float32).reshape(-1, layer.config.input_dim)
        B = X.shape[0]
        cap = B * max(layer.config.num_neurons, layer.index.num_tables() * layer.index.cap)
        off = torch.empty(B + 1, dtype=torch.int64, device=X.device)
        ids = torch.empty(max(cap, 1), dtype=torch.int32, device=X.device)
        act = torch.empty(max(cap, 1), dtype=torch.float32, device=X.device)
        _lib.call("kh_sparse_inference", layer._h, ptr(X), B, int(base_top_k), self._m, 1 if relu else 0, ptr(off),
                  ptr(ids), ptr(act), cap, stream_ptr(stream))
        o = off.cpu().numpy()
        i = ids.cpu().numpy().view(np.uint32)
        a = act.cpu().numpy()
        return [list(zip(i[o[b]:o[b + 1]].tolist(), a[o[b]:o[b + 1]].tolist())) for b in range(B)]

    def infer(self, x, layer: Layer, base_top_k: int):
        """(neuron_id, relu(w.x + b)) in hit-count order."""
        return self._run(layer, np.asarray(x, np.float32)[None, :], base_top_k, True)[0]

    def infer_linear(self, x, layer: Layer, base_top_k: int):
        return self._run(layer, np.asarray(x, np.float32)[None, :], base_top_k, False)[0]

    def infer_batch(self, X, layer: Layer, base_top_k: int, relu=True):
        return self._run(layer, X, base_top_k, relu)
