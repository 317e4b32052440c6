"""Deja Vu host mirror: SparsityPredictor, PredictorStore, sparse MLP, top-k.

Mirrors the reference's interfaces (same names, argument meaning, panics ->
exceptions):
  SparsityPredictor  crates/klearu-dejavu/src/predictor/mlp_predictor.rs:11-135
  PredictorStore     crates/klearu-llm/src/sparse/predictor_store.rs:6-89
  forward_sparse     crates/klearu-llm/src/sparse/sparse_mlp.rs:4-37
  Mlp                crates/klearu-llm/src/model/mlp.rs:6-21
All compute runs in libklearu_hip.so on the current torch stream.
"""
from __future__ import annotations

import ctypes as C
import math
import os

import numpy as np
import torch

from . import _lib
from ._dev import hptr, ptr, stream_ptr, to_device

ORDER_SCORE, ORDER_ASCENDING = 0, 1


def keep_count(n: int, frac: float) -> int:
    """ceil(n_f32 * frac_f32) as the reference computes it (sparse/mod.rs:76-77, :120-121)."""
    return int(math.ceil(float(np.float32(n) * np.float32(frac))))


class SparsityPredictor:
    """Two-layer predictor (ReLU -> sigmoid) with reference-exact scores."""

    def __init__(self, w1, b1, w2, b2):
        w1 = np.ascontiguousarray(w1, np.float32)
        w2 = np.ascontiguousarray(w2, np.float32)
        b1 = np.ascontiguousarray(b1, np.float32)
        b2 = np.ascontiguousarray(b2, np.float32)
        self.hidden_dim, self.input_dim = w1.shape
        self.output_dim = w2.shape[0]
        if w2.shape[1] != self.hidden_dim or b1.size != self.hidden_dim or b2.size != self.output_dim:
            raise ValueError("inconsistent predictor shapes")
        h = C.c_void_p()
        _lib.call("kh_predictor_create", self.input_dim, self.hidden_dim, self.output_dim, hptr(w1),
                  hptr(b1), hptr(w2), hptr(b2), C.byref(h))
        self._h = h

    from_weights = classmethod(lambda cls, w1, b1, w2, b2: cls(w1, b1, w2, b2))

    @classmethod
    def _adopt(cls, h):
        self = cls.__new__(cls)
        self._h = h
        din, dh, dout = C.c_int(), C.c_int(), C.c_int()
        _lib.call("kh_predictor_dims", h, C.byref(din), C.byref(dh), C.byref(dout))
        self.input_dim, self.hidden_dim, self.output_dim = din.value, dh.value, dout.value
        return self

    @classmethod
    def load(cls, path):
        """SparsityPredictor::load (mlp_predictor.rs:94-98): the serde JSON file
        {w1, b1, w2, b2, input_dim, hidden_dim, output_dim}, parsed natively."""
        h = C.c_void_p()
        _lib.call("kh_predictor_load", os.fsencode(path), C.byref(h))
        return cls._adopt(h)

    def save(self, path):
        """SparsityPredictor::save (mlp_predictor.rs:87-92)."""
        _lib.call("kh_predictor_save", self._h, os.fsencode(path))

    def weights(self):
        """(w1 [hidden][input], b1, w2 [output][hidden], b2) as f32 host arrays."""
        w1 = np.empty((self.hidden_dim, self.input_dim), np.float32)
        b1 = np.empty(self.hidden_dim, np.float32)
        w2 = np.empty((self.output_dim, self.hidden_dim), np.float32)
        b2 = np.empty(self.output_dim, np.float32)
        _lib.call("kh_predictor_weights", self._h, hptr(w1), hptr(b1), hptr(w2), hptr(b2))
        return w1, b1, w2, b2

    def status(self):
        """Raises KlearuError if a batched call since the last check gave up a
        bounded wait between its waves (its scores are then not trusted)."""
        _lib.call("kh_predictor_status", self._h)

    def set_spin_limit(self, spins: int):
        """Test hook: sleeps after which such a wait gives up (default 4194304)."""
        _lib.call("kh_predictor_set_spin_limit", self._h, int(spins))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_predictor_destroy(h)
            except Exception:
                pass

    def predict(self, x: torch.Tensor, stream=None) -> torch.Tensor:
        """Scores in [0,1]: x [input] or [batch, input] -> [output] / [batch, output]."""
        x = to_device(x, np.float32)
        squeeze = x.dim() == 1
        xb = x.reshape(-1, self.input_dim)
        out = torch.empty(xb.shape[0], self.output_dim, dtype=torch.float32, device=x.device)
        _lib.call("kh_predictor_predict", self._h, ptr(xb), xb.shape[0], ptr(out), stream_ptr(stream))
        return out[0] if squeeze else out

    def select_top_k(self, x: torch.Tensor, k: int, order: int = ORDER_SCORE, stream=None) -> torch.Tensor:
        """Top-k ids (int32), score order (reference) or ascending."""
        x = to_device(x, np.float32)
        squeeze = x.dim() == 1
        xb = x.reshape(-1, self.input_dim)
        kk = min(k, self.output_dim)
        out = torch.empty(xb.shape[0], kk, dtype=torch.int32, device=x.device)
        if kk > 0:
            _lib.call("kh_predictor_select_top_k", self._h, ptr(xb), xb.shape[0], k, order, ptr(out),
                      stream_ptr(stream))
        return out[0] if squeeze else out

    def select_top_k_union(self, x: torch.Tensor, k: int, stream=None):
        """Ascending top-k ids [batch, min(k, output)] and their union (ids, device count)."""
        x = to_device(x, np.float32)
        xb = x.reshape(-1, self.input_dim)
        kk = min(k, self.output_dim)
        ids = torch.empty(xb.shape[0], kk, dtype=torch.int32, device=x.device)
        uni = torch.empty(max(1, self.output_dim), dtype=torch.int32, device=x.device)
        cnt = torch.zeros(1, dtype=torch.int32, device=x.device)
        _lib.call("kh_predictor_select_top_k_union", self._h, ptr(xb), xb.shape[0], k, ptr(ids), ptr(uni),
                  ptr(cnt), stream_ptr(stream))
        return ids, uni, cnt


class PredictorStore:
    """Per-layer head / neuron predictors; missing ones fall back to 0..k."""

    def __init__(self, num_layers: int):
        self.head_predictors = [None] * num_layers
        self.neuron_predictors = [None] * num_layers
        self.num_layers = num_layers

    def set_head_predictor(self, layer, p):
        self.head_predictors[layer] = p

    def set_neuron_predictor(self, layer, p):
        self.neuron_predictors[layer] = p

    def is_calibrated(self) -> bool:
        return any(p is not None for p in self.head_predictors + self.neuron_predictors)

    def _pick(self, p, x, k, order, stream):
        if p is None:
            x = to_device(x, np.float32)
            return torch.arange(k, dtype=torch.int32, device=x.device)
        return p.select_top_k(x, k, order, stream)

    def predict_heads(self, layer, x, k, order=ORDER_SCORE, stream=None):
        return self._pick(self.head_predictors[layer], x, k, order, stream)

    def predict_neurons(self, layer, x, k, order=ORDER_SCORE, stream=None):
        return self._pick(self.neuron_predictors[layer], x, k, order, stream)

    def save(self, directory):
        """PredictorStore::save (predictor_store.rs:59-74): layer_{i}_{head,neuron}.json."""
        os.makedirs(directory, exist_ok=True)
        for i, p in enumerate(self.head_predictors):
            if p is not None:
                p.save(os.path.join(directory, f"layer_{i}_head.json"))
        for i, p in enumerate(self.neuron_predictors):
            if p is not None:
                p.save(os.path.join(directory, f"layer_{i}_neuron.json"))

    @classmethod
    def load(cls, directory, num_layers):
        """PredictorStore::load (predictor_store.rs:76-89): layer_{i}_{head,neuron}.json;
        a missing file leaves that layer on the first-k fallback."""
        s = cls(num_layers)
        for i in range(num_layers):
            hp = os.path.join(directory, f"layer_{i}_head.json")
            npth = os.path.join(directory, f"layer_{i}_neuron.json")
            if os.path.exists(hp):
                s.head_predictors[i] = SparsityPredictor.load(hp)
            if os.path.exists(npth):
                s.neuron_predictors[i] = SparsityPredictor.load(npth)
        return s


def topk_select(scores: torch.Tensor, k: int, order: int = ORDER_SCORE, stream=None) -> torch.Tensor:
    """Stable top-k of scores [batch, n] (or [n]) -> int32 ids."""
    scores = to_device(scores, np.float32)
    squeeze = scores.dim() == 1
    s2 = scores.reshape(-1, scores.shape[-1])
    kk = min(k, s2.shape[1])
    out = torch.empty(s2.shape[0], kk, dtype=torch.int32, device=scores.device)
    if kk > 0:
        _lib.call("kh_topk_select", ptr(s2), s2.shape[0], s2.shape[1], k, order, ptr(out),
                  stream_ptr(stream))
    return out[0] if squeeze else out


def union_active(ids: torch.Tensor, n: int, stream=None):
    """Union of per-token id sets [batch, k] over [0, n): (ids ascending [<=n], count tensor)."""
    ids = to_device(ids, np.int32)
    out = torch.empty(n, dtype=torch.int32, device=ids.device)
    cnt = torch.zeros(1, dtype=torch.int32, device=ids.device)
    b = ids.shape[0] if ids.dim() == 2 else 1
    k = ids.shape[-1]
    _lib.call("kh_union_active", ptr(ids), b, k, n, ptr(out), ptr(cnt), stream_ptr(stream))
    return out, cnt


class Mlp:
    """SwiGLU MLP with BF16 weights (bits as uint16) in the reference layout."""

    def __init__(self, w_gate, w_up, w_down, max_batch: int = 16):
        w_gate = np.ascontiguousarray(w_gate, np.uint16)
        w_up = np.ascontiguousarray(w_up, np.uint16)
        w_down = np.ascontiguousarray(w_down, np.uint16)
        self.intermediate_size, self.hidden_size = w_gate.shape
        if w_up.shape != w_gate.shape or w_down.shape != (self.hidden_size, self.intermediate_size):
            raise ValueError("inconsistent MLP shapes")
        h = C.c_void_p()
        _lib.call("kh_sparse_ffn_create", self.hidden_size, self.intermediate_size, hptr(w_gate),
                  hptr(w_up), hptr(w_down), max_batch, C.byref(h))
        self._h = h
        self.max_batch = max_batch

    @classmethod
    def from_safetensors(cls, st, layer: int, max_batch: int = 16):
        """Layer `layer`'s mlp.{gate,up,down}_proj.weight (weight/loader.rs:125-133) from a
        formats.SafeTensorsFile, uploaded as BF16 without a host-side float copy."""
        h = C.c_void_p()
        _lib.call("kh_sparse_ffn_create_from_safetensors", st._h, layer, max_batch, C.byref(h))
        self = cls.__new__(cls)
        self._h = h
        self.max_batch = max_batch
        self.intermediate_size, self.hidden_size = st.info(st.layer_name(layer, "mlp.gate_proj.weight")).shape
        return self

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_sparse_ffn_destroy(h)
            except Exception:
                pass

    def forward_sparse_into(self, x, active, y, accumulate=False, n_active_dev=None, stream=None,
                            n_active=None):
        n = active.numel() if n_active is None else n_active
        b = x.shape[0] if x.dim() == 2 else 1
        _lib.call("kh_sparse_ffn_forward", self._h, ptr(x), b, ptr(active), n, ptr(n_active_dev), ptr(y),
                  1 if accumulate else 0, stream_ptr(stream))
        return y

    def last_hidden(self, batch, n_active, stream=None):
        h = torch.empty(batch, n_active, dtype=torch.float32, device="cuda")
        _lib.call("kh_sparse_ffn_last_hidden", self._h, ptr(h), batch, n_active, stream_ptr(stream))
        return h

    def status(self):
        """Raise KlearuError (KH_ERR_ARG) if a forward since the last status call saw an
        active id outside [0, intermediate) (the reference panics in get_weights)."""
        _lib.call("kh_sparse_ffn_status", self._h)


def forward_sparse(mlp: Mlp, x, active_neurons, stream=None) -> torch.Tensor:
    """sparse_mlp::forward_sparse: x [hidden] or [batch, hidden] sharing one active set."""
    x = to_device(x, np.float32)
    act = to_device(active_neurons, np.int32)
    if act.dtype != torch.int32:
        act = act.to(torch.int32)
    squeeze = x.dim() == 1
    xb = x.reshape(-1, mlp.hidden_size)
    y = torch.empty_like(xb)
    mlp.forward_sparse_into(xb, act, y, stream=stream)
    return y[0] if squeeze else y


def rmsnorm(x, w, eps: float, stream=None) -> torch.Tensor:
    """RmsNorm::forward (model/rms_norm.rs:43-64) over the last dimension."""
    x = to_device(x, np.float32)
    w = to_device(w, np.float32)
    n = x.shape[-1]
    y = torch.empty_like(x)
    _lib.call("kh_rmsnorm", ptr(x), ptr(w), x.numel() // n, n, float(eps), ptr(y), stream_ptr(stream))
    return y


def mlp_block(predictor: SparsityPredictor, mlp: Mlp, hidden: torch.Tensor, norm_w: torch.Tensor, eps: float,
              k: int, active: torch.Tensor | None = None, norm_ws: torch.Tensor | None = None, stream=None):
    """One decode step of the Deja Vu MLP block (crates/klearu-llm/src/sparse/mod.rs:115-142), in place:
    hidden += forward_sparse(mlp, RmsNorm(hidden), predictor.select_top_k(RmsNorm(hidden), k)).
    The norm, and so the selection, is bit-identical to the reference's.  `norm_ws` (one float on
    the device, allocated when None) receives the row's RmsNorm scale.  Returns the active ids
    (ascending)."""
    if norm_ws is None:
        norm_ws = torch.empty(1, dtype=torch.float32, device=hidden.device)
    if active is None:
        active = torch.empty(k, dtype=torch.int32, device=hidden.device)
    _lib.call("kh_dejavu_mlp_block", predictor._h, mlp._h, ptr(hidden), ptr(norm_w), float(eps), k, ptr(active),
              ptr(norm_ws), stream_ptr(stream))
    return active


def mlp_block_batch(predictor: SparsityPredictor, mlp: Mlp, hidden: torch.Tensor, norm_w: torch.Tensor, eps: float,
                    k: int, active: torch.Tensor | None = None, norm_ws: torch.Tensor | None = None, stream=None):
    """mlp_block for rows 0..B-1 of hidden [B][hidden] (crates/klearu-llm/src/sparse/mod.rs:115-142
    per row): each row's norm and top-k selection are the reference's, bit for bit, and the FFN
    runs over the union of the rows' selections, the shared active set of
    Mlp.forward_sparse_into with the union from select_top_k_union.  `norm_ws` [B] receives the
    rows' RmsNorm scales.  Returns the active ids [B][k] (ascending per row)."""
    B = hidden.shape[0]
    if norm_ws is None:
        norm_ws = torch.empty(B, dtype=torch.float32, device=hidden.device)
    if active is None:
        active = torch.empty(B, k, dtype=torch.int32, device=hidden.device)
    _lib.call("kh_dejavu_mlp_block_batch", predictor._h, mlp._h, ptr(hidden), B, ptr(norm_w), float(eps), k,
              ptr(active), ptr(norm_ws), stream_ptr(stream))
    return active
