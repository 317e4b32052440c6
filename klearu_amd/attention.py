"""Head-sparse decode attention host mirror.

Mirrors sparse_attention::forward_sparse
(crates/klearu-llm/src/sparse/sparse_attention.rs:7-79) over an Attention's
q/k/v/o projections (model/attention.rs:8-64), a KvCache (model/kv_cache.rs:5-78)
and a RotaryEmbedding (model/rope.rs:17-87).  One SparseAttention owns one
layer's BF16 weights, its RoPE tables and the KV caches of up to max_batch
sequences on the GPU; forward_sparse runs one decode step for sequences
0..batch-1, each with its own selected heads.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from ._dev import hptr, ptr, stream_ptr, to_device

KV_BF16, KV_F32 = 0, 1


def _bf16_bits(w):
    """BF16 weights as uint16 bits (numpy) or a device tensor (bf16 / int16)."""
    if isinstance(w, torch.Tensor):
        if w.dtype == torch.bfloat16:
            w = w.view(torch.int16)
        if w.dtype != torch.int16:
            raise TypeError("device weights must be bfloat16 (or int16 bit patterns)")
        return w.contiguous()
    a = np.ascontiguousarray(w)
    if a.dtype != np.uint16:
        raise TypeError("host weights must be uint16 BF16 bit patterns")
    return a


class SparseAttention:
    def __init__(self, hidden_size, num_heads, num_kv_heads, head_dim, wq, wk, wv, wo, max_seq_len,
                 max_batch=1, rope_theta=10000.0, kv_dtype=KV_BF16):
        ws = [_bf16_bits(w) for w in (wq, wk, wv, wo)]
        qd, kvd = num_heads * head_dim, num_kv_heads * head_dim
        shapes = [(qd, hidden_size), (kvd, hidden_size), (kvd, hidden_size), (hidden_size, qd)]
        for w, s in zip(ws, shapes):
            if tuple(w.shape) != s:
                raise ValueError(f"weight shape {tuple(w.shape)} != {s}")
        self.hidden_size, self.num_heads, self.num_kv_heads, self.head_dim = (hidden_size, num_heads,
                                                                              num_kv_heads, head_dim)
        self.max_seq_len, self.max_batch = max_seq_len, max_batch
        h = C.c_void_p()
        dev = isinstance(ws[0], torch.Tensor)
        fn = "kh_sparse_attn_create_dev" if dev else "kh_sparse_attn_create"
        args = [ptr(w) for w in ws] if dev else [hptr(w) for w in ws]
        _lib.call(fn, hidden_size, num_heads, num_kv_heads, head_dim, max_seq_len, max_batch,
                  float(rope_theta), kv_dtype, *args, C.byref(h))
        self._h = h

    @classmethod
    def from_safetensors(cls, st, layer, num_heads, num_kv_heads, head_dim, max_seq_len, max_batch=1,
                         rope_theta=10000.0, kv_dtype=KV_BF16):
        """Layer `layer`'s self_attn.{q,k,v,o}_proj.weight (weight/loader.rs:96-111) from a
        formats.SafeTensorsFile, uploaded as BF16; the head geometry comes from the config."""
        h = C.c_void_p()
        _lib.call("kh_sparse_attn_create_from_safetensors", st._h, layer, num_heads, num_kv_heads, head_dim,
                  max_seq_len, max_batch, float(rope_theta), kv_dtype, C.byref(h))
        self = cls.__new__(cls)
        self._h = h
        self.hidden_size = st.info(st.layer_name(layer, "self_attn.q_proj.weight")).shape[1]
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.max_seq_len, self.max_batch = max_seq_len, max_batch
        return self

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_sparse_attn_destroy(h)
            except Exception:
                pass

    # -- KvCache
    def load_cache(self, b, k, v):
        """k, v: f32 [num_kv_heads][len][head_dim] -> positions 0..len-1 of sequence b."""
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        if k.shape != v.shape or k.ndim != 3 or k.shape[0] != self.num_kv_heads or k.shape[2] != self.head_dim:
            raise ValueError("cache arrays must be [num_kv_heads][len][head_dim]")
        _lib.call("kh_sparse_attn_load_cache", self._h, b, hptr(k), hptr(v), k.shape[1])

    def load_cache_dev(self, b, k, v, stream=None):
        """Device f32 tensors [num_kv_heads][len][head_dim] -> sequence b (enqueued)."""
        k = to_device(k, np.float32)
        v = to_device(v, np.float32)
        if k.shape != v.shape or k.dim() != 3 or k.shape[0] != self.num_kv_heads or k.shape[2] != self.head_dim:
            raise ValueError("cache tensors must be [num_kv_heads][len][head_dim]")
        _lib.call("kh_sparse_attn_load_cache_dev", self._h, b, ptr(k), ptr(v), k.shape[1], stream_ptr(stream))

    def read_cache(self, b, length):
        k = np.zeros((self.num_kv_heads, length, self.head_dim), np.float32)
        v = np.zeros_like(k)
        _lib.call("kh_sparse_attn_read_cache", self._h, b, hptr(k), hptr(v), length)
        return k, v

    def current_len(self, b=0) -> int:
        n = C.c_int64()
        _lib.call("kh_sparse_attn_cache_len", self._h, b, C.byref(n))
        return n.value

    def clear(self, stream=None):
        _lib.call("kh_sparse_attn_clear", self._h, stream_ptr(stream))

    # -- forward
    def forward_sparse(self, x, active_heads, positions=None, out=None, accumulate=False, stream=None):
        """x [batch, hidden] f32; active_heads [batch, n] ints (or a list for batch 1).
        Returns out [batch, hidden] on the device."""
        x = to_device(x, np.float32).reshape(-1, self.hidden_size)
        B = x.shape[0]
        if isinstance(active_heads, torch.Tensor):
            heads = active_heads.to(device=x.device, dtype=torch.int32).reshape(B, -1).contiguous()
        else:
            heads = to_device(np.asarray(active_heads, np.int32).reshape(B, -1))
        pos = None
        if positions is not None:
            pos = to_device(np.asarray(positions, np.int64).reshape(B)) if not isinstance(positions, torch.Tensor) \
                else positions.to(device=x.device, dtype=torch.int64).contiguous()
        if out is None:
            out = torch.empty(B, self.hidden_size, dtype=torch.float32, device=x.device)
        _lib.call("kh_sparse_attn_forward", self._h, ptr(x), B, ptr(pos), ptr(heads), heads.shape[1], ptr(out),
                  1 if accumulate else 0, stream_ptr(stream))
        return out


def forward_sparse(attn: SparseAttention, input, position, active_heads):
    """sparse_attention::forward_sparse for sequence 0: one token, host in / host out."""
    out = attn.forward_sparse(np.asarray(input, np.float32)[None, :], np.asarray(active_heads, np.int32)[None, :],
                              positions=[position])
    return out[0].cpu().numpy()


def attn_block(predictor, attn: SparseAttention, hidden: torch.Tensor, norm_w: torch.Tensor, eps: float, k: int,
               heads: torch.Tensor | None = None, norm_ws: torch.Tensor | None = None, stream=None):
    """One decode step of the attention half of a sparse decoder layer for sequence 0
    (crates/klearu-llm/src/sparse/mod.rs:56-112), in place:
    hidden += forward_sparse(attn, RmsNorm(hidden), position, predictor.select_top_k(RmsNorm(hidden), k)).
    The norm, and so the head selection, is bit-identical to the reference's.  `norm_ws` (one
    float on the device, allocated when None) receives the row's RmsNorm scale.  Returns the
    head ids (ascending)."""
    if norm_ws is None:
        norm_ws = torch.empty(1, dtype=torch.float32, device=hidden.device)
    if heads is None:
        heads = torch.empty(k, dtype=torch.int32, device=hidden.device)
    _lib.call("kh_dejavu_attn_block", predictor._h, attn._h, ptr(hidden), ptr(norm_w), float(eps), k, ptr(heads),
              ptr(norm_ws), stream_ptr(stream))
    return heads


def attn_block_batch(predictor, attn: SparseAttention, hidden: torch.Tensor, norm_w: torch.Tensor, eps: float,
                     k: int, heads: torch.Tensor | None = None, norm_ws: torch.Tensor | None = None, stream=None):
    """attn_block for sequences 0..B-1 of hidden [B][hidden], one decode step each (the
    reference decodes a batch one token at a time, crates/klearu-llm/src/sparse/mod.rs:56-112):
    each row's norm and head selection are the reference's, bit for bit.  `norm_ws` [B]
    receives the rows' RmsNorm scales.  Returns the heads [B][k] (ascending per row)."""
    B = hidden.shape[0]
    if norm_ws is None:
        norm_ws = torch.empty(B, dtype=torch.float32, device=hidden.device)
    if heads is None:
        heads = torch.empty(B, k, dtype=torch.int32, device=hidden.device)
    _lib.call("kh_dejavu_attn_block_batch", predictor._h, attn._h, ptr(hidden), B, ptr(norm_w), float(eps), k,
              ptr(heads), ptr(norm_ws), stream_ptr(stream))
    return heads
