"""LSH host mirror: hash families, SparseVector, LshIndex, create_lsh_index.

Mirrors the reference interfaces (names, argument meaning, errors):
  HashFamily         crates/klearu-core/src/hash/mod.rs:24-39
  SimHash            crates/klearu-core/src/hash/simhash.rs:21-139
  SparseRandomProjection  crates/klearu-core/src/hash/srp.rs:22-175
  SparseVector       crates/klearu-core/src/tensor/sparse.rs:14-150
  LshIndexTrait      crates/klearu-core/src/lsh/index.rs:21-67 (+ create_lsh_index :339-373)
  LshConfig          crates/klearu-core/src/config.rs:41-65
Queries return candidates in ascending id order (the reference returns HashMap
order, which is randomised per process).  Batched device entry points
(hash_dense_batch, query_batch) are the performance path; the per-vector
methods exist for drop-in use and tests.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._dev import hptr, ptr, stream_ptr, to_device

FIFO, RESERVOIR = 0, 1


@dataclass
class LshCandidate:
    neuron_id: int
    count: int


class SparseVector:
    """Sorted (index, value) pairs of a `dim`-dimensional vector."""

    def __init__(self, indices, values, dim):
        self.indices = np.ascontiguousarray(indices, np.uint32)
        self.values = np.ascontiguousarray(values, np.float32)
        self.dim = int(dim)
        if self.indices.size != self.values.size:
            raise ValueError("indices/values length mismatch")

    @classmethod
    def from_dense(cls, dense):
        d = np.asarray(dense, np.float32)
        nz = np.nonzero(d != 0.0)[0]
        return cls(nz, d[nz], d.size)

    def to_dense(self):
        out = np.zeros(self.dim, np.float32)
        out[self.indices] = self.values
        return out

    def nnz(self):
        return int(self.indices.size)


def csr_batch(vectors):
    """List of SparseVector -> device CSR (offsets int64 [B+1], idx uint32, val f32)."""
    off = np.zeros(len(vectors) + 1, np.int64)
    for i, v in enumerate(vectors):
        off[i + 1] = off[i] + v.nnz()
    idx = np.concatenate([v.indices for v in vectors]) if vectors else np.zeros(0, np.uint32)
    val = np.concatenate([v.values for v in vectors]) if vectors else np.zeros(0, np.float32)
    return to_device(off), to_device(idx.astype(np.uint32) if idx.size else np.zeros(1, np.uint32)), \
        to_device(val if val.size else np.zeros(1, np.float32))


class HashFamily:
    """Ternary random-hyperplane family (SimHash or SRP) resident on the GPU."""

    def __init__(self, handle: C.c_void_p):
        self._h = handle
        k, d, L = C.c_int(), C.c_int(), C.c_int()
        _lib.call("kh_hash_family_dims", handle, C.byref(k), C.byref(d), C.byref(L))
        self._k, self._dim, self._L = k.value, d.value, L.value

    @classmethod
    def from_planes(cls, planes):
        planes = np.ascontiguousarray(planes, np.int8)
        L, k, dim = planes.shape
        h = C.c_void_p()
        _lib.call("kh_hash_family_from_planes", dim, k, L, hptr(planes), C.byref(h))
        return cls(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_hash_family_destroy(h)
            except Exception:
                pass

    def k(self):
        return self._k

    def input_dim(self):
        return self._dim

    def num_tables(self):
        return self._L

    def planes(self):
        out = np.empty((self._L, self._k, self._dim), np.int8)
        _lib.call("kh_hash_family_planes", self._h, hptr(out))
        return out

    def kind(self):
        """"ternary", "wta", "dwta" or "minhash" and the window size."""
        kd, ws = C.c_int(), C.c_int()
        _lib.call("kh_hash_family_kind", self._h, C.byref(kd), C.byref(ws))
        return ("ternary", "wta", "dwta", "minhash")[kd.value], ws.value

    def tables(self):
        """WTA / DWTA windows [L][k][ws] or MinHash permutations [L][dim]."""
        kind, ws = self.kind()
        shape = (self._L, self._dim) if kind == "minhash" else (self._L, self._k, ws)
        out = np.empty(shape, np.uint32)
        _lib.call("kh_hash_family_tables", self._h, hptr(out))
        return out

    def hash_dense_batch(self, X, stream=None) -> torch.Tensor:
        """codes[b][t] for X [batch, input_dim] (int32 bit patterns of u32 codes)."""
        X = to_device(X, np.float32).reshape(-1, self._dim)
        codes = torch.empty(X.shape[0], self._L, dtype=torch.int32, device=X.device)
        _lib.call("kh_hash_dense", self._h, ptr(X), X.shape[0], ptr(codes), stream_ptr(stream))
        return codes

    def hash_sparse_batch(self, vectors, stream=None) -> torch.Tensor:
        off, idx, val = csr_batch(vectors)
        codes = torch.empty(len(vectors), self._L, dtype=torch.int32, device="cuda")
        _lib.call("kh_hash_sparse", self._h, ptr(off), ptr(idx), ptr(val), len(vectors), ptr(codes),
                  stream_ptr(stream))
        return codes

    def hash_dense(self, x, table: int) -> int:
        if np.asarray(x).size != self._dim:
            raise ValueError("input dim mismatch")
        return int(self.hash_dense_batch(np.asarray(x, np.float32))[0, table].item()) & 0xFFFFFFFF

    def hash_sparse(self, sv: SparseVector, table: int) -> int:
        return int(self.hash_sparse_batch([sv])[0, table].item()) & 0xFFFFFFFF


def WtaHash(input_dim: int, k: int, num_tables: int, window_size: int, seed: int) -> HashFamily:
    """WtaHash::new (hash/wta.rs:42-90)."""
    h = C.c_void_p()
    _lib.call("kh_wta_create", input_dim, k, num_tables, window_size, seed, C.byref(h))
    return HashFamily(h)


def DwtaHash(input_dim: int, k: int, num_tables: int, window_size: int, seed: int) -> HashFamily:
    """DwtaHash::new (hash/dwta.rs:40-88)."""
    h = C.c_void_p()
    _lib.call("kh_dwta_create", input_dim, k, num_tables, window_size, seed, C.byref(h))
    return HashFamily(h)


def MinHash(input_dim: int, k: int, num_tables: int, seed: int) -> HashFamily:
    """MinHash::new (hash/minhash.rs:38-60)."""
    h = C.c_void_p()
    _lib.call("kh_minhash_create", input_dim, k, num_tables, seed, C.byref(h))
    return HashFamily(h)


def family_from_windows(windows, input_dim, dwta=False) -> HashFamily:
    """WTA / DWTA over windows [L][k][window_size] drawn elsewhere (e.g. by the reference)."""
    w = np.ascontiguousarray(windows, np.uint32)
    L, k, ws = w.shape
    h = C.c_void_p()
    _lib.call("kh_wta_from_windows", 1 if dwta else 0, input_dim, k, L, ws, hptr(w), C.byref(h))
    return HashFamily(h)


def family_from_permutations(perms, k) -> HashFamily:
    """MinHash over permutations [L][input_dim] (permutations[table][dim])."""
    p = np.ascontiguousarray(perms, np.uint32)
    L, dim = p.shape
    h = C.c_void_p()
    _lib.call("kh_minhash_from_permutations", dim, k, L, hptr(p), C.byref(h))
    return HashFamily(h)


def SimHash(input_dim: int, k: int, num_tables: int, seed: int) -> HashFamily:
    h = C.c_void_p()
    _lib.call("kh_simhash_create", input_dim, k, num_tables, seed, C.byref(h))
    return HashFamily(h)


def SparseRandomProjection(input_dim: int, k: int, num_tables: int, sparsity: float, seed: int) -> HashFamily:
    h = C.c_void_p()
    _lib.call("kh_srp_create", input_dim, k, num_tables, float(sparsity), seed, C.byref(h))
    return HashFamily(h)


@dataclass
class LshConfig:
    """config.rs:41-65 defaults; range_pow is not read; the rebuild fields set a Network's scheduler."""
    hash_function: str = "SimHash"
    bucket_type: str = "Fifo"
    num_tables: int = 50
    range_pow: int = 6
    num_hashes: int = 6
    bucket_capacity: int = 128
    rebuild_interval_base: int = 100
    rebuild_decay: float = 0.1


class LshIndex:
    """L tables x 2^K buckets of neuron ids on the GPU (insert / query / clear)."""

    def __init__(self, hash_family: HashFamily, bucket_type: int, bucket_capacity: int):
        if bucket_capacity <= 0:
            raise ValueError("bucket capacity must be positive")
        self.hash_family = hash_family
        h = C.c_void_p()
        _lib.call("kh_lsh_index_create", hash_family._h, bucket_type, bucket_capacity, C.byref(h))
        self._h = h
        self.cap = bucket_capacity
        self.bucket_type = bucket_type

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_lsh_index_destroy(h)
            except Exception:
                pass

    def num_tables(self):
        return self.hash_family.num_tables()

    # -- mutation (&mut self in the reference)
    def insert_batch(self, ids, W, stream=None):
        ids = to_device(np.asarray(ids, np.uint32) if not isinstance(ids, torch.Tensor) else ids, np.uint32)
        W = to_device(W, np.float32).reshape(ids.numel(), -1)
        _lib.call("kh_lsh_index_insert", self._h, ptr(ids), ptr(W), ids.numel(), W.shape[1], stream_ptr(stream))

    def insert(self, id: int, dense_weights):
        self.insert_batch(np.array([id], np.uint32), np.asarray(dense_weights, np.float32)[None, :])

    def insert_codes(self, ids, codes, stream=None):
        ids = to_device(ids, np.uint32)
        codes = to_device(codes, np.uint32)
        _lib.call("kh_lsh_index_insert_codes", self._h, ptr(ids), ptr(codes), ids.numel(), stream_ptr(stream))

    def insert_sparse_batch(self, ids, vectors, stream=None):
        """insert_sparse (index.rs:264-269) for (id, SparseVector) pairs in order."""
        ids = to_device(np.asarray(ids, np.uint32) if not isinstance(ids, torch.Tensor) else ids, np.uint32)
        xo, xi, xv = csr_batch(vectors)
        _lib.call("kh_lsh_index_insert_sparse", self._h, ptr(ids), ptr(xo), ptr(xi), ptr(xv), ids.numel(),
                  stream_ptr(stream))

    def insert_sparse(self, id: int, weights):
        self.insert_sparse_batch(np.array([id], np.uint32), [weights])

    def remove_with_weights_batch(self, ids, W, stream=None):
        """remove_with_weights (index.rs:271-276) for (id, dense weights) pairs in order."""
        ids = to_device(np.asarray(ids, np.uint32) if not isinstance(ids, torch.Tensor) else ids, np.uint32)
        W = to_device(W, np.float32).reshape(ids.numel(), -1)
        _lib.call("kh_lsh_index_remove_with_weights", self._h, ptr(ids), ptr(W), ids.numel(), W.shape[1],
                  stream_ptr(stream))

    def remove_with_weights(self, id: int, dense_weights):
        self.remove_with_weights_batch(np.array([id], np.uint32), np.asarray(dense_weights, np.float32)[None, :])

    def remove_batch(self, ids, stream=None):
        """remove (index.rs:278-280) of each id, in order, from every bucket."""
        ids = to_device(np.asarray(ids, np.uint32) if not isinstance(ids, torch.Tensor) else ids, np.uint32)
        _lib.call("kh_lsh_index_remove", self._h, ptr(ids), ids.numel(), stream_ptr(stream))

    def remove(self, id: int):
        self.remove_batch(np.array([id], np.uint32))

    def clear(self, stream=None):
        _lib.call("kh_lsh_index_clear", self._h, stream_ptr(stream))

    def rebuild(self, neurons, stream=None):
        """neurons: iterable of (id, dense weights); clear then insert in order (index.rs:302-307)."""
        neurons = list(neurons)
        dim = self.hash_family.input_dim()
        ids = to_device(np.array([n[0] for n in neurons], np.uint32)) if neurons else None
        W = (to_device(np.stack([np.asarray(n[1], np.float32) for n in neurons]).reshape(-1, dim))
             if neurons else None)
        _lib.call("kh_lsh_index_rebuild", self._h, ptr(ids), ptr(W), len(neurons), dim, stream_ptr(stream))

    # -- queries (&self)
    def query_batch(self, X, counts=True, capacity=None, stream=None):
        """Dense batch -> (off int64 [B+1], ids uint32-as-int32, counts) on the device."""
        X = to_device(X, np.float32).reshape(-1, self.hash_family.input_dim())
        B = X.shape[0]
        cap = capacity or B * self.num_tables() * self.cap
        off = torch.empty(B + 1, dtype=torch.int64, device=X.device)
        ids = torch.empty(max(cap, 1), dtype=torch.int32, device=X.device)
        cnt = torch.empty(max(cap, 1), dtype=torch.int32, device=X.device) if counts else None
        _lib.call("kh_lsh_index_query", self._h, ptr(X), B, ptr(off), ptr(ids), ptr(cnt), cap, stream_ptr(stream))
        return off, ids, cnt

    def query_sparse_batch(self, vectors, counts=True, capacity=None, stream=None):
        xo, xi, xv = csr_batch(vectors)
        B = len(vectors)
        cap = capacity or B * self.num_tables() * self.cap
        off = torch.empty(B + 1, dtype=torch.int64, device="cuda")
        ids = torch.empty(max(cap, 1), dtype=torch.int32, device="cuda")
        cnt = torch.empty(max(cap, 1), dtype=torch.int32, device="cuda") if counts else None
        _lib.call("kh_lsh_index_query_sparse", self._h, ptr(xo), ptr(xi), ptr(xv), B, ptr(off), ptr(ids), ptr(cnt),
                  cap, stream_ptr(stream))
        return off, ids, cnt

    @staticmethod
    def _unpack(off, ids, cnt, row=0):
        o = off.cpu().numpy()
        i = ids[o[row]:o[row + 1]].cpu().numpy().view(np.uint32)
        c = cnt[o[row]:o[row + 1]].cpu().numpy().view(np.uint32) if cnt is not None else None
        return i, c

    def query(self, x):
        i, c = self._unpack(*self.query_batch(np.asarray(x, np.float32)))
        return [LshCandidate(int(a), int(b)) for a, b in zip(i, c)]

    query_with_counts = query

    def query_union(self, x):
        i, _ = self._unpack(*self.query_batch(np.asarray(x, np.float32), counts=False))
        return [int(a) for a in i]

    def query_sparse_with_counts(self, sv: SparseVector):
        i, c = self._unpack(*self.query_sparse_batch([sv]))
        return [LshCandidate(int(a), int(b)) for a, b in zip(i, c)]

    def query_sparse_union(self, sv: SparseVector):
        i, _ = self._unpack(*self.query_sparse_batch([sv], counts=False))
        return [int(a) for a in i]

    def query_top_k(self, X, top_k, stream=None):
        """Per row of X: the candidate ids by hit count descending (ties: ascending id), at most top_k."""
        X = to_device(X, np.float32).reshape(-1, self.hash_family.input_dim())
        B = X.shape[0]
        ids = torch.empty(B, max(top_k, 1), dtype=torch.int32, device=X.device)
        n = torch.empty(B, dtype=torch.int32, device=X.device)
        _lib.call("kh_lsh_index_query_top_k", self._h, ptr(X), B, int(top_k), ptr(ids), ptr(n), stream_ptr(stream))
        ids, n = ids.cpu().numpy().view(np.uint32), n.cpu().numpy()
        return [ids[b, :n[b]].tolist() for b in range(B)]

    def buckets(self):
        """(data [L][2^K][cap], len [L][2^K], count [L][2^K]) copied to the host."""
        L, K = self.num_tables(), self.hash_family.k()
        nb = 1 << K
        data = np.zeros((L, nb, self.cap), np.uint32)
        ln = np.zeros((L, nb), np.uint32)
        cnt = np.zeros((L, nb), np.uint64)
        _lib.call("kh_lsh_index_buckets", self._h, hptr(data), hptr(ln), hptr(cnt))
        return data, ln, cnt


def create_lsh_index(config: LshConfig, input_dim: int, seed: int) -> LshIndex:
    """create_lsh_index (lsh/index.rs:339-373) for the SimHash and SRP families."""
    k, L = config.num_hashes, config.num_tables
    if config.hash_function == "SimHash":
        hf = SimHash(input_dim, k, L, seed)
    elif config.hash_function == "SparseRandomProjection":
        hf = SparseRandomProjection(input_dim, k, L, 1.0 / 3.0, seed)
    elif config.hash_function == "WtaHash":
        hf = WtaHash(input_dim, k, L, min(8, input_dim), seed)      # DEFAULT_WINDOW_SIZE (index.rs:330)
    elif config.hash_function == "DwtaHash":
        hf = DwtaHash(input_dim, k, L, min(8, input_dim), seed)
    elif config.hash_function == "MinHash":
        hf = MinHash(input_dim, k, L, seed)
    else:
        raise NotImplementedError(f"hash family {config.hash_function} is not on the GPU path")
    bt = FIFO if config.bucket_type == "Fifo" else RESERVOIR
    return LshIndex(hf, bt, config.bucket_capacity)


class LshSparsityPredictor:
    """LshSparsityPredictor (crates/klearu-dejavu/src/predictor/lsh_predictor.rs:7-43):
    an LSH index over observed inputs, one entry per (input, important id)."""

    def __init__(self, config: LshConfig, input_dim: int, top_k: int, seed: int):
        self.index = create_lsh_index(config, input_dim, seed)
        self.top_k = top_k

    def build_from_observations(self, observations):
        """clear, then insert each input under each of its important ids, in order (:22-30)."""
        self.index.clear()
        ids, rows = [], []
        for inp, important in observations:
            for i in important:
                ids.append(int(i))
                rows.append(np.asarray(inp, np.float32))
        if ids:
            self.index.insert_batch(np.array(ids, np.uint32), np.stack(rows))

    def predict(self, x):
        """Ids by hit count descending, at most top_k (:33-43)."""
        return self.index.query_top_k(np.asarray(x, np.float32)[None, :], self.top_k)[0]

    def predict_batch(self, X):
        return self.index.query_top_k(X, self.top_k)
