"""On-disk formats: safetensors model weights and predictor JSON files.

Mirrors the reference's readers over the native parsers in libklearu_hip.so:
  SafeTensorsFile   crates/klearu-llm/src/weight/safetensors.rs:24-159
  load_model's file discovery (a directory of *.safetensors)  weight/loader.rs:30-64
  layer naming       weight/name_map.rs:36-98
The open / info / read calls run on the host only; Mlp / SparseAttention
construction from a file uploads the layer's BF16 matrices to the GPU.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import _lib
from ._dev import hptr

DTYPES = {0: "F32", 1: "F16", 2: "BF16"}
_NP = {0: np.float32, 1: np.float16, 2: np.uint16}


@dataclass
class TensorInfo:
    """TensorInfo (safetensors.rs:7-14) without the byte offsets."""
    name: str
    dtype: str
    shape: tuple


class SafeTensorsFile:
    """A memory-mapped safetensors file, or every *.safetensors file of a directory."""

    def __init__(self, path):
        h = C.c_void_p()
        _lib.call("kh_safetensors_open", os.fsencode(path), C.byref(h))
        self._h = h
        self.path = path

    open = classmethod(lambda cls, path: cls(path))

    def close(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            _lib.load().kh_safetensors_close(h)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def names(self) -> list[str]:
        n = C.c_int64()
        _lib.call("kh_safetensors_count", self._h, C.byref(n))
        out = []
        buf = C.create_string_buffer(4096)
        for i in range(n.value):
            _lib.call("kh_safetensors_name", self._h, i, buf, len(buf))
            out.append(buf.value.decode())
        return out

    def info(self, name: str) -> TensorInfo:
        dt, nd = C.c_int(), C.c_int()
        shape = (C.c_int64 * 16)()
        _lib.call("kh_safetensors_info", self._h, name.encode(), C.byref(dt), C.byref(nd), shape, 16)
        return TensorInfo(name, DTYPES[dt.value], tuple(shape[i] for i in range(min(nd.value, 16))))

    def layer_name(self, layer: int, suffix: str) -> str:
        """The file's name for `{prefix}layers.{layer}.{suffix}`, prefix "model.",
        "model.language_model." or "" (name_map.rs:36-49)."""
        names = set(self.names())
        for pre in ("model.layers.", "model.language_model.layers.", "layers."):
            n = f"{pre}{layer}.{suffix}"
            if n in names:
                return n
        raise KeyError(f"missing weight model.layers.{layer}.{suffix}")

    def tensors(self) -> dict[str, TensorInfo]:
        """SafeTensorsFile::tensors (safetensors.rs:114-117)."""
        return {n: self.info(n) for n in self.names()}

    def tensor_data(self, name: str) -> np.ndarray:
        """The raw elements in the file's dtype (BF16 as uint16 bits), shaped."""
        ti = self.info(name)
        code = {v: k for k, v in DTYPES.items()}[ti.dtype]
        a = np.empty(ti.shape, _NP[code])
        _lib.call("kh_safetensors_read_raw", self._h, name.encode(), a.ctypes.data_as(C.c_void_p), a.nbytes)
        return a

    def tensor_to_f32(self, name: str) -> np.ndarray:
        """SafeTensorsFile::tensor_to_f32 (safetensors.rs:135-159), shaped."""
        ti = self.info(name)
        a = np.empty(ti.shape, np.float32)
        _lib.call("kh_safetensors_read_f32", self._h, name.encode(), a.ctypes.data_as(C.c_void_p), a.size)
        return a


class LibSvmDataset:
    """LibSvmDataset (crates/klearu-core/src/data/libsvm.rs:22-200) parsed by
    the native loader.  examples are (SparseVector, labels) pairs; the CSR
    arrays (off, idx, val, label_off, labels) are kept on the host and
    upload(row0, rows) copies a range of examples to the device."""

    def __init__(self, handle):
        self._h = handle
        n, nnz, nl, fd, nlab = (C.c_int64() for _ in range(5))
        _lib.call("kh_libsvm_dims", handle, C.byref(n), C.byref(nnz), C.byref(nl), C.byref(fd), C.byref(nlab))
        self.n, self.feature_dim, self.num_labels = n.value, fd.value, nlab.value
        self.off = np.zeros(self.n + 1, np.int64)
        self.idx = np.zeros(max(nnz.value, 1), np.uint32)
        self.val = np.zeros(max(nnz.value, 1), np.float32)
        self.label_off = np.zeros(self.n + 1, np.int64)
        self.labels = np.zeros(max(nl.value, 1), np.uint32)
        _lib.call("kh_libsvm_copy", handle, hptr(self.off), hptr(self.idx), hptr(self.val), hptr(self.label_off),
                  hptr(self.labels))
        self.idx, self.val, self.labels = self.idx[:nnz.value], self.val[:nnz.value], self.labels[:nl.value]

    @classmethod
    def load(cls, path, feature_dim, num_labels):
        h = C.c_void_p()
        _lib.call("kh_libsvm_load", str(path).encode(), int(feature_dim), int(num_labels), C.byref(h))
        return cls(h)

    @classmethod
    def load_from_bytes(cls, data, feature_dim, num_labels):
        """load_from_reader over an in-memory buffer."""
        data = data.encode() if isinstance(data, str) else bytes(data)
        h = C.c_void_p()
        _lib.call("kh_libsvm_parse", data, len(data), int(feature_dim), int(num_labels), C.byref(h))
        return cls(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib.load().kh_libsvm_free(h)
            except Exception:
                pass

    def __len__(self):
        return self.n

    def get(self, i):
        """Example i: (indices, values, labels)."""
        a, b = self.off[i], self.off[i + 1]
        return self.idx[a:b].copy(), self.val[a:b].copy(), self.labels[self.label_off[i]:self.label_off[i + 1]].tolist()

    def upload(self, row0, rows, stream=None):
        """Examples [row0, row0 + rows) as device CSR (off, idx, val)."""
        import torch
        from ._dev import ptr, stream_ptr
        a, b = int(self.off[row0]), int(self.off[row0 + rows])
        off = torch.empty(rows + 1, dtype=torch.int64, device="cuda")
        idx = torch.empty(max(b - a, 1), dtype=torch.int32, device="cuda")
        val = torch.empty(max(b - a, 1), dtype=torch.float32, device="cuda")
        _lib.call("kh_libsvm_upload", self._h, int(row0), int(rows), ptr(off), ptr(idx), ptr(val), stream_ptr(stream))
        return off, idx, val
