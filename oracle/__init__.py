"""ctypes view of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` -- as the checker, or as the timed CPU port of
the reference.  The product package ``klearu_amd`` never imports this module.

Each wrapper converts numpy arrays and calls the C restatement in ``oracle.c`` /
``oracle_avx2.c``; the reference citations live there.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "liboracle.so")


def build(force: bool = False) -> str:
    """Compile liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE, "-B" if force else "all"], check=True)
    return _SO


def _load() -> C.CDLL:
    if not os.path.exists(_SO):
        build()
    return C.CDLL(_SO)


lib = _load()

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i64 = C.c_int64
_int = C.c_int
_f = C.c_float


def _sig(name, res, *args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_sig("or_dense_dot_avx2_order", _f, _f32p, _f32p, _i64)
_sig("or_dense_dot_scalar", _f, _f32p, _f32p, _i64)
_sig("or_avx2_dense_dot", _f, _f32p, _f32p, _i64)
_sig("or_sparse_dot_dense_avx2_order", _f, _u32p, _f32p, _i64, _f32p)
_sig("or_sparse_dot_dense_scalar", _f, _u32p, _f32p, _i64, _f32p)
_sig("or_avx2_sparse_dot_dense", _f, _u32p, _f32p, _i64, _f32p)
_sig("or_scatter_add", None, _u32p, _f32p, _i64, _f32p, _f)
_sig("or_bf16_from_f32", C.c_uint16, _f)
_sig("or_bf16_to_f32", _f, C.c_uint16)
_sig("or_bf16_from_f32_n", None, _f32p, _u16p, _i64)
_sig("or_bf16_dot_f32", _f, _u16p, _f32p, _i64)
_sig("or_bf16_full_dot", _f, _u16p, _u16p, _i64)
_sig("or_bf16_update_from_f32", None, _u16p, _f32p, _i64)
_sig("or_expf_n", None, _f32p, _f32p, _i64)
_sig("or_chacha_block", None, _u32p, _int, _u32p)
_sig("or_pcg32_output", C.c_uint32, C.c_uint64)
_sig("or_simhash_planes", None, _int, _int, _int, C.c_uint64, _i8p)
_sig("or_srp_planes", None, _int, _int, _int, _f, C.c_uint64, _i8p)
_sig("or_hash_dense", C.c_uint64, _i8p, _int, _int, _int, _f32p)
_sig("or_hash_sparse", C.c_uint64, _i8p, _int, _int, _int, _u32p, _f32p, _i64)
_sig("or_hash_dense_batch", None, _i8p, _int, _int, _int, _f32p, _i64, _u32p)
_sig("or_reservoir_rand", C.c_uint64, C.c_uint64, C.c_uint64)
_sig("or_lsh_insert_many", None, _int, _int, _int, _int, _u32p, _u32p, _u64p, _i64, _u32p, _u32p)
_sig("or_lsh_remove_many", None, _int, _int, _int, _u32p, _u32p, _i64, _u32p, _u32p)
_sig("or_lsh_remove_all", None, _int, _int, _int, _u32p, _u32p, _i64, _u32p)
_sig("or_lsh_query", _i64, _int, _int, _int, _u32p, _u32p, _u32p, _u32p, _u32p)
_sig("or_sample_topk", _i64, _u32p, _u32p, _i64, _i64, _u32p)
_sig("or_sample_threshold", _i64, _u32p, _u32p, _i64, C.c_uint32, _u32p)
_sig("or_neuron_forward", _f, _f32p, _f, _f32p, _i64)
_sig("or_neuron_forward_sparse", _f, _f32p, _f, _u32p, _f32p, _i64)
_sig("or_layer_activate", None, _f32p, _i64, _int, _f32p)
_sig("or_predictor_predict", None, _f32p, _f32p, _f32p, _f32p, _int, _int, _int, _f32p, _f32p, _f32p)
_sig("or_predictor_predict_bf16", None, _u16p, _f32p, _u16p, _f32p, _int, _int, _int, _f32p, _f32p,
     _f32p)
_sig("or_select_top_k", None, _f32p, _i64, _i64, _i64p)
_sig("or_sigmoid", _f, _f)
_sig("or_silu", _f, _f)
_sig("or_sparse_mlp_forward_bf16", None, _u16p, _u16p, _u16p, _int, _int, _f32p, _i64p, _i64, _f32p,
     _f32p)
_sig("or_rms_inv", _f, _f32p, _i64, _f)
_sig("or_rmsnorm", None, _f32p, _f32p, _i64, _f)
_sig("or_rope_tables", None, _int, _int, _f, _f32p, _f32p)
_sig("or_rope_apply", None, _f32p, _int, _f32p, _f32p, _i64)
_sig("or_linear_forward_bf16", None, _u16p, _int, _int, _f32p, _f32p)
_sig("or_sparse_attention_forward_bf16", None, _u16p, _u16p, _u16p, _u16p, _int, _int, _int, _int,
     _f32p, _i64, _f32p, _f32p, _f32p, _f32p, _i64, _i64p, _i64, _f32p)
_sig("or_dejavu_linear_forward_sparse", None, _f32p, _f32p, _int, _f32p, _i64p, _i64, _f32p)
_sig("or_dejavu_sparse_mlp_forward", None, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _int, _int,
     _f32p, _i64p, _i64, _f32p)
_sig("or_dejavu_linear_forward", None, _f32p, _f32p, _int, _int, _f32p, _f32p)
_sig("or_dejavu_sparse_attention_forward", None, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p, _f32p,
     _int, _int, _int, _f32p, _i64p, _i64, _f32p)
_sig("or_cpu_dejavu_ffn_layer", None, _f32p, _f32p, _f32p, _f32p, _f, _f32p, _f32p, _f32p, _f32p, _int,
     _int, _int, _i64, _f32p, _f32p, _i64p)

_sig("or_cpu_sparse_attention_layer", None, _f32p, _f32p, _f32p, _f32p, _f32p, _f, _f32p, _f32p, _f32p,
     _f32p, _int, _int, _int, _int, _int, _i64, _f32p, _f32p, _f32p, _f32p, _i64, _i64, _f32p, _f32p,
     _i64p)
_sig("or_slide_forward", _i64, _i8p, _int, _int, _int, _int, _u32p, _u32p, _f32p, _f32p, _int, _f32p,
     _int, _int, _int, _int, _u32p, _f32p, _f32p)

_sig("or_slide_forward_ordered", _i64, _i8p, _int, _int, _int, _int, _u32p, _u32p, _f32p, _f32p, _int,
     _f32p, _int, _int, _int, _int, _u32p, _f32p, _f32p)
_sig("or_powi_f32", _f, _f, C.c_int32)
_sig("or_sgd_update", None, _f32p, _f32p, _i64, _f32p, _f, C.c_double, _f, _f32p, _f32p)
_sig("or_adam_update", None, _f32p, _f32p, _i64, _f32p, _f, C.c_double, C.c_uint64, _f, _f, _f, _f32p,
     _f32p, _f32p, _f32p)
_sig("or_activation_derivative", _f, _f, _f, _int)
_sig("or_softmax_local_grads", None, _f32p, _f32p, _i64, _f32p)
_sig("or_compute_loss", _f, _f32p, _u32p, _i64, _u32p, _i64)
_sig("or_compute_loss_gradient", None, _f32p, _u32p, _i64, _u32p, _i64, _i64, _f32p)
_sig("or_layer_backward", None, _f32p, _f32p, _int, _int, _int, _f32p, _u32p, _i64, _f32p, _f32p, _f32p,
     _i64, _int, _f, _f, _f, _f, _f32p, _f32p, _f32p, _f32p, C.c_double, C.c_uint64, C.c_void_p)

_sig("or_compiler_version", C.c_char_p)
_sig("or_cpu_rank_hash_batch", None, _int, _u32p, _int, _int, _int, _int, _f32p, _i64, _u64p)
_sig("or_cpu_bolt_batch", _i64, _i8p, _int, _int, _int, _int, _u32p, _u32p, _f32p, _f32p, _f32p, _i64, _int,
     _int, _i64p, _f32p)
_sig("or_cpu_lsh_topk_batch", None, _i8p, _int, _int, _int, _int, _u32p, _u32p, _f32p, _i64, _int, _i64p,
     _u32p)

ACT = {"relu": 0, "sigmoid": 1, "tanh": 2, "softmax": 3, "identity": 4}
FIFO, RESERVOIR = 0, 1


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def i64(a):
    return np.ascontiguousarray(a, dtype=np.int64)


# --------------------------------------------------------------------------- accel
def dense_dot(a, b):
    a, b = f32(a), f32(b)
    return np.float32(lib.or_dense_dot_avx2_order(a, b, a.size))


def dense_dot_avx2(a, b):
    a, b = f32(a), f32(b)
    return np.float32(lib.or_avx2_dense_dot(a, b, a.size))


def dense_dot_scalar(a, b):
    a, b = f32(a), f32(b)
    return np.float32(lib.or_dense_dot_scalar(a, b, a.size))


def sparse_dot_dense(idx, val, dense):
    idx, val, dense = u32(idx), f32(val), f32(dense)
    return np.float32(lib.or_sparse_dot_dense_avx2_order(idx, val, idx.size, dense))


def sparse_dot_dense_avx2(idx, val, dense):
    idx, val, dense = u32(idx), f32(val), f32(dense)
    return np.float32(lib.or_avx2_sparse_dot_dense(idx, val, idx.size, dense))


def sparse_dot_dense_scalar(idx, val, dense):
    idx, val, dense = u32(idx), f32(val), f32(dense)
    return np.float32(lib.or_sparse_dot_dense_scalar(idx, val, idx.size, dense))


def scatter_add(idx, val, dense, scale):
    idx, val = u32(idx), f32(val)
    out = f32(dense).copy()
    lib.or_scatter_add(idx, val, idx.size, out, float(scale))
    return out


def bf16_from_f32(x):
    x = f32(x)
    out = np.empty(x.shape, np.uint16)
    lib.or_bf16_from_f32_n(x.ravel(), out.reshape(-1), x.size)
    return out


def bf16_to_f32(b):
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_dot_f32(w, x):
    w, x = np.ascontiguousarray(w, np.uint16), f32(x)
    return np.float32(lib.or_bf16_dot_f32(w, x, w.size))


def bf16_full_dot(a, b):
    a, b = np.ascontiguousarray(a, np.uint16), np.ascontiguousarray(b, np.uint16)
    return np.float32(lib.or_bf16_full_dot(a, b, a.size))


def expf(x):
    """glibc expf of every element (float32 in, float32 out)."""
    x = f32(x)
    y = np.empty_like(x)
    lib.or_expf_n(x.reshape(-1), y.reshape(-1), x.size)
    return y


def bf16_update_from_f32(w, delta):
    w = np.ascontiguousarray(w, np.uint16).copy()
    lib.or_bf16_update_from_f32(w, f32(delta), w.size)
    return w


# --------------------------------------------------------------------------- rng / hash
def chacha_block(words16, rounds):
    inp = u32(words16)
    out = np.zeros(16, np.uint32)
    lib.or_chacha_block(inp, rounds, out)
    return out


def simhash_planes(dim, k, num_tables, seed):
    p = np.empty(num_tables * k * dim, np.int8)
    lib.or_simhash_planes(dim, k, num_tables, seed, p)
    return p.reshape(num_tables, k, dim)


def srp_planes(dim, k, num_tables, sparsity, seed):
    p = np.empty(num_tables * k * dim, np.int8)
    lib.or_srp_planes(dim, k, num_tables, float(sparsity), seed, p)
    return p.reshape(num_tables, k, dim)


def hash_dense(planes, x, table):
    L, k, dim = planes.shape
    return int(lib.or_hash_dense(np.ascontiguousarray(planes).reshape(-1), dim, k, table, f32(x)))


def hash_sparse(planes, idx, val, table):
    L, k, dim = planes.shape
    idx, val = u32(idx), f32(val)
    return int(lib.or_hash_sparse(np.ascontiguousarray(planes).reshape(-1), dim, k, table, idx, val,
                                  idx.size))


def hash_dense_batch(planes, X):
    L, k, dim = planes.shape
    X = f32(X).reshape(-1, dim)
    codes = np.zeros((X.shape[0], L), np.uint32)
    lib.or_hash_dense_batch(np.ascontiguousarray(planes).reshape(-1), dim, k, L, X.reshape(-1),
                            X.shape[0], codes.reshape(-1))
    return codes


class LshIndex:
    """Dense bucket tables [L][2^K][cap] filled by the reference insert rules."""

    def __init__(self, num_tables, k, cap, bucket_type):
        self.L, self.k, self.cap, self.type = num_tables, k, cap, bucket_type
        nb = 1 << k
        self.data = np.zeros(num_tables * nb * cap, np.uint32)
        self.len = np.zeros(num_tables * nb, np.uint32)
        self.count = np.zeros(num_tables * nb, np.uint64)

    def insert_many(self, ids, codes):
        ids, codes = u32(ids), u32(codes).reshape(-1)
        lib.or_lsh_insert_many(self.L, self.k, self.cap, self.type, self.data, self.len, self.count,
                               ids.size, ids, codes)

    def remove_many(self, ids, codes):
        """remove_with_weights for each (id, codes row) in order (lsh/index.rs:271-276)."""
        ids, codes = u32(ids), u32(codes).reshape(-1)
        lib.or_lsh_remove_many(self.L, self.k, self.cap, self.data, self.len, ids.size, ids, codes)

    def remove_all(self, ids):
        """remove for each id in order: every bucket drops the id (lsh/index.rs:278-280)."""
        ids = u32(ids)
        lib.or_lsh_remove_all(self.L, self.k, self.cap, self.data, self.len, ids.size, ids)

    def query(self, codes):
        codes = u32(codes).reshape(-1)
        ids = np.zeros(self.L * self.cap + 1, np.uint32)
        cnt = np.zeros(self.L * self.cap + 1, np.uint32)
        n = lib.or_lsh_query(self.L, self.k, self.cap, self.data, self.len, codes, ids, cnt)
        return ids[:n].copy(), cnt[:n].copy()

    def bucket(self, t, b):
        nb = 1 << self.k
        s = t * nb + b
        return self.data[s * self.cap: s * self.cap + int(self.len[s])].copy()


def sample_topk(ids, counts, k):
    ids, counts = u32(ids), u32(counts)
    out = np.zeros(max(ids.size, 1), np.uint32)
    n = lib.or_sample_topk(ids, counts, ids.size, k, out)
    return out[:n].copy()


def sample_threshold(ids, counts, t):
    ids, counts = u32(ids), u32(counts)
    out = np.zeros(max(ids.size, 1), np.uint32)
    n = lib.or_sample_threshold(ids, counts, ids.size, t, out)
    return out[:n].copy()


# --------------------------------------------------------------------------- SLIDE
def neuron_forward(w, b, x):
    w, x = f32(w), f32(x)
    return np.float32(lib.or_neuron_forward(w, float(b), x, w.size))


def neuron_forward_sparse(w, b, idx, val):
    w, idx, val = f32(w), u32(idx), f32(val)
    return np.float32(lib.or_neuron_forward_sparse(w, float(b), idx, val, idx.size))


def layer_activate(pre, act):
    pre = f32(pre)
    out = np.zeros_like(pre)
    lib.or_layer_activate(pre, pre.size, ACT[act] if isinstance(act, str) else act, out)
    return out


# --------------------------------------------------------------------------- Deja Vu
def predictor_predict(w1, b1, w2, b2, x):
    hid, ind = w1.shape
    out = w2.shape[0]
    scores = np.zeros(out, np.float32)
    h = np.zeros(hid, np.float32)
    if w1.dtype == np.uint16:
        lib.or_predictor_predict_bf16(np.ascontiguousarray(w1).reshape(-1), f32(b1),
                                      np.ascontiguousarray(w2).reshape(-1), f32(b2), ind, hid, out,
                                      f32(x), scores, h)
    else:
        lib.or_predictor_predict(f32(w1).reshape(-1), f32(b1), f32(w2).reshape(-1), f32(b2), ind,
                                 hid, out, f32(x), scores, h)
    return scores, h


def select_top_k(scores, k):
    scores = f32(scores)
    m = min(k, scores.size)
    out = np.zeros(max(m, 1), np.int64)
    lib.or_select_top_k(scores, scores.size, k, out)
    return out[:m].copy()


def sparse_mlp_forward_bf16(wg, wu, wd, x, active):
    inter, hidden = wg.shape
    active = i64(active)
    y = np.zeros(hidden, np.float32)
    h = np.zeros(max(active.size, 1), np.float32)
    lib.or_sparse_mlp_forward_bf16(np.ascontiguousarray(wg).reshape(-1),
                                   np.ascontiguousarray(wu).reshape(-1),
                                   np.ascontiguousarray(wd).reshape(-1), hidden, inter, f32(x),
                                   active, active.size, y, h)
    return y, h[:active.size].copy()


def rms_inv(x, eps):
    """RmsNorm's scale 1/rms of one row (rms_norm.rs:48-52), as an f32."""
    x = f32(x)
    return np.float32(lib.or_rms_inv(x, x.size, float(eps)))


def rmsnorm(x, w, eps):
    x = f32(x).copy()
    lib.or_rmsnorm(x, f32(w), x.size, float(eps))
    return x


def rope_tables(head_dim, max_seq, theta):
    c = np.zeros(max_seq * (head_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib.or_rope_tables(head_dim, max_seq, float(theta), c, s)
    return c, s


def linear_forward_bf16(w, x):
    out_f, in_f = w.shape
    y = np.zeros(out_f, np.float32)
    lib.or_linear_forward_bf16(np.ascontiguousarray(w).reshape(-1), out_f, in_f, f32(x), y)
    return y


def sparse_attention_forward_bf16(wq, wk, wv, wo, num_heads, num_kv_heads, head_dim, x, pos, cos_t,
                                  sin_t, k_cache, v_cache, heads):
    """k_cache/v_cache: float32 [kv_heads][max_seq][d], modified in place (row pos appended)."""
    hidden = wq.shape[1]
    max_seq = k_cache.shape[1]
    out = np.zeros(hidden, np.float32)
    heads = i64(heads)
    lib.or_sparse_attention_forward_bf16(
        np.ascontiguousarray(wq).reshape(-1), np.ascontiguousarray(wk).reshape(-1),
        np.ascontiguousarray(wv).reshape(-1), np.ascontiguousarray(wo).reshape(-1), hidden,
        num_heads, num_kv_heads, head_dim, f32(x), pos, cos_t, sin_t, k_cache.reshape(-1),
        v_cache.reshape(-1), max_seq, heads, heads.size, out)
    return out


def dejavu_sparse_mlp_forward(wg, bg, wu, bu, wd, bd, x, sel):
    inter, hidden = wg.shape
    sel = i64(sel)
    y = np.zeros(hidden, np.float32)
    lib.or_dejavu_sparse_mlp_forward(f32(wg).reshape(-1), f32(bg), f32(wu).reshape(-1), f32(bu),
                                     f32(wd).reshape(-1), f32(bd), hidden, inter, f32(x), sel,
                                     sel.size, y)
    return y


def dejavu_linear_forward(w, b, x):
    out_f, in_f = w.shape
    y = np.zeros(out_f, np.float32)
    lib.or_dejavu_linear_forward(f32(w).reshape(-1), f32(b), in_f, out_f, f32(x), y)
    return y


def dejavu_linear_forward_sparse(w, b, x, idx):
    idx = i64(idx)
    y = np.zeros(max(idx.size, 1), np.float32)
    lib.or_dejavu_linear_forward_sparse(f32(w).reshape(-1), f32(b), w.shape[1], f32(x), idx, idx.size, y)
    return y[:idx.size].copy()


def dejavu_sparse_attention_forward(wq, bq, wk, bk, wv, bv, wo, bo, num_heads, head_dim, x, heads):
    hidden = wq.shape[1]
    heads = i64(heads)
    y = np.zeros(hidden, np.float32)
    lib.or_dejavu_sparse_attention_forward(f32(wq).reshape(-1), f32(bq), f32(wk).reshape(-1), f32(bk),
                                           f32(wv).reshape(-1), f32(bv), f32(wo).reshape(-1), f32(bo), hidden,
                                           num_heads, head_dim, f32(x), heads, heads.size, y)
    return y


def slide_layer_oracle(planes, cap, bucket_type, W, b, X, sampling=0, top_k=0, threshold=2, act="relu",
                       index=None):
    """Build the index like Layer::new (neurons 0..n-1 in order) and run
    Layer::forward for every row of X.  Returns a list of (ids, pre, act)."""
    L, k, dim = planes.shape
    W = f32(W)
    n = W.shape[0]
    if index is None:
        index = LshIndex(L, k, cap, bucket_type)
        index.insert_many(np.arange(n, dtype=np.uint32), hash_dense_batch(planes, W))
    pl = np.ascontiguousarray(planes).reshape(-1)
    m = max(n, L * cap) + 1
    out = []
    for x in f32(X).reshape(-1, dim):
        ids = np.zeros(m, np.uint32)
        pre = np.zeros(m, np.float32)
        a_ = np.zeros(m, np.float32)
        cnt = lib.or_slide_forward(pl, dim, k, L, cap, index.data, index.len, W.reshape(-1), f32(b), n,
                                   np.ascontiguousarray(x), sampling, top_k, threshold,
                                   ACT[act] if isinstance(act, str) else act, ids, pre, a_)
        out.append((ids[:cnt].copy(), pre[:cnt].copy(), a_[:cnt].copy()))
    return out, index


# --------------------------------------------------------------------------- SLIDE training
SGD, ADAM = 0, 1
_U64_MAX = (1 << 64) - 1


def powi_f32(a, b):
    return float(np.float32(lib.or_powi_f32(float(np.float32(a)), int(b))))


def sgd_update(w, gw, bias, gb, lr, momentum=0.0, mw=None, mb=None):
    """In place on w (f32 array), mw; returns (bias, mb) (optim/sgd.rs:18-57)."""
    b = np.array([bias], np.float32)
    mbv = np.array([0.0 if mb is None else mb], np.float32)
    if mw is None:
        mw = np.zeros_like(w)
    lib.or_sgd_update(w, f32(gw), w.size, b, float(np.float32(gb)), float(lr), float(np.float32(momentum)), mw, mbv)
    return float(b[0]), float(mbv[0])


def adam_update(w, gw, bias, gb, lr, step, m_w, v_w, m_b, v_b, beta1=0.9, beta2=0.999, eps=1e-8):
    """In place on w, m_w, v_w; returns (bias, m_b, v_b) (optim/adam.rs:28-77)."""
    b = np.array([bias], np.float32)
    mb = np.array([m_b], np.float32)
    vb = np.array([v_b], np.float32)
    lib.or_adam_update(w, f32(gw), w.size, b, float(np.float32(gb)), float(lr), int(step), float(np.float32(beta1)),
                       float(np.float32(beta2)), float(np.float32(eps)), m_w, v_w, mb, vb)
    return float(b[0]), float(mb[0]), float(vb[0])


def softmax_local_grads(s, go):
    s, go = f32(s), f32(go)
    out = np.zeros(max(s.size, 1), np.float32)
    lib.or_softmax_local_grads(s, go, s.size, out)
    return out[:s.size].copy()


def compute_loss(act_dense, active, labels):
    return float(lib.or_compute_loss(f32(act_dense), u32(active), u32(active).size, u32(labels), u32(labels).size))


def compute_loss_gradient(act_dense, active, labels, num_output):
    g = np.zeros(max(num_output, 1), np.float32)
    lib.or_compute_loss_gradient(f32(act_dense), u32(active), u32(active).size, u32(labels), u32(labels).size,
                                 num_output, g)
    return g[:num_output].copy()


class RebuildScheduler:
    """RebuildScheduler (lsh/maintenance.rs:20-98) in Python integers: the
    interval after the i-th rebuild is (usize)(base * exp(decay * i)) -- f64
    exp, truncation toward zero, saturating at 0 and 2^64-1 as `as usize` does
    -- at least 1, and the step sum wraps modulo 2^64 (release arithmetic).
    Pinned: the reference's own scheduler tests (maintenance.rs:103-207)."""

    def __init__(self, base_interval, decay):
        self.base_interval, self.decay = int(base_interval), float(decay)
        self.rebuild_count, self.next_rebuild_step, self.current_step = 0, int(base_interval), 0

    def _interval(self):
        import math
        v = float(self.base_interval) * math.exp(self.decay * float(self.rebuild_count))
        if v != v or v <= 0.0:
            n = 0
        elif v >= 18446744073709551616.0:
            n = _U64_MAX
        else:
            n = int(v)
        return max(n, 1)

    def _due(self):
        if self.current_step >= self.next_rebuild_step:
            self.rebuild_count += 1
            self.next_rebuild_step = (self.current_step + self._interval()) & _U64_MAX
            return True
        return False

    def step(self):
        self.current_step = (self.current_step + 1) & _U64_MAX
        return self._due()

    def should_rebuild(self, step):
        self.current_step = int(step) & _U64_MAX
        return self._due()


class SlideNetOracle:
    """Network (network/net.rs:10-230) over explicit layer weights, each layer an
    LSH index built like Layer::new (neurons 0..n-1 in order).  Forward lists
    active neurons in the sampler's order (or_slide_forward_ordered).

    layers: dicts with planes [L][k][dim] int8, cap, bucket_type, W [n][dim],
    b [n], sampling, top_k, threshold, act."""

    def __init__(self, layers, optimizer=SGD, momentum=0.9, beta1=0.9, beta2=0.999, eps=1e-8,
                 rebuild_base=100, rebuild_decay=0.1):
        self.layers = []
        for spec in layers:
            l = dict(spec)
            l["W"] = f32(spec["W"]).copy()
            l["b"] = f32(spec["b"]).copy()
            n, dim = l["W"].shape
            L, k, _ = l["planes"].shape
            l["n"], l["dim"], l["L"], l["k"] = n, dim, L, k
            l["act"] = ACT[l["act"]] if isinstance(l["act"], str) else l["act"]
            l["pl"] = np.ascontiguousarray(l["planes"]).reshape(-1)
            l["index"] = LshIndex(L, k, l["cap"], l["bucket_type"])
            l["st_w1"] = np.zeros(n * dim, np.float32)
            l["st_w2"] = np.zeros(n * dim, np.float32)
            l["st_b1"] = np.zeros(n, np.float32)
            l["st_b2"] = np.zeros(n, np.float32)
            self.layers.append(l)
            if spec.get("index") is not None:
                # a prebuilt index (e.g. downloaded from the GPU, whose buckets
                # the tests pin bit-exact): data [L][2^K][cap], len, count
                d, ln, cnt = spec["index"]
                l["index"].data[:] = np.ascontiguousarray(d, np.uint32).reshape(-1)
                l["index"].len[:] = np.ascontiguousarray(ln, np.uint32).reshape(-1)
                l["index"].count[:] = np.ascontiguousarray(cnt, np.uint64).reshape(-1)
            else:
                self.rebuild_layer(l)
        self.opt, self.momentum, self.beta1, self.beta2, self.eps = optimizer, momentum, beta1, beta2, eps
        self.step = 0
        self.scheduler = RebuildScheduler(rebuild_base, rebuild_decay)

    @staticmethod
    def rebuild_layer(l):
        """Layer::rebuild_index (layer.rs:228-233): clear, insert 0..n-1 in order."""
        idx = l["index"]
        idx.data[:] = 0
        idx.len[:] = 0
        idx.count[:] = 0
        idx.insert_many(np.arange(l["n"], dtype=np.uint32), hash_dense_batch(l["planes"], l["W"]))

    def layer_forward(self, l, x):
        m = max(l["n"], l["L"] * l["cap"]) + 1
        ids = np.zeros(m, np.uint32)
        pre = np.zeros(m, np.float32)
        a_ = np.zeros(m, np.float32)
        cnt = lib.or_slide_forward_ordered(l["pl"], l["dim"], l["k"], l["L"], l["cap"], l["index"].data,
                                           l["index"].len, l["W"].reshape(-1), l["b"], l["n"],
                                           np.ascontiguousarray(f32(x)), l["sampling"], l["top_k"],
                                           l["threshold"], l["act"], ids, pre, a_)
        dense = np.zeros(l["n"], np.float32)
        dense[ids[:cnt]] = a_[:cnt]
        return ids[:cnt].copy(), pre[:cnt].copy(), dense

    def forward(self, x):
        """Network::forward (net.rs:62-78): per layer (ids, pre, dense activations)."""
        outs, cur = [], f32(x)
        for l in self.layers:
            o = self.layer_forward(l, cur)
            outs.append(o)
            cur = o[2]
        return outs

    def predict(self, x):
        return self.forward(x)[-1][2]

    def layer_backward(self, l, x, out, grad_out, lr, want_grad_in=True):
        ids, pre, dense = out
        gi = np.zeros(l["dim"], np.float32) if want_grad_in else None
        lib.or_layer_backward(l["W"].reshape(-1), l["b"], l["dim"], l["n"], l["act"], np.ascontiguousarray(f32(x)),
                              u32(ids), ids.size, f32(pre), dense, f32(grad_out), grad_out.size, self.opt,
                              float(np.float32(self.momentum)), float(np.float32(self.beta1)),
                              float(np.float32(self.beta2)), float(np.float32(self.eps)), l["st_w1"], l["st_w2"],
                              l["st_b1"], l["st_b2"], float(lr), int(self.step),
                              gi.ctypes.data if gi is not None else None)
        return gi

    def train_step(self, X, labels, lr):
        """Network::train_step (net.rs:81-120); labels: one id list per row."""
        X = f32(X)
        if X.shape[0] == 0:
            return 0.0
        total = np.float32(0.0)
        for x, lab in zip(X, labels):
            outs = self.forward(x)
            ids, _, dense = outs[-1]
            total = np.float32(total + np.float32(compute_loss(dense, ids, lab)))
            grad = compute_loss_gradient(dense, ids, lab, self.layers[-1]["n"])
            for i in range(len(self.layers) - 1, -1, -1):
                inp = x if i == 0 else outs[i - 1][2]
                grad = self.layer_backward(self.layers[i], inp, outs[i], grad, lr)
        self.step += 1
        if self.scheduler.should_rebuild(self.step):
            for l in self.layers:
                self.rebuild_layer(l)
        return float(np.float32(total / np.float32(X.shape[0])))


# --------------------------------------------------------------------------- WTA / DWTA / MinHash
class _Rng(C.Structure):
    _fields_ = [("key", C.c_uint32 * 8), ("counter", C.c_uint64), ("buf", C.c_uint32 * 64), ("idx", C.c_int)]


_sig("or_stdrng_seed_from_u64", None, C.c_void_p, C.c_uint64)
_sig("or_stdrng_next_u32", C.c_uint32, C.c_void_p)
_sig("or_rand_gen_range_u32", C.c_uint32, C.c_void_p, C.c_uint32)
_sig("or_rand_shuffle_u32", None, C.c_void_p, _u32p, _i64)
_sig("or_wta_windows", None, _int, _int, _int, _int, C.c_uint64, _u32p)
_sig("or_minhash_perms", None, _int, _int, C.c_uint64, _u32p)
_sig("or_wta_bits", _int, _int)
_sig("or_wta_hash_dense", C.c_uint64, _u32p, _int, _int, _int, _f32p)
_sig("or_siphash", C.c_uint64, _int, _int, C.c_uint64, C.c_uint64, C.c_char_p, _i64)
_sig("or_dwta_fallback", C.c_uint32, C.c_uint64, C.c_uint64, _int)
_sig("or_dwta_hash_sparse", C.c_uint64, _u32p, _int, _int, _int, _u32p, _f32p, _i64)
_sig("or_minhash_hash", C.c_uint64, _u32p, _int, _int, _int, _u32p, _i64)


class StdRng:
    """rand 0.8.5 StdRng restated in oracle.c (u32 stream and gen_range / shuffle)."""

    def __init__(self, seed):
        self._s = C.create_string_buffer(4096)   # larger than the C struct
        lib.or_stdrng_seed_from_u64(C.cast(self._s, C.c_void_p), int(seed))

    def next_u32(self):
        return int(lib.or_stdrng_next_u32(C.cast(self._s, C.c_void_p)))

    def gen_range(self, n):
        return int(lib.or_rand_gen_range_u32(C.cast(self._s, C.c_void_p), int(n)))

    def shuffle(self, a):
        a = u32(a).copy()
        lib.or_rand_shuffle_u32(C.cast(self._s, C.c_void_p), a, a.size)
        return a


def wta_windows(dim, k, L, ws, seed):
    w = np.zeros(L * k * ws, np.uint32)
    lib.or_wta_windows(dim, k, L, ws, seed, w)
    return w.reshape(L, k, ws)


def minhash_perms(dim, L, seed):
    p = np.zeros(L * dim, np.uint32)
    lib.or_minhash_perms(dim, L, seed, p)
    return p.reshape(L, dim)


def wta_hash_dense(windows, x, table):
    L, k, ws = windows.shape
    return int(lib.or_wta_hash_dense(np.ascontiguousarray(windows, np.uint32).reshape(-1), k, ws, table, f32(x)))


def dwta_hash_sparse(windows, idx, val, table):
    L, k, ws = windows.shape
    idx, val = u32(idx), f32(val)
    return int(lib.or_dwta_hash_sparse(np.ascontiguousarray(windows, np.uint32).reshape(-1), k, ws, table,
                                       idx, val, idx.size))


def siphash(c, d, k0, k1, msg):
    return int(lib.or_siphash(c, d, k0, k1, bytes(msg), len(msg)))


def minhash_hash(perms, k, table, nz):
    L, dim = perms.shape
    nz = u32(nz)
    return int(lib.or_minhash_hash(np.ascontiguousarray(perms, np.uint32).reshape(-1), dim, k, table, nz, nz.size))


def minhash_hash_dense(perms, k, table, x):
    return minhash_hash(perms, k, table, np.nonzero(f32(x) != 0.0)[0].astype(np.uint32))
