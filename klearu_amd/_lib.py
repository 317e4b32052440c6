"""ctypes binding of libklearu_hip.so (the C ABI in include/klearu_hip.h).

The library is loaded from the package directory.  There is no CPU fallback:
if the library is missing or no GPU is visible, calls raise.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libklearu_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "klearu_hip.h")


class KlearuError(RuntimeError):
    """A negative status from the C ABI; .code holds it."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{code}] {msg}")
        self.code = code


KH_OK, KH_ERR_ARG, KH_ERR_HIP, KH_ERR_CAPACITY, KH_ERR_ALLOC, KH_ERR_UNSUPPORTED = 0, -1, -2, -3, -4, -5


def header_functions(path: str = HEADER) -> list[str]:
    """Names of every function the C header declares."""
    txt = open(path).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(kh_[a-z0-9_]+)\s*\(", txt)) - {"kh_"})


_lib = None

P = C.c_void_p
I = C.c_int
I64 = C.c_int64
U64 = C.c_uint64
F = C.c_float
PP = C.POINTER(C.c_void_p)
S = C.c_char_p

SIGS = {
    "kh_last_error": (C.c_char_p, []),
    "kh_version": (I, []),
    "kh_dense_dot_dense": (I, [P, I64, I64, P, I64, P, P]),
    "kh_expf": (I, [P, P, I64, P]),
    "kh_dejavu_linear_create": (I, [I, I, P, P, PP]),
    "kh_dejavu_linear_destroy": (I, [P]),
    "kh_dejavu_linear_forward": (I, [P, P, I64, P, P]),
    "kh_dejavu_linear_forward_sparse": (I, [P, P, I64, P, I64, P, P]),
    "kh_dejavu_sparse_mlp_create": (I, [I, I, PP]),
    "kh_dejavu_sparse_mlp_destroy": (I, [P]),
    "kh_dejavu_sparse_mlp_forward": (I, [P, P, I64, P, P, P, P, I64, P, P]),
    "kh_dejavu_sparse_attention_create": (I, [I, I, I, PP]),
    "kh_dejavu_sparse_attention_destroy": (I, [P]),
    "kh_dejavu_sparse_attention_forward": (I, [P, P, I64, P, P, P, P, P, I64, P, P]),
    "kh_sparse_dot_dense": (I, [P, P, I64, P, I64, P, P]),
    "kh_scatter_add": (I, [P, P, I64, P, I64, F, P]),
    "kh_bf16_from_f32": (I, [P, P, I64, P]),
    "kh_bf16_to_f32": (I, [P, P, I64, P]),
    "kh_bf16_dot_f32": (I, [P, I64, I64, P, I64, P, P]),
    "kh_bf16_full_dot": (I, [P, P, I64, P, P]),
    "kh_bf16_update_from_f32": (I, [P, P, I64, P]),
    "kh_simhash_create": (I, [I, I, I, U64, PP]),
    "kh_srp_create": (I, [I, I, I, F, U64, PP]),
    "kh_hash_family_from_planes": (I, [I, I, I, P, PP]),
    "kh_hash_family_destroy": (I, [P]),
    "kh_hash_family_dims": (I, [P, C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
    "kh_hash_family_planes": (I, [P, P]),
    "kh_hash_dense": (I, [P, P, I64, P, P]),
    "kh_hash_sparse": (I, [P, P, P, P, I64, P, P]),
    "kh_lsh_index_create": (I, [P, I, I, PP]),
    "kh_lsh_index_destroy": (I, [P]),
    "kh_lsh_index_insert": (I, [P, P, P, I64, I64, P]),
    "kh_lsh_index_insert_codes": (I, [P, P, P, I64, P]),
    "kh_lsh_index_clear": (I, [P, P]),
    "kh_lsh_index_insert_sparse": (I, [P, P, P, P, P, I64, P]),
    "kh_lsh_index_remove_codes": (I, [P, P, P, I64, P]),
    "kh_lsh_index_remove_with_weights": (I, [P, P, P, I64, I64, P]),
    "kh_lsh_index_remove": (I, [P, P, I64, P]),
    "kh_lsh_index_query": (I, [P, P, I64, P, P, P, I64, P]),
    "kh_lsh_index_query_sparse": (I, [P, P, P, P, I64, P, P, P, I64, P]),
    "kh_lsh_index_buckets": (I, [P, P, P, P]),
    "kh_slide_layer_create": (I, [I, I, P, P, P, I, I, I, I, PP]),
    "kh_slide_layer_destroy": (I, [P]),
    "kh_slide_layer_forward": (I, [P, P, I64, P, P, P, P, I64, P]),
    "kh_slide_layer_forward_sparse": (I, [P, P, P, P, I64, P, P, P, P, I64, P]),
    "kh_lsh_index_rebuild": (I, [P, P, P, I64, I64, P]),
    "kh_rebuild_scheduler_init": (None, [P, U64, C.c_double]),
    "kh_rebuild_scheduler_step": (I, [P]),
    "kh_rebuild_scheduler_should_rebuild": (I, [P, U64]),
    "kh_slide_layer_rebuild_index": (I, [P, P]),
    "kh_slide_layer_init_optimizer": (I, [P, I, F, F, F, F]),
    "kh_slide_layer_weights": (I, [P, P, P]),
    "kh_slide_layer_backward": (I, [P, P, P, P, P, P, P, I64, C.c_double, U64, P, P]),
    "kh_slide_network_create": (I, [PP, I, I, F, F, F, F, U64, C.c_double, PP]),
    "kh_slide_network_destroy": (I, [P]),
    "kh_slide_network_train_step": (I, [P, P, I64, P, P, C.c_double, P, P]),
    "kh_slide_network_predict": (I, [P, P, I64, P, P]),
    "kh_slide_network_train_step_sparse": (I, [P, P, P, P, I64, P, P, C.c_double, P, P]),
    "kh_slide_network_predict_sparse": (I, [P, P, P, P, I64, P, P]),
    "kh_slide_network_state": (I, [P, P, P]),
    "kh_libsvm_load": (I, [S, I64, I64, PP]),
    "kh_libsvm_parse": (I, [C.c_char_p, I64, I64, I64, PP]),
    "kh_libsvm_free": (I, [P]),
    "kh_libsvm_dims": (I, [P, P, P, P, P, P]),
    "kh_libsvm_copy": (I, [P, P, P, P, P, P]),
    "kh_libsvm_upload": (I, [P, I64, I64, P, P, P, P]),
    "kh_wta_create": (I, [I, I, I, I, U64, PP]),
    "kh_dwta_create": (I, [I, I, I, I, U64, PP]),
    "kh_wta_from_windows": (I, [I, I, I, I, I, P, PP]),
    "kh_minhash_create": (I, [I, I, I, U64, PP]),
    "kh_minhash_from_permutations": (I, [I, I, I, P, PP]),
    "kh_hash_family_kind": (I, [P, P, P]),
    "kh_hash_family_tables": (I, [P, P]),
    "kh_sparse_inference": (I, [P, P, I64, I64, F, I, P, P, P, I64, P]),
    "kh_lsh_index_query_top_k": (I, [P, P, I64, I64, P, P, P]),
    "kh_dense_layer_create": (I, [I, I, P, P, I, PP]),
    "kh_dense_layer_destroy": (I, [P]),
    "kh_dense_layer_forward_sparse": (I, [P, P, P, P, I64, P, P]),
    "kh_predictor_create": (I, [I, I, I, P, P, P, P, PP]),
    "kh_predictor_destroy": (I, [P]),
    "kh_predictor_status": (I, [P]),
    "kh_stream_read": (I, [P, I64, P, I, P]),
    "kh_predictor_set_spin_limit": (I, [P, I]),
    "kh_predictor_predict": (I, [P, P, I64, P, P]),
    "kh_predictor_select_top_k": (I, [P, P, I64, I, I, P, P]),
    "kh_predictor_select_top_k_noalloc": (I, [P, P, I64, I, I, P, P]),
    "kh_topk_select": (I, [P, I64, I, I, I, P, P]),
    "kh_union_active": (I, [P, I64, I, I, P, P, P]),
    "kh_predictor_select_top_k_union": (I, [P, P, I64, I, P, P, P, P]),
    "kh_sparse_ffn_create": (I, [I, I, P, P, P, I, PP]),
    "kh_sparse_ffn_create_dev": (I, [I, I, P, P, P, I, PP]),
    "kh_sparse_ffn_destroy": (I, [P]),
    "kh_sparse_ffn_forward": (I, [P, P, I64, P, I, P, P, I, P]),
    "kh_sparse_ffn_last_hidden": (I, [P, P, I64, I, P]),
    "kh_sparse_ffn_status": (I, [P]),
    "kh_rmsnorm": (I, [P, P, I64, I, F, P, P]),
    "kh_dejavu_mlp_block": (I, [P, P, P, P, F, I, P, P, P]),
    "kh_dejavu_mlp_block_batch": (I, [P, P, P, I64, P, F, I, P, P, P]),
    "kh_dejavu_attn_block": (I, [P, P, P, P, F, I, P, P, P]),
    "kh_dejavu_attn_block_batch": (I, [P, P, P, I64, P, F, I, P, P, P]),
    "kh_sparse_attn_create": (I, [I, I, I, I, I, I, F, I, P, P, P, P, PP]),
    "kh_sparse_attn_create_dev": (I, [I, I, I, I, I, I, F, I, P, P, P, P, PP]),
    "kh_sparse_attn_destroy": (I, [P]),
    "kh_sparse_attn_load_cache": (I, [P, I64, P, P, I64]),
    "kh_sparse_attn_load_cache_dev": (I, [P, I64, P, P, I64, P]),
    "kh_sparse_attn_read_cache": (I, [P, I64, P, P, I64]),
    "kh_sparse_attn_cache_len": (I, [P, I64, P]),
    "kh_sparse_attn_clear": (I, [P, P]),
    "kh_sparse_attn_forward": (I, [P, P, I64, P, P, I, P, I, P]),
    "kh_safetensors_open": (I, [S, PP]),
    "kh_safetensors_close": (I, [P]),
    "kh_safetensors_count": (I, [P, C.POINTER(I64)]),
    "kh_safetensors_name": (I, [P, I64, C.c_char_p, I64]),
    "kh_safetensors_info": (I, [P, S, C.POINTER(I), C.POINTER(I), P, I]),
    "kh_safetensors_read_f32": (I, [P, S, P, I64]),
    "kh_safetensors_read_raw": (I, [P, S, P, I64]),
    "kh_sparse_ffn_create_from_safetensors": (I, [P, I, I, PP]),
    "kh_sparse_attn_create_from_safetensors": (I, [P, I, I, I, I, I, I, F, I, PP]),
    "kh_predictor_load": (I, [S, PP]),
    "kh_predictor_read_json": (I, [S, C.POINTER(I), C.POINTER(I), C.POINTER(I), P, P, P, P]),
    "kh_predictor_write_json": (I, [S, I, I, I, P, P, P, P]),
    "kh_predictor_save": (I, [P, S]),
    "kh_predictor_dims": (I, [P, C.POINTER(I), C.POINTER(I), C.POINTER(I)]),
    "kh_predictor_weights": (I, [P, P, P, P, P]),
}


def load() -> C.CDLL:
    """Load the library (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} not built: run `python -m klearu_amd.build` "
                           "(or __graft_entry__.build()) first; there is no CPU fallback")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGS.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def call(name: str, *args) -> int:
    """Call an entry point; raise KlearuError on a negative status."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc < 0:
        raise KlearuError(rc, lib.kh_last_error().decode(errors="replace"))
    return rc
