#!/usr/bin/env python3
"""Writes the golden fixtures under tests/golden/.

  kats.json     the reference's own known answers, as data: the inputs and
                expected outputs its inline unit tests assert (file:line of
                each in "source").
  vectors.npz   small seeded cases for every function on the path, with the
                CPU oracle's outputs (oracle/, a C restatement of the
                reference's arithmetic whose pinning the oracle tests hold).

Run from the repository root:  python tests/golden/make_golden.py
The fixtures are checked in; tests/test_golden.py checks that the oracle still
reproduces them (CPU) and that the HIP library matches them (GPU).
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle as orc  # noqa: E402

FIFO, RES = 0, 1

KATS = {
    "sparse_dot": {"source": "crates/klearu-accel/src/simd/mod.rs:365-389, :405-425",
                   "cases": [{"dense": [1.0, 2.0, 3.0, 4.0, 5.0], "indices": [0, 2, 4],
                              "values": [1.0, 1.0, 1.0], "expect": 9.0},
                             {"dense": [10.0, 20.0, 30.0, 40.0], "indices": [1, 3],
                              "values": [0.5, 0.25], "expect": 20.0},
                             {"dense": [1.0, 2.0, 3.0], "indices": [], "values": [], "expect": 0.0},
                             {"dense": [float(i) for i in range(16)], "indices": list(range(8)),
                              "values": [1.0] * 8, "expect": 28.0}]},
    "dense_dot": {"source": "crates/klearu-accel/src/simd/mod.rs:428-447",
                  "cases": [{"a": [1.0, 2.0, 3.0], "b": [4.0, 5.0, 6.0], "expect": 32.0},
                            {"a": [], "b": [], "expect": 0.0}]},
    "scatter_add": {"source": "crates/klearu-accel/src/simd/mod.rs:451-488",
                    "cases": [{"dense": [0.0] * 8, "indices": [1, 3, 5], "values": [1.0, 2.0, 3.0],
                               "scale": 2.0, "expect": [0.0, 2.0, 0.0, 4.0, 0.0, 6.0, 0.0, 0.0]},
                              {"dense": [5.0] * 4, "indices": [], "values": [], "scale": 1.0,
                               "expect": [5.0] * 4}]},
    "fifo": {"source": "crates/klearu-core/src/bucket/fifo.rs:74-161",
             "cases": [{"cap": 4, "ids": [1, 2, 3], "expect": [1, 2, 3]},
                       {"cap": 3, "ids": [10, 20, 30, 40], "expect": [20, 30, 40]},
                       {"cap": 2, "ids": [1, 2, 3], "expect": [2, 3]},
                       {"cap": 2, "ids": [1, 2, 3, 4], "expect": [3, 4]},
                       {"cap": 2, "ids": [1, 2, 3, 4, 5], "expect": [4, 5]},
                       {"cap": 1, "ids": [10], "expect": [10]},
                       {"cap": 1, "ids": [10, 20], "expect": [20]}]},
    "reservoir": {"source": "crates/klearu-core/src/bucket/reservoir.rs:110-131",
                  "cases": [{"cap": 4, "ids": [1, 2, 3], "expect_set": [1, 2, 3], "expect_count": 3},
                            {"cap": 3, "ids": list(range(100)), "expect_max_len": 3, "expect_count": 100}]},
    "self_query": {"source": "crates/klearu-core/src/lsh/index.rs:386-397, :417-434",
                   "dim": 8, "num_hashes": 3, "num_tables": 4, "bucket_capacity": 32, "seed": 42,
                   "id": 100, "w": [1.0, 0.5, -0.3, 0.0, 2.0, -1.0, 0.1, 0.7], "expect_count": 4},
    "zero_vector_hash": {"source": "crates/klearu-core/src/hash/simhash.rs:149-152, :230-240",
                         "dim": 128, "k": 8, "tables": 4, "seed": 42, "expect": 255},
    "topk_sampling": {"source": "crates/klearu-core/src/sampling/topk.rs:41-98",
                      "cases": [{"c": [[0, 3], [1, 5], [2, 1], [3, 4]], "k": 2, "expect": [1, 3]},
                                {"c": [[0, 1], [1, 2]], "k": 10, "expect": [1, 0]},
                                {"c": [[10, 5], [20, 3], [30, 1]], "k": 3, "expect": [10, 20, 30]},
                                {"c": [], "k": 5, "expect": []},
                                {"c": [[0, 5], [1, 3]], "k": 0, "expect": []},
                                {"c": [[5, 3], [2, 3], [8, 3], [1, 3]], "k": 2, "expect": [1, 2]},
                                {"c": [[42, 10]], "k": 5, "expect": [42]}]},
    "threshold_sampling": {"source": "crates/klearu-core/src/sampling/threshold.rs:50-133",
                           "cases": [{"c": [[0, 5], [1, 2], [2, 3], [3, 1]], "t": 3, "expect": [0, 2]},
                                     {"c": [[0, 5], [1, 2], [2, 3]], "t": 1, "expect": [0, 1, 2]},
                                     {"c": [[0, 3], [1, 5], [2, 1]], "t": 10, "expect": [1]},
                                     {"c": [[5, 3], [2, 3], [8, 3]], "t": 100, "expect": [2]},
                                     {"c": [], "t": 1, "expect": []},
                                     {"c": [[42, 1]], "t": 1, "expect": [42]},
                                     {"c": [[42, 2]], "t": 5, "expect": [42]},
                                     {"c": [[0, 0], [1, 0], [2, 0]], "t": 0, "expect": [0, 1, 2]}]},
    "rmsnorm": {"source": "crates/klearu-llm/src/model/rms_norm.rs:74-110",
                "cases": [{"x": [1.0, 2.0, 3.0, 4.0], "w": [1.0, 1.0, 1.0, 1.0], "eps": 1e-5,
                           "expect_formula": "x / sqrt(7.5 + 1e-5)", "tol": 1e-5},
                          {"x": [3.0, 3.0, 3.0], "w": [2.0, 0.5, 1.0], "eps": 1e-5,
                           "expect_formula": "3 / sqrt(9 + 1e-5) * w", "tol": 1e-5}]},
    "rope": {"source": "crates/klearu-llm/src/model/rope.rs:122-136",
             "head_dim": 2, "max_seq": 4, "theta": 1.0, "pos": 1, "x": [1.0, 0.0],
             "expect_formula": "[cos(1), sin(1)]", "tol": 1e-5},
}


def bf16(a):
    return orc.bf16_from_f32(np.asarray(a, np.float32))


def vectors():
    rng = np.random.default_rng(20260101)
    v = {}
    # SimHash planes from StdRng (seeded like SimHash::new)
    v["planes_d16_k4_l3_s42"] = orc.simhash_planes(16, 4, 3, 42)
    v["srp_d16_k4_l3_s42"] = orc.srp_planes(16, 4, 3, 1.0 / 3.0, 42)
    # hash codes
    dim, K, L = 64, 6, 5
    planes = orc.simhash_planes(dim, K, L, 7)
    X = rng.uniform(0, 1, (16, dim)).astype(np.float32)
    X[rng.uniform(0, 1, X.shape) < 0.8] = 0.0
    X[0] = 0.0
    v["hash_planes"], v["hash_x"] = planes, X
    v["hash_codes"] = orc.hash_dense_batch(planes, X)
    # LSH index (FIFO and reservoir) and queries
    W = rng.normal(0, 0.01, (200, dim)).astype(np.float32)
    v["lsh_w"] = W
    for name, typ, cap, n in (("fifo", FIFO, 8, 200), ("res", RES, 4, 200)):
        idx = orc.LshIndex(L, K, cap, typ)
        idx.insert_many(np.arange(n, dtype=np.uint32), orc.hash_dense_batch(planes, W[:n]))
        v[f"lsh_{name}_data"], v[f"lsh_{name}_len"], v[f"lsh_{name}_count"] = idx.data, idx.len, idx.count
        offs, ids, cnts = [0], [], []
        for r in range(X.shape[0]):
            i, c = idx.query(v["hash_codes"][r])
            ids.append(i)
            cnts.append(c)
            offs.append(offs[-1] + i.size)
        v[f"lsh_{name}_q_off"] = np.array(offs, np.int64)
        v[f"lsh_{name}_q_ids"] = np.concatenate(ids).astype(np.uint32)
        v[f"lsh_{name}_q_cnt"] = np.concatenate(cnts).astype(np.uint32)
    # SLIDE layer (Layer::new uses SimHash seed + 1_000_000 for its index)
    n, seed = 200, 5
    sp = orc.simhash_planes(dim, K, L, seed + 1_000_000)
    b = rng.normal(0, 0.01, n).astype(np.float32)
    v["slide_planes"], v["slide_w"], v["slide_b"] = sp, W, b
    for act in ("relu", "softmax"):
        out, _ = orc.slide_layer_oracle(sp, 8, FIFO, W, b, X, act=act)
        v[f"slide_{act}_off"] = np.cumsum([0] + [o[0].size for o in out]).astype(np.int64)
        v[f"slide_{act}_ids"] = np.concatenate([o[0] for o in out]).astype(np.uint32)
        v[f"slide_{act}_pre"] = np.concatenate([o[1] for o in out]).astype(np.float32)
        v[f"slide_{act}_act"] = np.concatenate([o[2] for o in out]).astype(np.float32)
    # predictor + top-k (BF16-valued weights, as the LLM predictors hold)
    ind, hid, out_n, k = 128, 64, 300, 45
    w1, w2 = bf16(rng.normal(0, 0.02, (hid, ind))), bf16(rng.normal(0, 0.1, (out_n, hid)))
    b1, b2 = rng.normal(0, 0.1, hid).astype(np.float32), rng.normal(0, 0.1, out_n).astype(np.float32)
    px = rng.standard_normal((2, ind)).astype(np.float32)
    v["pred_w1"], v["pred_b1"], v["pred_w2"], v["pred_b2"], v["pred_x"] = w1, b1, w2, b2, px
    sc = np.stack([orc.predictor_predict(w1, b1, w2, b2, px[i])[0] for i in range(2)])
    v["pred_scores"] = sc
    v["pred_topk"] = np.stack([orc.select_top_k(sc[i], k) for i in range(2)]).astype(np.int64)
    # sparse SwiGLU FFN
    H, I, ka = 128, 256, 40
    wg, wu = bf16(rng.normal(0, 0.02, (I, H))), bf16(rng.normal(0, 0.02, (I, H)))
    wd = bf16(rng.normal(0, 0.02, (H, I)))
    fx = rng.standard_normal((3, H)).astype(np.float32)
    act = np.sort(rng.choice(I, ka, replace=False)).astype(np.int64)
    v["ffn_wg"], v["ffn_wu"], v["ffn_wd"], v["ffn_x"], v["ffn_active"] = wg, wu, wd, fx, act
    v["ffn_y"] = np.stack([orc.sparse_mlp_forward_bf16(wg, wu, wd, fx[i], act)[0] for i in range(3)])
    # head-sparse decode attention (f32 cache, GQA 2:1)
    hidden, nh, nkv, d, max_seq, plen = 128, 2, 1, 64, 32, 12
    wq, wk = bf16(rng.normal(0, 0.02, (nh * d, hidden))), bf16(rng.normal(0, 0.02, (nkv * d, hidden)))
    wv, wo = bf16(rng.normal(0, 0.02, (nkv * d, hidden))), bf16(rng.normal(0, 0.02, (hidden, nh * d)))
    kc = np.zeros((nkv, max_seq, d), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :plen] = rng.standard_normal((nkv, plen, d))
    vc[:, :plen] = rng.standard_normal((nkv, plen, d))
    ax = rng.standard_normal(hidden).astype(np.float32)
    v.update(attn_wq=wq, attn_wk=wk, attn_wv=wv, attn_wo=wo, attn_k=kc[:, :plen].copy(),
             attn_v=vc[:, :plen].copy(), attn_x=ax, attn_heads=np.array([1], np.int64))
    cos_t, sin_t = orc.rope_tables(d, max_seq, 10000.0)
    v["attn_out"] = orc.sparse_attention_forward_bf16(wq, wk, wv, wo, nh, nkv, d, ax, plen, cos_t, sin_t,
                                                      kc, vc, [1])
    v["attn_k_appended"] = kc[:, plen].copy()
    v["attn_v_appended"] = vc[:, plen].copy()
    # klearu-accel
    a, bb = rng.standard_normal(37).astype(np.float32), rng.standard_normal(37).astype(np.float32)
    v["acc_a"], v["acc_b"], v["acc_dot"] = a, bb, np.float32(orc.dense_dot(a, bb))
    si = np.sort(rng.choice(37, 11, replace=False)).astype(np.uint32)
    sv = rng.standard_normal(11).astype(np.float32)
    v["acc_sidx"], v["acc_sval"] = si, sv
    v["acc_sdot"] = np.float32(orc.sparse_dot_dense(si, sv, bb))
    di = rng.integers(0, 16, 40).astype(np.uint32)
    dv = rng.standard_normal(40).astype(np.float32)
    dense = rng.standard_normal(16).astype(np.float32)
    v["acc_didx"], v["acc_dval"], v["acc_dense"] = di, dv, dense
    v["acc_scatter"] = orc.scatter_add(di, dv, dense.copy(), 0.75)
    v["acc_bf16"] = bf16(a)
    return v


def main():
    with open(os.path.join(HERE, "kats.json"), "w") as f:
        json.dump(KATS, f, indent=1)
    np.savez_compressed(os.path.join(HERE, "vectors.npz"), **vectors())
    print("wrote", os.path.join(HERE, "kats.json"), os.path.join(HERE, "vectors.npz"))


if __name__ == "__main__":
    main()
