"""Golden fixtures (tests/golden/): the reference's known answers and seeded
vectors for every function on the path.

CPU: the oracle still reproduces every fixture bit for bit and passes every
known answer.  GPU: the HIP library matches the same fixtures -- bit-exact for
codes, buckets, candidate sets, active sets, pre-activations, predictor scores
and top-k; within 2e-3 relative for BF16-weight outputs (FFN, attention) and
1e-5 for softmax, with max-abs printed.
"""
import json
import math
import os
import sys

import numpy as np
import pytest

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KATS = json.load(open(os.path.join(HERE, "kats.json")))
VEC = dict(np.load(os.path.join(HERE, "vectors.npz")))
FIFO, RES = 0, 1


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def close(got, ref, rtol, what):
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    print(f"{what}: max|ref|={scale:.4g} max-abs-err={err:.3g}")
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=1e-4 * scale + 1e-30)


# ------------------------------------------------------------------------ CPU
def test_oracle_reproduces_vectors(orc):
    sys.path.insert(0, HERE)
    try:
        import make_golden
    finally:
        sys.path.remove(HERE)
    fresh = make_golden.vectors()
    assert sorted(fresh) == sorted(VEC)
    for k, v in fresh.items():
        a, b = np.atleast_1d(np.asarray(v)), np.atleast_1d(VEC[k])
        assert a.dtype == b.dtype and a.shape == b.shape, k
        np.testing.assert_array_equal(a.view(np.uint8), b.view(np.uint8), err_msg=k)


def test_oracle_kats(orc):
    for c in KATS["sparse_dot"]["cases"]:
        assert orc.sparse_dot_dense(c["indices"], c["values"], c["dense"]) == c["expect"]
    for c in KATS["dense_dot"]["cases"]:
        assert orc.dense_dot(c["a"], c["b"]) == c["expect"]
    for c in KATS["scatter_add"]["cases"]:
        np.testing.assert_array_equal(orc.scatter_add(c["indices"], c["values"], c["dense"], c["scale"]),
                                      np.array(c["expect"], np.float32))
    for c in KATS["fifo"]["cases"]:
        idx = orc.LshIndex(1, 1, c["cap"], FIFO)
        idx.insert_many(c["ids"], np.zeros(len(c["ids"]), np.uint32))
        assert list(idx.bucket(0, 0)) == c["expect"]
    for c in KATS["reservoir"]["cases"]:
        idx = orc.LshIndex(1, 1, c["cap"], RES)
        idx.insert_many(c["ids"], np.zeros(len(c["ids"]), np.uint32))
        got = list(idx.bucket(0, 0))
        assert int(idx.count[0]) == c["expect_count"]
        if "expect_set" in c:
            assert sorted(got) == c["expect_set"]
        else:
            assert len(got) <= c["expect_max_len"]
    q = KATS["self_query"]
    planes = orc.simhash_planes(q["dim"], q["num_hashes"], q["num_tables"], q["seed"])
    codes = orc.hash_dense_batch(planes, np.array(q["w"], np.float32))
    idx = orc.LshIndex(q["num_tables"], q["num_hashes"], q["bucket_capacity"], FIFO)
    idx.insert_many([q["id"]], codes)
    ids, cnt = idx.query(codes[0])
    assert list(ids) == [q["id"]] and list(cnt) == [q["expect_count"]]
    z = KATS["zero_vector_hash"]
    planes = orc.simhash_planes(z["dim"], z["k"], z["tables"], z["seed"])
    assert all(c == z["expect"] for c in orc.hash_dense_batch(planes, np.zeros(z["dim"], np.float32))[0])
    for c in KATS["topk_sampling"]["cases"]:
        assert list(orc.sample_topk([a for a, _ in c["c"]], [b for _, b in c["c"]], c["k"])) == c["expect"]
    for c in KATS["threshold_sampling"]["cases"]:
        assert list(orc.sample_threshold([a for a, _ in c["c"]], [b for _, b in c["c"]], c["t"])) == c["expect"]
    c0, c1 = KATS["rmsnorm"]["cases"]
    np.testing.assert_allclose(orc.rmsnorm(c0["x"], c0["w"], c0["eps"]),
                               np.array(c0["x"]) / math.sqrt(7.5 + 1e-5), atol=c0["tol"])
    np.testing.assert_allclose(orc.rmsnorm(c1["x"], c1["w"], c1["eps"]),
                               3.0 / math.sqrt(9 + 1e-5) * np.array(c1["w"]), atol=c1["tol"])
    r = KATS["rope"]
    cos_t, sin_t = orc.rope_tables(r["head_dim"], r["max_seq"], r["theta"])
    x = np.array(r["x"], np.float32)
    orc.lib.or_rope_apply(x, r["head_dim"] // 2, cos_t, sin_t, r["pos"])
    np.testing.assert_allclose(x, [math.cos(1), math.sin(1)], atol=r["tol"])


# ------------------------------------------------------------------------ GPU
@pytest.mark.gpu
def test_gpu_kats(kh):
    import torch
    from klearu_amd.accel import dense_dot_dense_simd, scatter_add_simd, sparse_dot_dense_simd
    from klearu_amd.dejavu import rmsnorm
    from klearu_amd.lsh import HashFamily, LshIndex, SimHash
    for c in KATS["sparse_dot"]["cases"]:
        if c["indices"]:
            assert float(sparse_dot_dense_simd(np.array(c["indices"], np.uint32), c["values"], c["dense"])) \
                == c["expect"]
    assert float(dense_dot_dense_simd(KATS["dense_dot"]["cases"][0]["a"],
                                      KATS["dense_dot"]["cases"][0]["b"])) == 32.0
    c = KATS["scatter_add"]["cases"][0]
    d = torch.zeros(len(c["dense"]), device="cuda")
    scatter_add_simd(np.array(c["indices"], np.uint32), c["values"], d, c["scale"])
    np.testing.assert_array_equal(d.cpu().numpy(), np.array(c["expect"], np.float32))
    one = HashFamily.from_planes(np.ones((1, 1, 1), np.int8))
    for typ, key in ((FIFO, "fifo"), (RES, "reservoir")):
        for c in KATS[key]["cases"]:
            idx = LshIndex(one, typ, c["cap"])
            idx.insert_codes(np.array(c["ids"], np.uint32), np.zeros(len(c["ids"]), np.uint32))
            data, ln, cnt = idx.buckets()
            got = list(data[0, 0, : ln[0, 0]])
            if "expect" in c:
                assert got == c["expect"]
            elif "expect_set" in c:
                assert sorted(got) == c["expect_set"] and int(cnt[0, 0]) == c["expect_count"]
            else:
                assert len(got) <= c["expect_max_len"] and int(cnt[0, 0]) == c["expect_count"]
    q = KATS["self_query"]
    idx = LshIndex(SimHash(q["dim"], q["num_hashes"], q["num_tables"], q["seed"]), FIFO, q["bucket_capacity"])
    idx.insert(q["id"], q["w"])
    assert [(c.neuron_id, c.count) for c in idx.query(q["w"])] == [(q["id"], q["expect_count"])]
    z = KATS["zero_vector_hash"]
    fam = SimHash(z["dim"], z["k"], z["tables"], z["seed"])
    codes = fam.hash_dense_batch(np.zeros((1, z["dim"]), np.float32)).cpu().numpy()
    assert np.all(codes == z["expect"])
    c0, c1 = KATS["rmsnorm"]["cases"]
    for c, ref in ((c0, np.array(c0["x"]) / math.sqrt(7.5 + 1e-5)),
                   (c1, 3.0 / math.sqrt(9 + 1e-5) * np.array(c1["w"]))):
        got = rmsnorm(np.array([c["x"]], np.float32), np.array(c["w"], np.float32), c["eps"]).cpu().numpy()[0]
        np.testing.assert_allclose(got, ref, atol=c["tol"])


@pytest.mark.gpu
def test_gpu_hash_and_index_vectors(kh):
    from klearu_amd.lsh import HashFamily, LshIndex, SimHash, SparseRandomProjection
    np.testing.assert_array_equal(SimHash(16, 4, 3, 42).planes(), VEC["planes_d16_k4_l3_s42"])
    np.testing.assert_array_equal(SparseRandomProjection(16, 4, 3, 1.0 / 3.0, 42).planes(),
                                  VEC["srp_d16_k4_l3_s42"])
    fam = HashFamily.from_planes(VEC["hash_planes"])
    codes = fam.hash_dense_batch(VEC["hash_x"]).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(codes, VEC["hash_codes"])
    for name, typ, cap in (("fifo", FIFO, 8), ("res", RES, 4)):
        idx = LshIndex(fam, typ, cap)
        idx.insert_batch(np.arange(200, dtype=np.uint32), VEC["lsh_w"])
        data, ln, cnt = idx.buckets()
        np.testing.assert_array_equal(ln.reshape(-1), VEC[f"lsh_{name}_len"])
        np.testing.assert_array_equal(cnt.reshape(-1), VEC[f"lsh_{name}_count"])
        ref = VEC[f"lsh_{name}_data"].reshape(data.shape)
        for t in range(data.shape[0]):
            for b in range(data.shape[1]):
                np.testing.assert_array_equal(data[t, b, : ln[t, b]], ref[t, b, : ln[t, b]])
        off, ids, c = idx.query_batch(VEC["hash_x"])
        off = off.cpu().numpy()
        np.testing.assert_array_equal(off, VEC[f"lsh_{name}_q_off"])
        n = int(off[-1])
        np.testing.assert_array_equal(ids[:n].cpu().numpy().view(np.uint32), VEC[f"lsh_{name}_q_ids"])
        np.testing.assert_array_equal(c[:n].cpu().numpy().view(np.uint32), VEC[f"lsh_{name}_q_cnt"])


@pytest.mark.gpu
@pytest.mark.parametrize("act", ["relu", "softmax"])
def test_gpu_slide_vectors(kh, act):
    from klearu_amd.lsh import LshConfig
    from klearu_amd.slide import Layer, LayerConfig
    lsh = LshConfig(num_tables=5, num_hashes=6, bucket_capacity=8, bucket_type="Fifo")
    cfg = LayerConfig(64, 200, act.capitalize(), lsh, "Vanilla", 2, 0)
    layer = Layer(cfg, VEC["slide_w"], VEC["slide_b"], 5)
    np.testing.assert_array_equal(layer.index.hash_family.planes(), VEC["slide_planes"])
    off, ids, pre, a = (t.cpu().numpy() for t in layer.forward_batch(VEC["hash_x"]))
    np.testing.assert_array_equal(off, VEC[f"slide_{act}_off"])
    n = int(off[-1])
    np.testing.assert_array_equal(ids[:n].view(np.uint32), VEC[f"slide_{act}_ids"])
    np.testing.assert_array_equal(bits(pre[:n]), bits(VEC[f"slide_{act}_pre"]))
    if act == "relu":
        np.testing.assert_array_equal(bits(a[:n]), bits(VEC[f"slide_{act}_act"]))
    else:
        close(a[:n], VEC[f"slide_{act}_act"], 1e-5, "softmax")


@pytest.mark.gpu
def test_gpu_predictor_vectors(kh, orc):
    import torch
    from klearu_amd.dejavu import SparsityPredictor
    p = SparsityPredictor(orc.bf16_to_f32(VEC["pred_w1"]), VEC["pred_b1"], orc.bf16_to_f32(VEC["pred_w2"]),
                          VEC["pred_b2"])
    x = torch.from_numpy(VEC["pred_x"]).cuda()
    np.testing.assert_array_equal(bits(p.predict(x).cpu().numpy()), bits(VEC["pred_scores"]))
    np.testing.assert_array_equal(p.select_top_k(x, VEC["pred_topk"].shape[1]).cpu().numpy(), VEC["pred_topk"])


@pytest.mark.gpu
def test_gpu_ffn_vectors(kh):
    import torch
    from klearu_amd.dejavu import Mlp
    mlp = Mlp(VEC["ffn_wg"], VEC["ffn_wu"], VEC["ffn_wd"], max_batch=4)
    x = torch.from_numpy(VEC["ffn_x"]).cuda()
    y = torch.empty_like(x)
    mlp.forward_sparse_into(x, torch.from_numpy(VEC["ffn_active"].astype(np.int32)).cuda(), y)
    close(y.cpu().numpy(), VEC["ffn_y"], 2e-3, "ffn batch 3")
    y1 = torch.empty_like(x[:1])
    mlp.forward_sparse_into(x[:1].contiguous(), torch.from_numpy(VEC["ffn_active"].astype(np.int32)).cuda(), y1)
    close(y1.cpu().numpy(), VEC["ffn_y"][:1], 2e-3, "ffn batch 1")


@pytest.mark.gpu
def test_gpu_attention_vectors(kh):
    from klearu_amd.attention import KV_F32, SparseAttention
    k, v = VEC["attn_k"], VEC["attn_v"]
    nkv, plen, d = k.shape
    hidden = VEC["attn_x"].size
    nh = VEC["attn_wq"].shape[0] // d
    a = SparseAttention(hidden, nh, nkv, d, VEC["attn_wq"], VEC["attn_wk"], VEC["attn_wv"], VEC["attn_wo"], 32, 1,
                        10000.0, KV_F32)
    a.load_cache(0, k, v)
    out = a.forward_sparse(VEC["attn_x"][None, :], VEC["attn_heads"].astype(np.int32)[None, :]).cpu().numpy()[0]
    close(out, VEC["attn_out"], 2e-3, "attention")
    kk, vv = a.read_cache(0, plen + 1)
    close(kk[:, plen], VEC["attn_k_appended"], 2e-3, "appended k")
    close(vv[:, plen], VEC["attn_v_appended"], 2e-3, "appended v")
    assert a.current_len(0) == plen + 1


@pytest.mark.gpu
def test_gpu_accel_vectors(kh):
    import torch
    from klearu_amd.accel import Bf16Weights, dense_dot_dense_simd, scatter_add_simd, sparse_dot_dense_simd
    assert bits(dense_dot_dense_simd(VEC["acc_a"], VEC["acc_b"]).cpu().numpy()) == bits(VEC["acc_dot"])
    assert bits(sparse_dot_dense_simd(VEC["acc_sidx"], VEC["acc_sval"], VEC["acc_b"]).cpu().numpy()) \
        == bits(VEC["acc_sdot"])
    d = torch.from_numpy(VEC["acc_dense"].copy()).cuda()
    scatter_add_simd(VEC["acc_didx"], VEC["acc_dval"], d, 0.75)
    np.testing.assert_array_equal(bits(d.cpu().numpy()), bits(VEC["acc_scatter"]))
    w = Bf16Weights.from_f32(VEC["acc_a"])
    np.testing.assert_array_equal(w.data.cpu().numpy().view(np.uint16), VEC["acc_bf16"])
