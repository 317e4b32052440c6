"""Handles built from on-disk files equal handles built from the same arrays (GPU).

PredictorStore directories (crates/klearu-llm/src/sparse/predictor_store.rs:31-89)
and safetensors decoder layers (crates/klearu-llm/src/weight/loader.rs:96-133)
load into the same device state as kh_predictor_create / kh_sparse_ffn_create /
kh_sparse_attn_create from the arrays, so every output is compared bit for bit.
The predictor's selections are also checked against the oracle.
"""
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "predictor_store")


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_predictor_store_fixture_loads_and_selects_exactly(kh, orc):
    from klearu_amd.dejavu import ORDER_SCORE, PredictorStore, SparsityPredictor
    exp = np.load(os.path.join(GOLD, "expected.npz"))
    store = PredictorStore.load(GOLD, 3)
    assert store.is_calibrated()
    assert store.head_predictors[1] is None and store.neuron_predictors[1] is None
    assert store.head_predictors[2] is None and store.neuron_predictors[2] is not None
    rng = np.random.default_rng(0)
    xs = [np.full(8, 0.1, np.float32), np.full(8, 0.5, np.float32), rng.standard_normal(8).astype(np.float32)]
    for name, p in (("layer_0_head", store.head_predictors[0]), ("layer_0_neuron", store.neuron_predictors[0]),
                    ("layer_2_neuron", store.neuron_predictors[2])):
        w1, b1, w2, b2 = (exp[f"{name}.{k}"] for k in ("w1", "b1", "w2", "b2"))
        for g, e in zip(p.weights(), (w1, b1, w2, b2)):
            np.testing.assert_array_equal(bits(g), bits(e))
        ref = SparsityPredictor(w1, b1, w2, b2)
        for x in xs:
            s = p.predict(torch.from_numpy(x).cuda()).cpu().numpy()
            np.testing.assert_array_equal(bits(s), bits(ref.predict(torch.from_numpy(x).cuda()).cpu().numpy()))
            os_, _ = orc.predictor_predict(w1, b1, w2, b2, x)
            fin = np.isfinite(os_)
            np.testing.assert_array_equal(bits(s[fin]), bits(os_[fin]))
            k = 3
            ids = p.select_top_k(torch.from_numpy(x).cuda(), k, ORDER_SCORE).cpu().numpy()
            np.testing.assert_array_equal(ids, orc.select_top_k(os_, k))
    # layer 1 has no predictor: the first k ids (predictor_store.rs:31-36)
    x = torch.full((8,), 0.1, device="cuda")
    np.testing.assert_array_equal(store.predict_heads(1, x, 3).cpu().numpy(), [0, 1, 2])
    np.testing.assert_array_equal(store.predict_neurons(1, x, 5).cpu().numpy(), [0, 1, 2, 3, 4])


def test_predictor_save_load_roundtrip_cfg2_shape(kh, tmp_path):
    """A 2048 -> 128 -> 5632 predictor (cfg2) saved and reloaded keeps every bit."""
    from klearu_amd.dejavu import ORDER_SCORE, PredictorStore, SparsityPredictor
    rng = np.random.default_rng(5)
    w1 = (rng.standard_normal((128, 2048)) * 0.03).astype(np.float32)
    w2 = (rng.standard_normal((5632, 128)) * 0.1).astype(np.float32)
    b1 = (rng.standard_normal(128) * 0.01).astype(np.float32)
    b2 = (rng.standard_normal(5632) * 0.01).astype(np.float32)
    p = SparsityPredictor(w1, b1, w2, b2)
    store = PredictorStore(2)
    store.set_neuron_predictor(1, p)
    store.save(str(tmp_path))
    assert sorted(os.listdir(tmp_path)) == ["layer_1_neuron.json"]
    q = PredictorStore.load(str(tmp_path), 2).neuron_predictors[1]
    for g, e in zip(q.weights(), (w1, b1, w2, b2)):
        np.testing.assert_array_equal(bits(g), bits(e))
    x = torch.randn(4, 2048, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))
    np.testing.assert_array_equal(bits(q.predict(x).cpu().numpy()), bits(p.predict(x).cpu().numpy()))
    np.testing.assert_array_equal(q.select_top_k(x, 564, ORDER_SCORE).cpu().numpy(),
                                  p.select_top_k(x, 564, ORDER_SCORE).cpu().numpy())


def _bf16(rng, shape, scale):
    f = (rng.standard_normal(shape) * scale).astype(np.float32)
    return (f.view(np.uint32) >> 16).astype(np.uint16)


def _save(path, tensors):
    from safetensors.torch import save_file
    save_file({k: torch.from_numpy(v.view(np.int16)).view(torch.bfloat16) if v.dtype == np.uint16
               else torch.from_numpy(v) for k, v in tensors.items()}, path)


@pytest.mark.parametrize("prefix", ["model.", "model.language_model."])
def test_mlp_from_safetensors_equals_arrays(kh, tmp_path, prefix):
    from klearu_amd._lib import KH_ERR_UNSUPPORTED, KlearuError
    from klearu_amd.dejavu import Mlp, forward_sparse
    from klearu_amd.formats import SafeTensorsFile
    H, I = 1024, 2816
    rng = np.random.default_rng(9)
    wg, wu, wd = _bf16(rng, (I, H), 0.02), _bf16(rng, (I, H), 0.02), _bf16(rng, (H, I), 0.02)
    path = str(tmp_path / "m.safetensors")
    _save(path, {f"{prefix}layers.1.mlp.gate_proj.weight": wg, f"{prefix}layers.1.mlp.up_proj.weight": wu,
                 f"{prefix}layers.1.mlp.down_proj.weight": wd, f"{prefix}layers.1.input_layernorm.weight":
                 np.ones(H, np.float32)})
    ref = Mlp(wg, wu, wd, max_batch=4)
    with SafeTensorsFile(path) as st:
        got = Mlp.from_safetensors(st, 1, max_batch=4)
        assert (got.hidden_size, got.intermediate_size) == (H, I)
        with pytest.raises(KlearuError):
            Mlp.from_safetensors(st, 0)
    x = torch.randn(4, H, device="cuda", generator=torch.Generator(device="cuda").manual_seed(2))
    act = torch.from_numpy(np.sort(rng.choice(I, 423, replace=False)).astype(np.int32)).cuda()
    for xb in (x[:1], x):
        a = forward_sparse(got, xb, act).cpu().numpy()
        b = forward_sparse(ref, xb, act).cpu().numpy()
        np.testing.assert_array_equal(bits(a), bits(b))
    # f32 tensors are taken when every value is a BF16 value, refused otherwise
    f32 = lambda u: (u.astype(np.uint32) << 16).view(np.float32)
    p2 = str(tmp_path / "f.safetensors")
    _save(p2, {f"{prefix}layers.0.mlp.gate_proj.weight": f32(wg), f"{prefix}layers.0.mlp.up_proj.weight": f32(wu),
               f"{prefix}layers.0.mlp.down_proj.weight": f32(wd)})
    with SafeTensorsFile(p2) as st:
        got2 = Mlp.from_safetensors(st, 0, max_batch=4)
    np.testing.assert_array_equal(bits(forward_sparse(got2, x, act).cpu().numpy()),
                                  bits(forward_sparse(ref, x, act).cpu().numpy()))
    bad = f32(wd).copy()
    bad[3, 5] = np.float32(1.0000001)
    p3 = str(tmp_path / "g.safetensors")
    _save(p3, {f"{prefix}layers.0.mlp.gate_proj.weight": f32(wg), f"{prefix}layers.0.mlp.up_proj.weight": f32(wu),
               f"{prefix}layers.0.mlp.down_proj.weight": bad})
    with SafeTensorsFile(p3) as st:
        with pytest.raises(KlearuError) as e:
            Mlp.from_safetensors(st, 0)
        assert e.value.code == KH_ERR_UNSUPPORTED


def test_attention_from_safetensors_equals_arrays(kh, tmp_path):
    from klearu_amd.attention import SparseAttention
    from klearu_amd.formats import SafeTensorsFile
    H, nh, nkv, d, S = 512, 8, 2, 64, 64
    rng = np.random.default_rng(11)
    wq, wk, wv = _bf16(rng, (nh * d, H), 0.05), _bf16(rng, (nkv * d, H), 0.05), _bf16(rng, (nkv * d, H), 0.05)
    wo = _bf16(rng, (H, nh * d), 0.05)
    path = str(tmp_path / "a.safetensors")
    _save(path, {"model.layers.0.self_attn.q_proj.weight": wq, "model.layers.0.self_attn.k_proj.weight": wk,
                 "model.layers.0.self_attn.v_proj.weight": wv, "model.layers.0.self_attn.o_proj.weight": wo})
    ref = SparseAttention(H, nh, nkv, d, wq, wk, wv, wo, S, 2)
    with SafeTensorsFile(path) as st:
        got = SparseAttention.from_safetensors(st, 0, nh, nkv, d, S, 2)
    g = torch.Generator(device="cuda").manual_seed(4)
    for step in range(3):
        x = torch.randn(2, H, device="cuda", generator=g)
        heads = torch.tensor([[0, 3, 5, 6], [1, 2, 4, 7]], dtype=torch.int32, device="cuda")
        a = got.forward_sparse(x, heads).cpu().numpy()
        b = ref.forward_sparse(x, heads).cpu().numpy()
        np.testing.assert_array_equal(bits(a), bits(b), err_msg=f"step {step}")
