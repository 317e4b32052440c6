"""Pins the oracle's Deja Vu restatement (CPU only).

Known answers from the reference tests:
  predictor  crates/klearu-dejavu/src/predictor/mlp_predictor.rs:214-262 (range, count, no dups)
  RMSNorm    crates/klearu-llm/src/model/rms_norm.rs:78-110
  RoPE       crates/klearu-llm/src/model/rope.rs:95-140 (magnitude, identity at 0, known angle)
  sparse==dense invariants: klearu-llm sparse/sparse_mlp.rs:59-86 (hand-set weights),
             klearu-dejavu mlp.rs:88-130
Math pins: float64 evaluations bound every f32 result (sequential-sum error bound
gamma_n * sum|terms|); numpy's stable argsort pins the stable top-k order;
textbook softmax attention pins the sparse attention.
"""
import numpy as np
import pytest

U = 2.0 ** -24  # unit roundoff of f32


def bf16r(orc, a):
    return orc.bf16_from_f32(np.asarray(a, np.float32))


def test_predictor_matches_float64_within_bound(orc):
    rng = np.random.default_rng(0)
    ind, hid, out = 256, 32, 200
    w1 = rng.normal(0, 0.02, (hid, ind)).astype(np.float32)
    w2 = rng.normal(0, 0.05, (out, hid)).astype(np.float32)
    b1 = rng.normal(0, 0.1, hid).astype(np.float32)
    b2 = rng.normal(0, 0.1, out).astype(np.float32)
    x = rng.standard_normal(ind).astype(np.float32)
    s, h = orc.predictor_predict(w1, b1, w2, b2, x)
    h64 = np.maximum(w1.astype(np.float64) @ x + b1, 0)
    bound1 = (ind + 2) * U * (np.abs(w1.astype(np.float64)) @ np.abs(x) + np.abs(b1))
    assert np.all(np.abs(h - h64) <= bound1 + 1e-30)
    z64 = w2.astype(np.float64) @ h64 + b2
    np.testing.assert_allclose(s, 1 / (1 + np.exp(-z64)), rtol=1e-5, atol=1e-6)
    assert np.all((s >= 0) & (s <= 1))


def test_predictor_bf16_weights_equal_widened_f32(orc):
    rng = np.random.default_rng(1)
    w1 = bf16r(orc, rng.normal(0, 0.02, (16, 64)))
    w2 = bf16r(orc, rng.normal(0, 0.02, (40, 16)))
    b1, b2 = np.zeros(16, np.float32), np.zeros(40, np.float32)
    x = rng.standard_normal(64).astype(np.float32)
    s1, h1 = orc.predictor_predict(w1, b1, w2, b2, x)
    s2, h2 = orc.predictor_predict(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2, x)
    assert s1.tobytes() == s2.tobytes() and h1.tobytes() == h2.tobytes()


def test_select_top_k_is_stable_desc(orc):
    rng = np.random.default_rng(2)
    for n, k in ((12, 5), (12, 20), (5632, 564), (11008, 1652), (32, 16)):
        s = rng.random(n).astype(np.float32)
        s[rng.random(n) < 0.3] = 0.5  # many ties
        s[:3] = 0.0
        s[3] = -0.0  # -0.0 == +0.0 for partial_cmp
        ref = np.argsort(-s.astype(np.float64), kind="stable")[:k]
        got = orc.select_top_k(s, k)
        np.testing.assert_array_equal(got, ref)
        assert len(set(got.tolist())) == len(got) == min(k, n)


def test_sigmoid_silu_closed_form(orc):
    for z in (-30.0, -5.0, -0.5, 0.0, 0.25, 3.0, 17.0, 90.0):
        assert abs(orc.lib.or_sigmoid(z) - 1 / (1 + np.exp(-z))) <= 2e-7
        assert abs(orc.lib.or_silu(z) - z / (1 + np.exp(-z))) <= 4e-7 * max(1.0, abs(z))
    assert orc.lib.or_sigmoid(0.0) == 0.5 and orc.lib.or_silu(0.0) == 0.0


def test_sparse_mlp_all_neurons_matches_dense_kat(orc):
    # sparse_mlp.rs:59-86: hidden 4, inter 8, gate/up rows have 0.1 at i%4,
    # down rows have 0.1 at j; input ones; all neurons == dense within 1e-5.
    wg = np.zeros((8, 4), np.float32)
    for i in range(8):
        wg[i, i % 4] = 0.1
    wd = np.zeros((4, 8), np.float32)
    for j in range(4):
        wd[j, j] = 0.1
    b = lambda a: bf16r(orc, a)
    y, h = orc.sparse_mlp_forward_bf16(b(wg), b(wg), b(wd), np.ones(4, np.float32), np.arange(8))
    g = orc.bf16_to_f32(b(wg)).astype(np.float64) @ np.ones(4)
    hd = g / (1 + np.exp(-g)) * g
    yd = orc.bf16_to_f32(b(wd)).astype(np.float64) @ hd
    np.testing.assert_allclose(y, yd, atol=1e-5)


def test_sparse_mlp_matches_float64_swiglu(orc):
    rng = np.random.default_rng(3)
    H, I, k = 256, 704, 71
    wg = bf16r(orc, rng.normal(0, 0.02, (I, H)))
    wu = bf16r(orc, rng.normal(0, 0.02, (I, H)))
    wd = bf16r(orc, rng.normal(0, 0.02, (H, I)))
    x = rng.standard_normal(H).astype(np.float32)
    act = rng.choice(I, k, replace=False)
    y, h = orc.sparse_mlp_forward_bf16(wg, wu, wd, x, act)
    G = orc.bf16_to_f32(wg).astype(np.float64)[act] @ x
    Uu = orc.bf16_to_f32(wu).astype(np.float64)[act] @ x
    h64 = G / (1 + np.exp(-G)) * Uu
    y64 = orc.bf16_to_f32(wd).astype(np.float64)[:, act] @ h64
    np.testing.assert_allclose(h, h64, rtol=1e-4, atol=1e-6)
    np.testing.assert_allclose(y, y64, rtol=1e-3, atol=1e-5)
    # the down projection sums in active-list order: permuting the active list
    # must leave the gate/up values unchanged and move y only by rounding
    perm = rng.permutation(k)
    y2, h2 = orc.sparse_mlp_forward_bf16(wg, wu, wd, x, act[perm])
    np.testing.assert_array_equal(h2, h[perm])
    np.testing.assert_allclose(y2, y, rtol=1e-4, atol=1e-6)


def test_rmsnorm_kats(orc):
    x = orc.rmsnorm([1, 2, 3, 4], np.ones(4, np.float32), 1e-5)
    r = np.float32(np.sqrt(np.float32(7.5) + np.float32(1e-5)))
    np.testing.assert_allclose(x, np.array([1, 2, 3, 4], np.float32) / r, atol=1e-5)
    x = orc.rmsnorm([3, 3, 3], np.array([2.0, 0.5, 1.0], np.float32), 1e-5)
    n = 3.0 / np.sqrt(9.0 + 1e-5)
    np.testing.assert_allclose(x, [n * 2, n * 0.5, n], atol=1e-5)
    x = orc.rmsnorm([1, 0, 0, 0], np.ones(4, np.float32), 1e-5)
    assert abs(float(np.sum(x * x)) - 4.0) < 0.01


def test_rms_inv_known_answers(orc):
    """The RmsNorm scale 1/rms (rms_norm.rs:48-52) that the fused decode blocks
    write out: closed forms and a known answer that only the left-to-right f32
    sum of squares reproduces."""
    assert orc.rms_inv(np.full(4, 2.0, np.float32), 0.0) == np.float32(0.5)  # 16/4 = 4, sqrt 2
    # 4096^2 = 2^24; every later square 1.0 is a tie that rounds back down, so
    # the sequential sum stays 2^24: 2^24/4096 = 4096, sqrt 64, scale 1/64.
    # The exact (or any tree-ordered) sum 2^24 + 4095 gives a different scale.
    stuck = np.ones(4096, np.float32)
    stuck[0] = 4096.0
    assert orc.rms_inv(stuck, 0.0) == np.float32(1.0 / 64.0)
    assert orc.rms_inv(stuck[::-1].copy(), 0.0) != np.float32(1.0 / 64.0)
    # a zero row: the scale is 1/sqrt(eps), each operation correctly rounded in f32
    eps = np.float32(1e-5)
    assert orc.rms_inv(np.zeros(64, np.float32), eps) == np.float32(1.0) / np.sqrt(eps)
    # RmsNorm::forward is x * scale * w, each product rounded
    rng = np.random.default_rng(5)
    x = rng.standard_normal(333).astype(np.float32)
    inv = orc.rms_inv(x, 1e-6)
    np.testing.assert_array_equal(orc.rmsnorm(x, np.ones(333, np.float32), 1e-6), x * inv)


def test_rope_kats(orc):
    c, s = orc.rope_tables(2, 4, 1.0)
    x = np.array([1.0, 0.0], np.float32)
    orc.lib.or_rope_apply(x, 1, c, s, 1)
    assert abs(x[0] - np.cos(1.0)) < 1e-5 and abs(x[1] - np.sin(1.0)) < 1e-5
    c, s = orc.rope_tables(8, 16, 10000.0)
    x = np.arange(1, 9, dtype=np.float32)
    m0 = float(np.sum(x * x))
    orc.lib.or_rope_apply(x, 4, c, s, 5)
    assert abs(float(np.sum(x.astype(np.float64) ** 2)) - m0) < 1e-4
    c, s = orc.rope_tables(4, 8, 10000.0)
    x = np.arange(1, 5, dtype=np.float32)
    orc.lib.or_rope_apply(x, 2, c, s, 0)
    np.testing.assert_array_equal(x, np.arange(1, 5, dtype=np.float32))
    # table closed form: angle = pos / theta^(2i/d)
    c, s = orc.rope_tables(128, 64, 10000.0)
    pos, i = np.meshgrid(np.arange(64), np.arange(64), indexing="ij")
    ang = pos / 10000.0 ** (2 * i / 128)
    np.testing.assert_allclose(c.reshape(64, 64), np.cos(ang), atol=2e-5)
    np.testing.assert_allclose(s.reshape(64, 64), np.sin(ang), atol=2e-5)


def _attn64(orc, wq, wk, wv, wo, nh, nkv, d, x, pos, kc, vc, heads, theta=10000.0):
    W = lambda w: orc.bf16_to_f32(w).astype(np.float64)
    q, k, v = W(wq) @ x, W(wk) @ x, W(wv) @ x
    half = d // 2
    ang = pos / theta ** (2 * np.arange(half) / d)
    def rope(t):
        t = t.reshape(-1, d).copy()
        a, b = t[:, :half].copy(), t[:, half:].copy()
        t[:, :half] = a * np.cos(ang) - b * np.sin(ang)
        t[:, half:] = b * np.cos(ang) + a * np.sin(ang)
        return t
    q, k = rope(q), rope(k)
    K = kc[:, :pos + 1].astype(np.float64).copy()
    V = vc[:, :pos + 1].astype(np.float64).copy()
    K[:, pos], V[:, pos] = k, v.reshape(-1, d)
    cat = np.zeros(nh * d)
    g = nh // nkv
    for h in heads:
        sc = K[h // g] @ q[h] / np.sqrt(d)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        cat[h * d:(h + 1) * d] = p @ V[h // g]
    return W(wo) @ cat


@pytest.mark.parametrize("nh,nkv", [(4, 4), (8, 2)])
def test_sparse_attention_matches_float64(orc, nh, nkv):
    rng = np.random.default_rng(nh * 10 + nkv)
    d, hid, pos, max_seq = 16, 64, 37, 64
    b = lambda a: bf16r(orc, a)
    wq = b(rng.normal(0, 0.1, (nh * d, hid)))
    wk = b(rng.normal(0, 0.1, (nkv * d, hid)))
    wv = b(rng.normal(0, 0.1, (nkv * d, hid)))
    wo = b(rng.normal(0, 0.1, (hid, nh * d)))
    kc = rng.standard_normal((nkv, max_seq, d)).astype(np.float32)
    vc = rng.standard_normal((nkv, max_seq, d)).astype(np.float32)
    x = rng.standard_normal(hid).astype(np.float32)
    c, s = orc.rope_tables(d, max_seq, 10000.0)
    heads = [0, 2] if nh == 4 else [1, 4, 6, 7]
    ref = _attn64(orc, wq, wk, wv, wo, nh, nkv, d, x, pos, kc, vc, heads)
    kc2, vc2 = kc.copy(), vc.copy()
    out = orc.sparse_attention_forward_bf16(wq, wk, wv, wo, nh, nkv, d, x, pos, c, s, kc2, vc2, heads)
    np.testing.assert_allclose(out, ref, rtol=1e-4, atol=1e-5)
    # the appended row is the roped K and raw V of this token
    assert not np.array_equal(kc2[:, pos], kc[:, pos])
    np.testing.assert_array_equal(kc2[:, :pos], kc[:, :pos])


def test_dejavu_toy_mlp_sparse_equals_dense(orc):
    # klearu-dejavu mlp.rs:88-130: all neurons selected == dense SwiGLU within 1e-4
    rng = np.random.default_rng(5)
    H, I = 32, 64
    std = lambda a, b: np.sqrt(2.0 / (a + b))
    wg = rng.normal(0, std(H, I), (I, H)).astype(np.float32)
    wu = rng.normal(0, std(H, I), (I, H)).astype(np.float32)
    wd = rng.normal(0, std(I, H), (H, I)).astype(np.float32)
    z = lambda n: np.zeros(n, np.float32)
    x = np.full(H, 0.3, np.float32)
    y = orc.dejavu_sparse_mlp_forward(wg, z(I), wu, z(I), wd, z(H), x, np.arange(I))
    g = wg.astype(np.float64) @ x
    u = wu.astype(np.float64) @ x
    ref = wd.astype(np.float64) @ (g / (1 + np.exp(-g)) * u)
    np.testing.assert_allclose(y, ref, atol=1e-4)


def _bf(orc, rng, shape, s=0.02):
    return orc.bf16_to_f32(orc.bf16_from_f32(rng.normal(0, s, shape).astype(np.float32)))


def test_cpu_ffn_port_equals_composition(orc):
    """The timed AVX2 port (bench cpu_baseline) computes exactly rmsnorm ->
    predictor -> stable top-k -> sparse SwiGLU -> residual of the portable oracle."""
    rng = np.random.default_rng(3)
    H, I, R, k = 64, 160, 16, 24
    wg, wu, wd = _bf(orc, rng, (I, H)), _bf(orc, rng, (I, H)), _bf(orc, rng, (H, I))
    p1, p2 = _bf(orc, rng, (R, H)), _bf(orc, rng, (I, R))
    b1, b2 = np.zeros(R, np.float32), np.zeros(I, np.float32)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    hs = x.copy()
    scratch = np.zeros(H + I + R + k + H + 16, np.float32)
    act = np.zeros(k, np.int64)
    orc.lib.or_cpu_dejavu_ffn_layer(wg.reshape(-1), wu.reshape(-1), wd.reshape(-1), wn, 1e-5, p1.reshape(-1),
                                    b1, p2.reshape(-1), b2, R, H, I, k, hs, scratch, act)
    norm = orc.rmsnorm(x, wn, 1e-5)
    scores, _ = orc.predictor_predict(p1, b1, p2, b2, norm)
    sel = orc.select_top_k(scores, k)
    np.testing.assert_array_equal(act, sel)
    y, _ = orc.sparse_mlp_forward_bf16(orc.bf16_from_f32(wg), orc.bf16_from_f32(wu), orc.bf16_from_f32(wd),
                                       norm, sel)
    np.testing.assert_array_equal(hs, x + y)


def test_cpu_attention_port_equals_composition(orc):
    rng = np.random.default_rng(4)
    H, nh, nkv, d, R, k, S, pos = 128, 8, 4, 16, 12, 3, 40, 17
    wq, wk, wv, wo = (_bf(orc, rng, s) for s in ((nh * d, H), (nkv * d, H), (nkv * d, H), (H, nh * d)))
    p1, p2 = _bf(orc, rng, (R, H)), _bf(orc, rng, (nh, R))
    b1, b2 = np.zeros(R, np.float32), np.zeros(nh, np.float32)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    cos_t, sin_t = orc.rope_tables(d, S, 10000.0)
    kc = np.zeros((nkv, S, d), np.float32)
    vc = np.zeros_like(kc)
    kc[:, :pos] = rng.standard_normal((nkv, pos, d))
    vc[:, :pos] = rng.standard_normal((nkv, pos, d))
    kc2, vc2 = kc.copy(), vc.copy()
    x = rng.standard_normal(H).astype(np.float32)
    hs = x.copy()
    scratch = np.zeros(2 * H + 2 * nh * d + 2 * nkv * d + nh + R + S + 16, np.float32)
    heads = np.zeros(k, np.int64)
    orc.lib.or_cpu_sparse_attention_layer(wq.reshape(-1), wk.reshape(-1), wv.reshape(-1), wo.reshape(-1), wn,
                                          1e-5, p1.reshape(-1), b1, p2.reshape(-1), b2, R, H, nh, nkv, d, k,
                                          cos_t, sin_t, kc.reshape(-1), vc.reshape(-1), S, pos, hs, scratch,
                                          heads)
    norm = orc.rmsnorm(x, wn, 1e-5)
    scores, _ = orc.predictor_predict(p1, b1, p2, b2, norm)
    sel = orc.select_top_k(scores, k)
    np.testing.assert_array_equal(heads, sel)
    out = orc.sparse_attention_forward_bf16(*(orc.bf16_from_f32(w) for w in (wq, wk, wv, wo)), nh, nkv, d, norm,
                                            pos, cos_t, sin_t, kc2, vc2, sel)
    np.testing.assert_array_equal(hs, x + out)
    np.testing.assert_array_equal(kc, kc2)


def _xavier(rng, out_f, in_f):
    return rng.normal(0, np.sqrt(2.0 / (in_f + out_f)), (out_f, in_f)).astype(np.float32)


def test_dejavu_linear_dense_and_sparse(orc):
    """transformer/mod.rs:114-134: forward over all rows == forward_sparse over
    0..out, rows in any order and repeated; float64 bound on every output."""
    rng = np.random.default_rng(8)
    w, b = _xavier(rng, 48, 40), rng.normal(0, 0.1, 48).astype(np.float32)
    x = rng.standard_normal(40).astype(np.float32)
    d = orc.dejavu_linear_forward(w, b, x)
    np.testing.assert_array_equal(d, orc.dejavu_linear_forward_sparse(w, b, x, np.arange(48)))
    idx = np.array([7, 3, 3, 47, 0])
    np.testing.assert_array_equal(orc.dejavu_linear_forward_sparse(w, b, x, idx), d[idx])
    ref = w.astype(np.float64) @ x + b
    bound = 41 * 2 ** -23 * (np.abs(w.astype(np.float64)) @ np.abs(x) + np.abs(b))
    assert np.all(np.abs(d - ref) <= bound)


def test_dejavu_toy_attention_all_heads_equals_dense(orc):
    """attention.rs:119-160 (hidden 64, 4 heads x 16): every head selected ==
    the dense restatement (full q/k/v, sigmoid score per head, dense o_proj)
    within 1e-5; two heads selected == the dense formula with the other
    heads' outputs zeroed, in float64 within 1e-5."""
    rng = np.random.default_rng(10)
    H, nh, hd = 64, 4, 16
    ws = [_xavier(rng, nh * hd, H) for _ in range(3)] + [_xavier(rng, H, nh * hd)]
    bs = [np.zeros(nh * hd, np.float32)] * 3 + [np.zeros(H, np.float32)]
    x = np.full(H, 0.5, np.float32)

    def dense(sel):
        q, k, v = (w.astype(np.float64) @ x for w in ws[:3])
        att = np.zeros(nh * hd)
        for h in sel:
            s = slice(h * hd, (h + 1) * hd)
            att[s] = v[s] / (1 + np.exp(-(q[s] @ k[s]) / np.sqrt(hd)))
        return ws[3].astype(np.float64) @ att

    args = [a for pair in zip(ws, bs) for a in pair]
    y = orc.dejavu_sparse_attention_forward(*args, nh, hd, x, np.arange(nh))
    np.testing.assert_allclose(y, dense(range(nh)), atol=1e-5)
    y2 = orc.dejavu_sparse_attention_forward(*args, nh, hd, x, [2, 0])
    np.testing.assert_allclose(y2, dense([0, 2]), atol=1e-5)
    # repeated heads recompute the same values
    np.testing.assert_array_equal(orc.dejavu_sparse_attention_forward(*args, nh, hd, x, [2, 0, 2]), y2)
