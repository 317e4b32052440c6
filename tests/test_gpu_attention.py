"""GPU parity: head-sparse decode attention vs the oracle.

Bar (north_star): BF16-weight outputs within 2e-3 relative, elementwise, with
an absolute floor of 1e-4 x max|ref| for entries near zero (max-abs printed).
The oracle restates sparse_attention::forward_sparse with an f32 KvCache
(kv_cache.rs:33-48), unchanged: appended rows stay f32 on both sides.  The
default KH_KV_BF16 handle keeps loaded rows that are BF16 values in BF16 (the
preloaded caches here are BF16-valued, as in cfg4) and every other row in f32,
so it holds exactly the reference's cache.
Shapes: cfg4 (hidden 4096, 32 heads x 128, cache 2048, 16 heads selected,
batch 1 and 8) plus small edge cases (GQA, empty cache, duplicate and
out-of-range head ids, full cache, explicit positions).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

RTOL = 2e-3


def close(got, ref, what=""):
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    err = float(np.max(np.abs(got - ref))) if ref.size else 0.0
    print(f"{what} max|ref|={scale:.4g} max-abs-err={err:.3g}")
    np.testing.assert_allclose(got, ref, rtol=RTOL, atol=1e-4 * scale + 1e-30)


def close_row(got, ref, kv, what=""):
    """An appended cache row: f32 on both sides (the projection's order differs)."""
    return close(got, ref, what)


def check_scale(orc, h_in, ws, what):
    """The RmsNorm scale a fused block wrote (norm_ws) is rms_norm.rs:48-52's, bit for bit."""
    inv = np.array([orc.rms_inv(h_in, 1e-5)], np.float32)
    got = ws.cpu().numpy()[:1]
    print(f"{what}: norm scale {float(got[0])!r} (oracle {float(inv[0])!r})")
    np.testing.assert_array_equal(got.view(np.uint32), inv.view(np.uint32), err_msg=f"{what}: norm scale")


def bf16_round(orc, a):
    return orc.bf16_to_f32(orc.bf16_from_f32(np.asarray(a, np.float32)))


class Case:
    """Weights, a preloaded cache per sequence and the oracle's own f32 caches."""

    def __init__(self, orc, rng, hidden, nh, nkv, d, max_seq, batch, pre_len, kv_dtype=0, theta=10000.0):
        from klearu_amd.attention import SparseAttention
        self.orc, self.hidden, self.nh, self.nkv, self.d, self.max_seq = orc, hidden, nh, nkv, d, max_seq
        self.kv_bf16 = kv_dtype == 0
        b16 = lambda shape, s: orc.bf16_from_f32(rng.normal(0, s, shape).astype(np.float32))  # noqa: E731
        self.wq = b16((nh * d, hidden), 0.02)
        self.wk = b16((nkv * d, hidden), 0.02)
        self.wv = b16((nkv * d, hidden), 0.02)
        self.wo = b16((hidden, nh * d), 0.02)
        self.attn = SparseAttention(hidden, nh, nkv, d, self.wq, self.wk, self.wv, self.wo, max_seq, batch,
                                    theta, kv_dtype)
        self.cos, self.sin = orc.rope_tables(d, max_seq, theta)
        self.kc = np.zeros((batch, nkv, max_seq, d), np.float32)
        self.vc = np.zeros_like(self.kc)
        self.len = [0] * batch
        for b in range(batch):
            L = pre_len[b] if isinstance(pre_len, (list, tuple)) else pre_len
            k = bf16_round(orc, rng.standard_normal((nkv, L, d)))
            v = bf16_round(orc, rng.standard_normal((nkv, L, d)))
            self.kc[b, :, :L] = k
            self.vc[b, :, :L] = v
            self.attn.load_cache(b, k, v)
            self.len[b] = L

    def oracle_step(self, b, x, heads, pos=None):
        p = self.len[b] if pos is None else pos
        assert p == self.len[b], "the oracle appends at the RoPE position"
        kc, vc = self.kc[b].copy(), self.vc[b].copy()
        out = self.orc.sparse_attention_forward_bf16(self.wq, self.wk, self.wv, self.wo, self.nh, self.nkv, self.d,
                                                     x, p, self.cos, self.sin, kc, vc, [h for h in heads])
        self.kc[b], self.vc[b] = kc, vc
        self.len[b] += 1
        return out


@pytest.mark.parametrize("hidden,nh,nkv,d,max_seq,pre,kv", [
    (512, 8, 8, 64, 400, 300, 0),
    (512, 8, 2, 128, 300, 129, 0),   # GQA, chunk boundary
    (256, 4, 4, 256, 200, 100, 0),
    (512, 8, 8, 64, 400, 255, 1),    # f32 cache
    (512, 8, 2, 128, 300, 64, 1),
    (256, 4, 1, 256, 100, 0, 0),     # empty cache: first token
])
def test_decode_step_matches_oracle(kh, orc, hidden, nh, nkv, d, max_seq, pre, kv):
    rng = np.random.default_rng(hidden + nh + d + pre + kv)
    c = Case(orc, rng, hidden, nh, nkv, d, max_seq, 1, pre, kv)
    heads = sorted(rng.choice(nh, nh // 2, replace=False).tolist())
    x = rng.standard_normal(hidden).astype(np.float32)
    got = c.attn.forward_sparse(x[None], [heads])[0].cpu().numpy()
    ref = c.oracle_step(0, x, heads)
    close(got, ref, f"step nh{nh} nkv{nkv} d{d} pre{pre} kv{kv}")
    assert c.attn.current_len(0) == pre + 1
    # appended row (roped k, v) equals the oracle's, to rounding
    k, v = c.attn.read_cache(0, pre + 1)
    close_row(k[:, pre], c.kc[0][:, pre], kv, "appended k")
    close_row(v[:, pre], c.vc[0][:, pre], kv, "appended v")
    np.testing.assert_array_equal(k[:, :pre], c.kc[0][:, :pre])


@pytest.mark.parametrize("kv", [0, 1])
def test_multi_step_decode(kh, orc, kv):
    rng = np.random.default_rng(5 + kv)
    c = Case(orc, rng, 384, 6, 3, 64, 64, 1, 60, kv)
    for step in range(4):   # fills the cache exactly
        heads = sorted(rng.choice(6, 3, replace=False).tolist())
        x = rng.standard_normal(384).astype(np.float32)
        got = c.attn.forward_sparse(x[None], [heads])[0].cpu().numpy()
        close(got, c.oracle_step(0, x, heads), f"step {step}")
    assert c.attn.current_len(0) == 64
    from klearu_amd import KlearuError
    with pytest.raises(KlearuError) as e:
        c.attn.forward_sparse(np.zeros((1, 384), np.float32), [[0]])
    assert e.value.code == -3
    c.attn.clear()
    assert c.attn.current_len(0) == 0


def test_head_list_edge_cases(kh, orc):
    rng = np.random.default_rng(9)
    c = Case(orc, rng, 256, 8, 4, 64, 100, 1, 50)
    x = rng.standard_normal(256).astype(np.float32)
    # duplicates add the head output twice; ids >= num_heads are skipped
    heads = [3, 1, 3, 8, 100]
    got = c.attn.forward_sparse(x[None], [heads])[0].cpu().numpy()
    close(got, c.oracle_step(0, x, heads), "duplicates / out of range")
    # negative ids are skipped too (the reference's ids are unsigned)
    x = rng.standard_normal(256).astype(np.float32)
    got = c.attn.forward_sparse(x[None], [[-1, 5, -7]])[0].cpu().numpy()
    close(got, c.oracle_step(0, x, [5]), "negative ids")
    # no heads: zero output, but K/V are still appended
    x = rng.standard_normal(256).astype(np.float32)
    got = c.attn.forward_sparse(x[None], np.zeros((1, 0), np.int32))[0].cpu().numpy()
    ref = c.oracle_step(0, x, [])
    np.testing.assert_array_equal(got, np.zeros(256, np.float32))
    np.testing.assert_array_equal(ref, np.zeros(256, np.float32))
    assert c.attn.current_len(0) == 53
    k, v = c.attn.read_cache(0, 53)
    close_row(k[:, 52], c.kc[0][:, 52], 0, "k appended with no heads")


def test_accumulate_and_explicit_positions(kh, orc):
    rng = np.random.default_rng(11)
    c = Case(orc, rng, 256, 4, 4, 64, 80, 2, [10, 30])
    x = rng.standard_normal((2, 256)).astype(np.float32)
    heads = [[0, 2], [1, 3]]
    base = torch.from_numpy(rng.standard_normal((2, 256)).astype(np.float32)).cuda()
    out = base.clone()
    c.attn.forward_sparse(x, heads, positions=[10, 30], out=out, accumulate=True)
    got = (out - base).cpu().numpy()
    for b in range(2):
        close(got[b], c.oracle_step(b, x[b], heads[b]), f"seq {b}")


@pytest.mark.parametrize("batch", [1, 2, 3, 16])
def test_long_context_and_duplicates(kh, orc, batch):
    """More than 16 cache chunks per head (head_dim 256: 64 positions per
    chunk) and repeated heads, with the chunks merged inside the o_proj kernel
    (batch <= 2) and by the separate merge kernel (batch > 2); hidden 1024
    puts the batched q/k/v projections on the matrix cores."""
    rng = np.random.default_rng(77 + batch)
    c = Case(orc, rng, 1024, 4, 2, 256, 1400, batch, [1300 - 40 * b for b in range(batch)])
    x = rng.standard_normal((batch, 1024)).astype(np.float32)
    heads = [[(b + 2) % 4, b % 4, (b + 2) % 4] for b in range(batch)]
    got = c.attn.forward_sparse(x, heads).cpu().numpy()
    for b in range(batch):
        close(got[b], c.oracle_step(b, x[b], heads[b]), f"seq {b}")


@pytest.mark.parametrize("batch", [1, 8])
def test_cfg4_7b_shape(kh, orc, batch):
    """cfg4: hidden 4096, 32 heads x 128, KV cache of 2048 positions (2047
    filled, this step writes the last), 16 of 32 heads per token."""
    rng = np.random.default_rng(4096 + batch)
    pre = [2047 - 97 * b for b in range(batch)]   # ragged lengths across the batch
    c = Case(orc, rng, 4096, 32, 32, 128, 2048, batch, pre)
    x = rng.standard_normal((batch, 4096)).astype(np.float32)
    heads = [sorted(rng.choice(32, 16, replace=False).tolist()) for _ in range(batch)]
    got = c.attn.forward_sparse(x, heads).cpu().numpy()
    for b in range(batch):
        close(got[b], c.oracle_step(b, x[b], heads[b]), f"cfg4 b{b}")


@pytest.mark.parametrize("kv", [0, 1])
def test_load_cache_dev_matches_host_load(kh, orc, kv):
    rng = np.random.default_rng(21 + kv)
    c = Case(orc, rng, 256, 4, 2, 64, 50, 2, [0, 0], kv)
    k = rng.standard_normal((2, 37, 64)).astype(np.float32)
    v = rng.standard_normal((2, 37, 64)).astype(np.float32)
    c.attn.load_cache(0, k, v)
    c.attn.load_cache_dev(1, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    assert c.attn.current_len(0) == 37 and c.attn.current_len(1) == 37
    k0, v0 = c.attn.read_cache(0, 37)
    k1, v1 = c.attn.read_cache(1, 37)
    np.testing.assert_array_equal(k0, k1)
    np.testing.assert_array_equal(v0, v1)
    # rows that are not BF16 values are kept in f32 by either kind of handle
    np.testing.assert_array_equal(k0, k)
    np.testing.assert_array_equal(k1, k)


@pytest.mark.parametrize("bf16_values", [True, False])
def test_device_load_decides_storage_exactly(kh, orc, bf16_values):
    """load_cache_dev on a KH_KV_BF16 handle: BF16-valued rows (a BF16 model's
    prefill) become a BF16 prefix, others stay f32; either way the decode
    equals the host-loaded cache's and the unrounded oracle's."""
    rng = np.random.default_rng(61 + bf16_values)
    c = Case(orc, rng, 256, 4, 2, 64, 60, 2, [0, 0], 0)
    k = rng.standard_normal((2, 45, 64)).astype(np.float32)
    v = rng.standard_normal((2, 45, 64)).astype(np.float32)
    if bf16_values:
        k, v = bf16_round(orc, k), bf16_round(orc, v)
    c.attn.load_cache(0, k, v)
    c.attn.load_cache_dev(1, torch.from_numpy(k).cuda(), torch.from_numpy(v).cuda())
    for b in range(2):
        c.kc[b][:, :45], c.vc[b][:, :45], c.len[b] = k, v, 45
    for step in range(3):
        x = rng.standard_normal((2, 256)).astype(np.float32)
        heads = [[0, 2], [0, 2]]
        got = c.attn.forward_sparse(x, heads).cpu().numpy()
        for b in range(2):
            close(got[b], c.oracle_step(b, x[b], heads[b]), f"device load bf16={bf16_values} step {step}")
    k1, _ = c.attn.read_cache(1, 48)
    np.testing.assert_array_equal(k1[:, :45], k)


def test_rejects_bad_shapes(kh, orc):
    from klearu_amd import KlearuError
    from klearu_amd.attention import SparseAttention
    w = np.zeros((4 * 96, 64), np.uint16)
    wo = np.zeros((64, 4 * 96), np.uint16)
    with pytest.raises(KlearuError):
        SparseAttention(64, 4, 4, 96, w, w, w, wo, 16)     # head_dim 96 unsupported
    w = np.zeros((3 * 64, 64), np.uint16)
    with pytest.raises(KlearuError):
        SparseAttention(64, 3, 2, 64, w, np.zeros((128, 64), np.uint16), np.zeros((128, 64), np.uint16),
                        np.zeros((64, 192), np.uint16), 16)   # 3 heads over 2 kv heads


@pytest.mark.parametrize("H,nh,nkv,d,R,k,pre,steps", [
    (4096, 32, 32, 128, 128, 16, 2000, 4),   # cfg4 (7B): 32 heads x 128, cache ~2048, top 50% of heads
    (512, 8, 4, 64, 32, 3, 20, 3),           # GQA, small
    (512, 8, 8, 64, 160, 3, 20, 2),          # head predictor wider than a wave's chain: separate top k
])
def test_attn_block_chained(kh, orc, H, nh, nkv, d, R, k, pre, steps):
    """kh_dejavu_attn_block over several decode steps against the oracle's
    RmsNorm -> head predictor -> select_top_k -> sparse attention -> residual
    (crates/klearu-llm/src/sparse/mod.rs:56-112).  For each step the oracle
    runs on the hidden row the GPU held before the block: the head set must
    equal the oracle's own top-k exactly, and the updated row must match the
    oracle's residual from the oracle's selection within the BF16-weight
    tolerance."""
    from klearu_amd.attention import attn_block
    from klearu_amd.dejavu import SparsityPredictor
    rng = np.random.default_rng(41 + H)
    c = Case(orc, rng, H, nh, nkv, d, pre + steps + 4, 1, pre)
    w1 = orc.bf16_from_f32(rng.normal(0, 0.05, (R, H)).astype(np.float32))
    w2 = orc.bf16_from_f32(rng.normal(0, 0.3, (nh, R)).astype(np.float32))
    b1 = rng.normal(0, 0.1, R).astype(np.float32)
    b2 = rng.normal(0, 0.1, nh).astype(np.float32)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    hd = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).cuda()
    wnd = torch.from_numpy(wn).cuda()
    ws = torch.empty(1, dtype=torch.float32, device="cuda")
    for step in range(steps):
        h_in = hd.cpu().numpy().copy()
        heads = attn_block(p, c.attn, hd, wnd, 1e-5, k, norm_ws=ws)
        check_scale(orc, h_in, ws, f"step {step}")
        norm = orc.rmsnorm(h_in, wn, 1e-5)
        scores, _ = orc.predictor_predict(w1, b1, w2, b2, norm)
        sel = np.sort(orc.select_top_k(scores, k))
        got = heads.cpu().numpy()
        np.testing.assert_array_equal(got, sel)
        want = h_in + c.oracle_step(0, norm, sel.tolist())
        close(hd.cpu().numpy(), want, f"step {step}")
    assert c.attn.current_len(0) == pre + steps


def _head_predictor(orc, rng, H, nh, R):
    from klearu_amd.dejavu import SparsityPredictor
    w1 = orc.bf16_from_f32(rng.normal(0, 0.05, (R, H)).astype(np.float32))
    w2 = orc.bf16_from_f32(rng.normal(0, 0.3, (nh, R)).astype(np.float32))
    b1 = rng.normal(0, 0.1, R).astype(np.float32)
    b2 = rng.normal(0, 0.1, nh).astype(np.float32)
    return (w1, b1, w2, b2), SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)


def _batch_block_step(orc, c, pw, p, hd, wn, wnd, ws, k, what):
    """One kh_dejavu_attn_block_batch call checked row by row against the oracle."""
    from klearu_amd.attention import attn_block_batch
    w1, b1, w2, b2 = pw
    h_in = hd.cpu().numpy().copy()
    ws.fill_(float("nan"))
    heads = attn_block_batch(p, c.attn, hd, wnd, 1e-5, k, norm_ws=ws).cpu().numpy()
    got = hd.cpu().numpy()
    scales = ws.cpu().numpy()
    for b in range(h_in.shape[0]):
        inv = np.array([orc.rms_inv(h_in[b], 1e-5)], np.float32)
        np.testing.assert_array_equal(scales[b:b + 1].view(np.uint32), inv.view(np.uint32),
                                      err_msg=f"{what} row {b}: norm scale")
        norm = orc.rmsnorm(h_in[b], wn, 1e-5)
        scores, _ = orc.predictor_predict(w1, b1, w2, b2, norm)
        sel = np.sort(orc.select_top_k(scores, k))
        np.testing.assert_array_equal(heads[b], sel, err_msg=f"{what} row {b}: heads")
        close(got[b], h_in[b] + c.oracle_step(b, norm, sel.tolist()), f"{what} row {b}")


@pytest.mark.parametrize("H,nh,nkv,d,R,k,pre,B,steps", [
    (4096, 32, 32, 128, 128, 16, 2000, 8, 2),   # cfg4 (7B), batch 8
    (1024, 16, 4, 64, 64, 5, 70, 3, 3),         # GQA, ragged batch
    (1024, 8, 8, 128, 128, 8, 40, 16, 2),       # k = every head, batch 16
    # hidden a multiple of 2048: the K/V rows in the head predictor's launch
    (2048, 16, 4, 64, 64, 6, 90, 5, 2),         # GQA
])
def test_attn_block_batch_chained(kh, orc, H, nh, nkv, d, R, k, pre, B, steps):
    """kh_dejavu_attn_block_batch: every row's RmsNorm scale is the
    reference's bit for bit (rms_norm.rs:43-53), its head set equals the
    oracle's own top k (selected inside the q/k/v projection here), and the
    updated rows match the oracle's residual from that selection
    (crates/klearu-llm/src/sparse/mod.rs:56-112, one token per sequence) within
    the BF16-weight tolerance, over several steps and cache lengths."""
    rng = np.random.default_rng(57 + H + B)
    lens = [max(0, pre - 3 * b) for b in range(B)]  # row 15 of batch 16: an empty cache
    c = Case(orc, rng, H, nh, nkv, d, pre + steps + 4, B, lens)
    pw, p = _head_predictor(orc, rng, H, nh, R)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    wnd = torch.from_numpy(wn).cuda()
    hd = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda()
    ws = torch.empty(B, dtype=torch.float32, device="cuda")
    for step in range(steps):
        _batch_block_step(orc, c, pw, p, hd, wn, wnd, ws, k, f"step {step}")
    for b in range(B):
        assert c.attn.current_len(b) == lens[b] + steps


def test_attn_block_batch_hard_norm_rows(kh, orc):
    """kh_dejavu_attn_block_batch fed the hard RmsNorm rows (ties stuck at
    2^24, round-up drift, leading zeros, all-zero, tiny, huge, wide-range) as
    one batch at the 7B shape: scales, heads and residuals as above."""
    from hard_rows import hard_hidden_rows
    H, nh, d, R, k, pre = 4096, 32, 128, 128, 16, 600
    rng = np.random.default_rng(97)
    rows = list(hard_hidden_rows(rng, H).values())[:16]
    B = len(rows)
    c = Case(orc, rng, H, nh, nh, d, pre + 4, B, pre)
    pw, p = _head_predictor(orc, rng, H, nh, R)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    wnd = torch.from_numpy(wn).cuda()
    hd = torch.from_numpy(np.stack(rows).astype(np.float32)).cuda()
    ws = torch.empty(B, dtype=torch.float32, device="cuda")
    _batch_block_step(orc, c, pw, p, hd, wn, wnd, ws, k, "hard rows")


@pytest.mark.parametrize("H,nh,d,R,k,pre", [
    (4096, 32, 128, 128, 16, 2000),   # cfg4 (7B)
    (2048, 16, 128, 128, 8, 300),     # a 1.1B-class width
])
def test_attn_block_hard_norm_rows(kh, orc, H, nh, d, R, k, pre):
    """kh_dejavu_attn_block fed hidden rows whose sum of squares defeats the
    exact sum's speculative windows (ties stuck at 2^24, round-up drift),
    leading zeros, an all-zero row, tiny, huge and wide-range magnitudes: the
    RmsNorm scale it writes is the reference's bit for bit, the head set is
    the oracle's, and the residual is within tolerance (rms_norm.rs:43-53,
    sparse/mod.rs:56-112)."""
    from hard_rows import hard_hidden_rows
    from klearu_amd.attention import attn_block
    from klearu_amd.dejavu import SparsityPredictor
    rng = np.random.default_rng(83 + H)
    rows = hard_hidden_rows(rng, H)
    c = Case(orc, rng, H, nh, nh, d, pre + len(rows) + 4, 1, pre)
    w1 = orc.bf16_from_f32(rng.normal(0, 0.05, (R, H)).astype(np.float32))
    w2 = orc.bf16_from_f32(rng.normal(0, 0.3, (nh, R)).astype(np.float32))
    b1 = rng.normal(0, 0.1, R).astype(np.float32)
    b2 = rng.normal(0, 0.1, nh).astype(np.float32)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    wnd = torch.from_numpy(wn).cuda()
    ws = torch.empty(1, dtype=torch.float32, device="cuda")
    for name, row in rows.items():
        hd = torch.from_numpy(row.copy()).cuda()
        ws.fill_(float("nan"))
        heads = attn_block(p, c.attn, hd, wnd, 1e-5, k, norm_ws=ws)
        check_scale(orc, row, ws, name)
        norm = orc.rmsnorm(row, wn, 1e-5)
        scores, _ = orc.predictor_predict(w1, b1, w2, b2, norm)
        sel = np.sort(orc.select_top_k(scores, k))
        np.testing.assert_array_equal(heads.cpu().numpy(), sel, err_msg=name)
        close(hd.cpu().numpy(), row + c.oracle_step(0, norm, sel.tolist()), name)


def test_decoder_layers_chained_7b(kh, orc):
    """Two sparse decoder layers at the 7B shape, as
    SparseModel::forward_decode_sparse runs them (crates/klearu-llm/src/sparse/mod.rs:55-143):
    per layer kh_dejavu_attn_block (RmsNorm -> head predictor -> top 16 of 32
    heads -> sparse attention over a ~2000-token cache -> residual) then
    kh_dejavu_mlp_block (RmsNorm -> neuron predictor -> top 1652 of 11008 ->
    sparse SwiGLU -> residual).  For every block the oracle runs on the
    hidden row the GPU held before it: the selection must equal the oracle's
    exactly, and the updated row the oracle's residual within the
    BF16-weight tolerance."""
    from klearu_amd.attention import attn_block
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block
    rng = np.random.default_rng(2024)
    H, nh, d, I, Rh, Rn, kh_, kn, pre = 4096, 32, 128, 11008, 128, 256, 16, 1652, 2000
    bf = lambda a: orc.bf16_from_f32(np.asarray(a, np.float32))  # noqa: E731
    hd = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).cuda()
    ws = torch.empty(1, dtype=torch.float32, device="cuda")
    for layer in range(2):
        c = Case(orc, rng, H, nh, nh, d, pre + 8, 1, pre)
        hw1, hw2 = bf(rng.normal(0, 0.05, (Rh, H))), bf(rng.normal(0, 0.3, (nh, Rh)))
        hb1, hb2 = rng.normal(0, 0.1, Rh).astype(np.float32), rng.normal(0, 0.1, nh).astype(np.float32)
        hp = SparsityPredictor(orc.bf16_to_f32(hw1), hb1, orc.bf16_to_f32(hw2), hb2)
        nw1, nw2 = bf(rng.normal(0, 0.02, (Rn, H))), bf(rng.normal(0, 0.02, (I, Rn)))
        nb1, nb2 = rng.normal(0, 0.1, Rn).astype(np.float32), rng.normal(0, 0.1, I).astype(np.float32)
        npred = SparsityPredictor(orc.bf16_to_f32(nw1), nb1, orc.bf16_to_f32(nw2), nb2)
        wg, wu = bf(rng.normal(0, 0.02, (I, H))), bf(rng.normal(0, 0.02, (I, H)))
        wd = bf(rng.normal(0, 0.02, (H, I)))
        mlp = Mlp(wg, wu, wd, max_batch=1)
        wn_a = rng.uniform(0.5, 1.5, H).astype(np.float32)
        wn_m = rng.uniform(0.5, 1.5, H).astype(np.float32)
        # attention half
        h_in = hd.cpu().numpy().copy()
        heads = attn_block(hp, c.attn, hd, torch.from_numpy(wn_a).cuda(), 1e-5, kh_, norm_ws=ws)
        check_scale(orc, h_in, ws, f"layer {layer} attention")
        norm = orc.rmsnorm(h_in, wn_a, 1e-5)
        s, _ = orc.predictor_predict(hw1, hb1, hw2, hb2, norm)
        sel = np.sort(orc.select_top_k(s, kh_))
        np.testing.assert_array_equal(heads.cpu().numpy(), sel)
        close(hd.cpu().numpy(), h_in + c.oracle_step(0, norm, sel.tolist()), f"layer {layer} attention")
        # MLP half
        h_in = hd.cpu().numpy().copy()
        act = mlp_block(npred, mlp, hd, torch.from_numpy(wn_m).cuda(), 1e-5, kn, norm_ws=ws)
        check_scale(orc, h_in, ws, f"layer {layer} MLP")
        norm = orc.rmsnorm(h_in, wn_m, 1e-5)
        s, _ = orc.predictor_predict(nw1, nb1, nw2, nb2, norm)
        sel = np.sort(orc.select_top_k(s, kn))
        np.testing.assert_array_equal(act.cpu().numpy(), sel)
        y, _ = orc.sparse_mlp_forward_bf16(wg, wu, wd, norm, sel.astype(np.int64))
        close(hd.cpu().numpy(), h_in + y, f"layer {layer} MLP")


def _decoder_layer(orc, seed, H, nh, nkv, d, I, Rh, Rn, pre, max_seq, B):
    """A sparse decoder layer's handles from one seed: the attention weights and
    preloaded caches, the head predictor, the neuron predictor and the MLP."""
    from klearu_amd.dejavu import Mlp, SparsityPredictor
    rng = np.random.default_rng(seed)
    bf = lambda a: orc.bf16_from_f32(np.asarray(a, np.float32))  # noqa: E731
    c = Case(orc, rng, H, nh, nkv, d, max_seq, B, pre)
    _, hp = _head_predictor(orc, rng, H, nh, Rh)
    nw1, nw2 = bf(rng.normal(0, 0.02, (Rn, H))), bf(rng.normal(0, 0.02, (I, Rn)))
    nb1, nb2 = rng.normal(0, 0.1, Rn).astype(np.float32), rng.normal(0, 0.1, I).astype(np.float32)
    npred = SparsityPredictor(orc.bf16_to_f32(nw1), nb1, orc.bf16_to_f32(nw2), nb2)
    wg, wu = bf(rng.normal(0, 0.02, (I, H))), bf(rng.normal(0, 0.02, (I, H)))
    mlp = Mlp(wg, wu, bf(rng.normal(0, 0.02, (H, I))), max_batch=B)
    return c.attn, hp, npred, mlp


@pytest.mark.parametrize("B", [1, 4])
def test_decoder_layer_graph_replays_match_eager(kh, orc, B):
    """One sparse decoder layer step (kh_dejavu_attn_block[_batch], then
    kh_dejavu_mlp_block[_batch]) captured in a HIP graph, as bench.py times it,
    and replayed step after step while the KV caches grow on the device.  A
    twin layer (the same weights and caches) runs the same steps eagerly on
    the same stream between the replays.  After every replay the rows, head
    sets, neuron sets and RmsNorm scales equal the eager step's bit for bit
    (the same kernels on the same inputs), and so do the cache lengths read
    back from the device."""
    from klearu_amd.attention import attn_block, attn_block_batch
    from klearu_amd.dejavu import mlp_block, mlp_block_batch
    H, nh, nkv, d, I, Rh, Rn, kh_, kn, pre, steps = 2048, 32, 4, 64, 5632, 64, 128, 8, 845, 150, 5
    pres = [pre - 5 * b for b in range(B)]  # ragged caches
    eager = _decoder_layer(orc, 77, H, nh, nkv, d, I, Rh, Rn, pres, pre + steps + 8, B)
    graph = _decoder_layer(orc, 77, H, nh, nkv, d, I, Rh, Rn, pres, pre + steps + 8, B)
    rng = np.random.default_rng(5)
    x0 = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda()
    wn_a = torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).cuda()
    wn_m = torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).cuda()

    def state():
        return dict(h=x0.clone(), heads=torch.full((B, kh_), -1, dtype=torch.int32, device="cuda"),
                    act=torch.full((B, kn), -1, dtype=torch.int32, device="cuda"),
                    wsa=torch.zeros(B, device="cuda"), wsm=torch.zeros(B, device="cuda"))

    def step(layer, t, s):
        attn, hp, npred, mlp = layer
        if B == 1:
            attn_block(hp, attn, t["h"][0], wn_a, 1e-5, kh_, heads=t["heads"][0], norm_ws=t["wsa"], stream=s)
            mlp_block(npred, mlp, t["h"][0], wn_m, 1e-5, kn, active=t["act"][0], norm_ws=t["wsm"], stream=s)
        else:
            attn_block_batch(hp, attn, t["h"], wn_a, 1e-5, kh_, heads=t["heads"], norm_ws=t["wsa"], stream=s)
            mlp_block_batch(npred, mlp, t["h"], wn_m, 1e-5, kn, active=t["act"], norm_ws=t["wsm"], stream=s)

    def same(te, tg, what):
        for key in ("h", "wsa", "wsm"):
            np.testing.assert_array_equal(tg[key].cpu().numpy().view(np.uint32), te[key].cpu().numpy().view(np.uint32),
                                          err_msg=f"{what}: {key}")
        for key in ("heads", "act"):
            np.testing.assert_array_equal(tg[key].cpu().numpy(), te[key].cpu().numpy(), err_msg=f"{what}: {key}")

    te, tg = state(), state()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step(eager, te, s)  # the warm-up call sizes the scratch buffers the capture records
        step(graph, tg, s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            step(graph, tg, s)
    torch.cuda.synchronize()
    same(te, tg, "warm-up step")
    for i in range(steps):
        with torch.cuda.stream(s):
            step(eager, te, s)
            s.synchronize()
            g.replay()
        torch.cuda.synchronize()
        print(f"B={B} replay {i}: heads {tg['heads'][0, :4].tolist()} ...", flush=True)
        same(te, tg, f"replay {i}")
        for b in range(B):
            assert graph[0].current_len(b) == eager[0].current_len(b) == pres[b] + 2 + i


@pytest.mark.parametrize("pre", [0, 200])
def test_bf16_handle_matches_unrounded_reference_cache(kh, orc, pre):
    """A default (KH_KV_BF16) handle over many decode steps against the oracle's
    f32 KvCache with unrounded appended rows (kv_cache.rs:33-48), from an empty
    cache and from a BF16-valued prefill; an f32 handle fed the same steps
    stays within the same bar, and the appended rows read back are f32."""
    rng = np.random.default_rng(40 + pre)
    hidden, nh, nkv, d, steps = 512, 8, 2, 128, 40
    c16 = Case(orc, rng, hidden, nh, nkv, d, pre + steps, 1, pre, 0)
    from klearu_amd.attention import SparseAttention
    c32 = SparseAttention(hidden, nh, nkv, d, c16.wq, c16.wk, c16.wv, c16.wo, pre + steps, 1, 10000.0, 1)
    if pre:
        k, v = c16.attn.read_cache(0, pre)
        c32.load_cache(0, k, v)
    for step in range(steps):
        heads = sorted(rng.choice(nh, 4, replace=False).tolist())
        x = rng.standard_normal(hidden).astype(np.float32)
        g16 = c16.attn.forward_sparse(x[None], [heads])[0].cpu().numpy()
        g32 = c32.forward_sparse(x[None], [heads])[0].cpu().numpy()
        ref = c16.oracle_step(0, x, heads)
        close(g16, ref, f"bf16 handle step {step}")
        close(g32, ref, f"f32 handle step {step}")
    k16, v16 = c16.attn.read_cache(0, pre + steps)
    k32, _ = c32.read_cache(0, pre + steps)
    np.testing.assert_array_equal(k16[:, :pre], c16.kc[0][:, :pre])
    close(k16[:, pre:], c16.kc[0][:, pre:pre + steps], "appended k rows")
    close(v16[:, pre:], c16.vc[0][:, pre:pre + steps], "appended v rows")
    # appended rows are f32: some carry bits a BF16 row cannot hold
    assert np.any(k16[:, pre:].view(np.uint32) & 0xffff)
    close(k16, k32, "bf16 vs f32 handle cache")
