"""GPU parity: Deja Vu predictor, top-k, union and sparse SwiGLU FFN vs the oracle.

Bars (north_star): selections bit-exact; BF16-weight outputs within 2e-3
relative (max-abs printed).  Shapes are the BASELINE configs (1.1B: H2048 I5632
k564, predictor 2048->128->5632; 7B: H4096 I11008 k1652, rank 256; heads
4096->128->32 k16) plus small edge cases.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

RTOL = 2e-3


def bf16(orc, a):
    return orc.bf16_from_f32(np.asarray(a, np.float32))


def make_predictor(orc, rng, ind, hid, out, bias=False):
    w1 = bf16(orc, rng.normal(0, 0.02, (hid, ind)))
    w2 = bf16(orc, rng.normal(0, 0.02 if hid > 64 else 0.1, (out, hid)))
    b1 = (rng.normal(0, 0.1, hid) if bias else np.zeros(hid)).astype(np.float32)
    b2 = (rng.normal(0, 0.1, out) if bias else np.zeros(out)).astype(np.float32)
    return w1, b1, w2, b2


@pytest.mark.parametrize("ind,hid,out,batch,bias", [
    (2048, 128, 5632, 1, False),   # cfg2 neuron predictor
    (4096, 256, 11008, 1, False),  # cfg3 neuron predictor
    (4096, 256, 11008, 16, False),  # cfg3 batch 16
    (4096, 128, 32, 8, False),     # cfg4 head predictor
    (100, 13, 77, 3, True),        # ragged shapes, biases
    # the batched layer-1 kernel (BF16, inputs a multiple of 512, more blocks
    # of 8 hidden units x rows than the device's 256 CUs): one round of the
    # ring, two rounds, four; rows and hidden units not multiples of the
    # block's 4 x 8.  Inputs of 128 take the single-row kernel per row.
    (512, 20, 77, 87, True),
    (1024, 13, 40, 130, True),
    (2048, 64, 300, 33, True),
    (128, 20, 77, 5, True),
    # the batched BF16 layer 2 (hidden units a multiple of 8, rows > 1): the
    # cases above with 128, 256 and 64 hidden units take it (outputs short of
    # a 64-block, rows not a multiple of 4); here 3 blocks of 8 inputs.
    (256, 24, 130, 6, True),
])
def test_predictor_scores_bit_exact(kh, orc, ind, hid, out, batch, bias):
    from klearu_amd.dejavu import SparsityPredictor
    rng = np.random.default_rng(ind + hid + out + batch)
    w1, b1, w2, b2 = make_predictor(orc, rng, ind, hid, out, bias)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    x = rng.standard_normal((batch, ind)).astype(np.float32)
    got = p.predict(torch.from_numpy(x).cuda()).cpu().numpy()
    for b in range(batch):
        ref, _ = orc.predictor_predict(w1, b1, w2, b2, x[b])
        np.testing.assert_array_equal(got[b].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("ind,hid,out,k,batch", [
    (2048, 128, 5632, 564, 1), (4096, 256, 11008, 1652, 1), (4096, 256, 11008, 1652, 4),
    (4096, 128, 32, 16, 8), (64, 32, 12, 5, 1), (64, 32, 12, 20, 1)])
def test_select_top_k_bit_exact(kh, orc, ind, hid, out, k, batch):
    from klearu_amd.dejavu import ORDER_ASCENDING, SparsityPredictor
    rng = np.random.default_rng(k + batch)
    w1, b1, w2, b2 = make_predictor(orc, rng, ind, hid, out)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    x = rng.standard_normal((batch, ind)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    got = p.select_top_k(xd, k).cpu().numpy()
    got_asc = p.select_top_k(xd, k, ORDER_ASCENDING).cpu().numpy()
    for b in range(batch):
        s, _ = orc.predictor_predict(w1, b1, w2, b2, x[b])
        ref = orc.select_top_k(s, k)
        np.testing.assert_array_equal(got[b], ref)
        np.testing.assert_array_equal(got_asc[b], np.sort(ref))


@pytest.mark.parametrize("out,k,batch", [(40, 7, 3), (64, 33, 2), (64, 64, 1), (65, 20, 2), (1, 1, 2)])
def test_select_top_k_small_rows_ties(kh, orc, out, k, batch):
    """Rows of up to 64 scores are selected inside layer 2; duplicated and
    zeroed weight rows make exact score ties (zero rows give sigmoid(0)), so
    the index tie-break is exercised.  65 scores take the separate top-k."""
    from klearu_amd.dejavu import ORDER_ASCENDING, SparsityPredictor
    rng = np.random.default_rng(out * 100 + k)
    ind, hid = 96, 24
    w1, b1, w2, b2 = make_predictor(orc, rng, ind, hid, out)
    w2 = orc.bf16_to_f32(w2).copy()
    w2[out // 3:: 4] = 0.0
    if out > 6:
        w2[5] = w2[2]
        w2[out - 1] = w2[2]
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, w2, b2)
    x = rng.standard_normal((batch, ind)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    got = p.select_top_k(xd, k).cpu().numpy()
    got_asc = p.select_top_k(xd, k, ORDER_ASCENDING).cpu().numpy()
    for b in range(batch):
        s, _ = orc.predictor_predict(w1, b1, bf16(orc, w2), b2, x[b])
        ref = orc.select_top_k(s, k)
        assert len(np.unique(s)) < out or out == 1
        np.testing.assert_array_equal(got[b], ref)
        np.testing.assert_array_equal(got_asc[b], np.sort(ref))


@pytest.mark.parametrize("n,k", [(11008, 1652), (5632, 564), (32, 16), (1000, 1000), (1000, 1),
                                 (20000, 3000), (40000, 4000), (65535, 64), (7, 0),
                                 (11264, 4000), (10001, 1500), (8193, 8193), (6143, 900)])
def test_topk_ties_and_edges(kh, orc, n, k):
    """Rows: heavy ties at the threshold (passes down to one key value), five
    distinct values, signed zeros, sigmoid-clustered scores (boundary bin
    ranked directly), uniform scores, and magnitudes from 1e-35 to 1e35 of
    both signs (key intervals as wide as the f32 range)."""
    from klearu_amd.dejavu import ORDER_ASCENDING, topk_select
    rng = np.random.default_rng(n + k)
    s = rng.random((6, n)).astype(np.float32)
    s[5] = (np.exp(rng.uniform(-80, 80, n)) * rng.choice([-1.0, 1.0], n)).astype(np.float32)
    s[0, rng.random(n) < 0.5] = 0.5          # heavy ties at the threshold
    s[1] = np.round(s[1] * 4) / 4            # only five distinct values
    s[2, : n // 2] = -0.0                    # -0.0 ties +0.0
    s[2, n // 2:] = 0.0
    s[3] = (1.0 / (1.0 + np.exp(-rng.normal(0, 0.14, n)))).astype(np.float32)
    got = topk_select(torch.from_numpy(s).cuda(), k).cpu().numpy() if k <= 4096 else None
    asc = topk_select(torch.from_numpy(s).cuda(), k, ORDER_ASCENDING).cpu().numpy()
    for b in range(6):
        ref = orc.select_top_k(s[b], k)
        if got is not None:
            np.testing.assert_array_equal(got[b], ref)
        np.testing.assert_array_equal(asc[b], np.sort(ref))


@pytest.mark.parametrize("n,k,batch", [
    (11008, 1652, 16),   # cfg3 batch 16 (byte marks)
    (11007, 900, 3),     # ragged: n not a multiple of 4, ids up to n - 1
    (5, 5, 2),           # every neuron, tiny row
    (200000, 3000, 4),   # above the byte-mark limit: bitmap path
])
def test_union_active(kh, n, k, batch):
    from klearu_amd.dejavu import union_active
    rng = np.random.default_rng(9 + n)
    ids = np.stack([rng.choice(n, k, replace=False) for _ in range(batch)]).astype(np.int32)
    ids[0, 0] = n - 1  # the last neuron is always marked
    u, c = union_active(torch.from_numpy(ids).cuda(), n)
    cnt = int(c.item())
    np.testing.assert_array_equal(u[:cnt].cpu().numpy(), np.unique(ids))


@pytest.mark.parametrize("ind,hid,out,k,batch", [
    (4096, 256, 11008, 1652, 16),  # the 7B decode batch: union from the top-k marks
    (2048, 128, 5630, 564, 3),     # ragged row (n % 4 != 0)
    (256, 64, 32768, 9000, 2),     # the largest row on the marks path
    (4096, 128, 32, 16, 8),        # rows selected inside layer 2: union from the ids
    (64, 32, 12, 20, 2)])          # k > output: every neuron
def test_select_top_k_union(kh, orc, ind, hid, out, k, batch):
    from klearu_amd.dejavu import SparsityPredictor
    rng = np.random.default_rng(out + batch)
    w1, b1, w2, b2 = make_predictor(orc, rng, ind, hid, out)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    # two calls in a row, the second smaller: the marks must start clear
    for bt in (batch, max(1, batch // 2)):
        x = rng.standard_normal((bt, ind)).astype(np.float32)
        ids, u, c = p.select_top_k_union(torch.from_numpy(x).cuda(), k)
        ids = ids.cpu().numpy()
        ref = []
        for b in range(bt):
            s, _ = orc.predictor_predict(w1, b1, w2, b2, x[b])
            ref.append(np.sort(orc.select_top_k(s, k)))
            np.testing.assert_array_equal(ids[b], ref[-1])
        cnt = int(c.item())
        np.testing.assert_array_equal(u[:cnt].cpu().numpy(), np.unique(np.concatenate(ref)))


def _ffn_case(orc, rng, H, I, k, batch):
    wg = bf16(orc, rng.normal(0, 0.02, (I, H)))
    wu = bf16(orc, rng.normal(0, 0.02, (I, H)))
    wd = bf16(orc, rng.normal(0, 0.02, (H, I)))
    x = rng.standard_normal((batch, H)).astype(np.float32)
    act = rng.choice(I, k, replace=False).astype(np.int64)
    return wg, wu, wd, x, act


@pytest.mark.parametrize("H,I,k,batch", [
    (4096, 11008, 1652, 1),   # cfg3 headline shape
    (2048, 5632, 564, 1),     # cfg2
    (4096, 11008, 1652, 2),
    (4096, 11008, 1652, 16),  # cfg3 batch 16 shared set
    (264, 100, 37, 3),        # ragged hidden (not a multiple of 256)
    (264, 100, 37, 1),        # single token, hidden not a multiple of 64 (general path)
    (1024, 2816, 403, 1),     # single token, partial last block
    (512, 64, 64, 1),         # every neuron active
    (512, 64, 1, 1),          # a single neuron
    (4096, 11008, 5000, 1),   # single token, more active rows than the consumers hold in registers
    (2048, 5632, 5632, 1),    # single token, every neuron active
])
def test_sparse_ffn_matches_oracle(kh, orc, H, I, k, batch):
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(H + I + k + batch)
    wg, wu, wd, x, act = _ffn_case(orc, rng, H, I, k, batch)
    mlp = Mlp(wg, wu, wd, max_batch=16)
    xd = torch.from_numpy(x).cuda()
    ad = torch.from_numpy(act.astype(np.int32)).cuda()
    y = torch.empty_like(xd)
    mlp.forward_sparse_into(xd, ad, y)
    h = mlp.last_hidden(batch, k).cpu().numpy()
    y = y.cpu().numpy()
    for b in range(batch):
        yr, hr = orc.sparse_mlp_forward_bf16(wg, wu, wd, x[b], act)
        scale = float(np.max(np.abs(yr)))
        err = float(np.max(np.abs(y[b] - yr)))
        print(f"H{H} I{I} k{k} b{b}: max-abs {err:.3e} (max |y| {scale:.3e}), "
              f"h max-abs {float(np.max(np.abs(h[b] - hr))):.3e}")
        np.testing.assert_allclose(h[b], hr, rtol=RTOL, atol=1e-6 * float(np.max(np.abs(hr))))
        np.testing.assert_allclose(y[b], yr, rtol=RTOL, atol=1e-4 * scale)


def test_sparse_ffn_accumulate_and_device_count(kh, orc):
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(77)
    H, I, k = 1024, 2816, 400
    wg, wu, wd, x, act = _ffn_case(orc, rng, H, I, k, 2)
    mlp = Mlp(wg, wu, wd, max_batch=4)
    xd = torch.from_numpy(x).cuda()
    full = torch.from_numpy(np.concatenate([act, np.arange(I)[~np.isin(np.arange(I), act)]])
                            .astype(np.int32)).cuda()
    y0 = torch.from_numpy(rng.standard_normal((2, H)).astype(np.float32)).cuda()
    y = y0.clone()
    cnt = torch.tensor([k], dtype=torch.int32, device="cuda")
    mlp.forward_sparse_into(xd, full, y, accumulate=True, n_active_dev=cnt, n_active=I)
    y = y.cpu().numpy()
    for b in range(2):
        yr, _ = orc.sparse_mlp_forward_bf16(wg, wu, wd, x[b], act)
        np.testing.assert_allclose(y[b] - y0[b].cpu().numpy(), yr, rtol=RTOL,
                                   atol=1e-4 * float(np.max(np.abs(yr))))


@pytest.mark.parametrize("cnt_k", [400, 401, 0])
def test_sparse_ffn_batch1_device_count(kh, orc, cnt_k):
    """Batch 1 (the fused kernel) with a device-side count below n_active: the
    blocks past the count contribute nothing, whatever the scratch held."""
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(78 + cnt_k)
    H, I = 1024, 2816
    wg, wu, wd, x, act = _ffn_case(orc, rng, H, I, 400, 1)
    act = np.sort(np.concatenate([act, rng.choice(np.setdiff1d(np.arange(I), act), 1)]))[:max(cnt_k, 1)]
    mlp = Mlp(wg, wu, wd, max_batch=1)
    xd = torch.from_numpy(x).cuda()
    full = torch.from_numpy(np.concatenate([act, np.arange(I)[~np.isin(np.arange(I), act)]])
                            .astype(np.int32)).cuda()
    # fill the scratch partial rows with a full-width call first
    mlp.forward_sparse_into(xd, full, torch.empty_like(xd))
    y0 = torch.from_numpy(rng.standard_normal((1, H)).astype(np.float32)).cuda()
    y = y0.clone()
    cnt = torch.tensor([cnt_k], dtype=torch.int32, device="cuda")
    mlp.forward_sparse_into(xd, full, y, accumulate=True, n_active_dev=cnt, n_active=I)
    yr = orc.sparse_mlp_forward_bf16(wg, wu, wd, x[0], act[:cnt_k])[0] if cnt_k else np.zeros(H, np.float32)
    got = y.cpu().numpy()[0] - y0.cpu().numpy()[0]
    print(f"count {cnt_k}: max-abs {float(np.max(np.abs(got - yr))):.3e}")
    np.testing.assert_allclose(got, yr, rtol=RTOL, atol=1e-4 * max(float(np.max(np.abs(yr))), 1e-3))


def test_sparse_ffn_empty_active_list(kh, orc):
    """No active neurons: the output is zero (written by a fill kernel, so the
    call stays capturable in a HIP graph), or left unchanged when accumulating;
    the same inside a captured graph replayed several times."""
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(3)
    H, I = 256, 512
    wg, wu, wd, _, _ = _ffn_case(orc, rng, H, I, 4, 1)
    mlp = Mlp(wg, wu, wd, max_batch=2)
    x = torch.from_numpy(rng.standard_normal((2, H)).astype(np.float32)).cuda()
    act = torch.zeros(1, dtype=torch.int32, device="cuda")
    y = torch.full((2, H), 7.0, device="cuda")
    mlp.forward_sparse_into(x, act, y, n_active=0)
    assert torch.count_nonzero(y).item() == 0
    y.fill_(3.0)
    mlp.forward_sparse_into(x, act, y, accumulate=True, n_active=0)
    assert torch.all(y == 3.0).item()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        mlp.forward_sparse_into(x, act, y, n_active=0, stream=s)   # sizes nothing; warm
        s.synchronize()
        with torch.cuda.graph(g, stream=s):
            mlp.forward_sparse_into(x, act, y, n_active=0, stream=s)
    for _ in range(3):
        y.fill_(5.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.count_nonzero(y).item() == 0


def test_sparse_ffn_rejects_bad_shapes(kh, orc):
    from klearu_amd import KlearuError
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(1)
    wg, wu, wd, x, act = _ffn_case(orc, rng, 256, 64, 8, 1)
    mlp = Mlp(wg, wu, wd, max_batch=2)
    xd = torch.zeros(3, 256, device="cuda")
    with pytest.raises(KlearuError):
        mlp.forward_sparse_into(xd, torch.zeros(8, dtype=torch.int32, device="cuda"),
                                torch.empty_like(xd))


def _rms_rows(rng):
    """Rows for the RmsNorm parity test, with the cases that stress the exact
    parallel sum of squares: every chunk's speculative window missing (a
    running sum stuck at 2^24 while the exact sum grows: each square 1.0 is a
    tie that rounds back down), squares just above half an ulp (each rounds
    up), zeros, tiny and huge magnitudes, a partial last chunk."""
    rows = {}
    rows["normal 4096"] = rng.standard_normal(4096)
    rows["normal 2048"] = rng.standard_normal(2048)
    rows["normal 8192"] = rng.standard_normal(8192)
    rows["ragged 1000"] = rng.standard_normal(1000)
    rows["ragged 130"] = rng.standard_normal(130)
    rows["single"] = np.array([3.0])
    stuck = np.ones(4096)
    stuck[0] = 4096.0  # 4096^2 = 2^24, then + 1.0 ties back to 2^24 every step
    rows["ties stuck at 2^24"] = stuck
    up = np.full(4096, np.sqrt(1.0000001))
    up[0] = 4096.0
    rows["round-up drift"] = up
    z = rng.standard_normal(4096)
    z[:700] = 0.0
    rows["leading zeros"] = z
    rows["all zero"] = np.zeros(4096)
    rows["tiny"] = rng.standard_normal(4096) * 1e-20
    rows["huge"] = rng.standard_normal(4096) * 1e17
    rows["wide range"] = rng.standard_normal(4096) * np.exp(rng.uniform(-20, 20, 4096))
    rows["long 12288"] = rng.standard_normal(12288)   # past the parallel kernel's limit
    return {k: v.astype(np.float32) for k, v in rows.items()}


def test_rmsnorm_bit_exact(kh, orc):
    """kh_rmsnorm against the oracle's RmsNorm::forward (rms_norm.rs:43-64):
    bit-identical, including rows that force the sequential fallback of every
    chunk, and a batch of 16 rows (the batched decode path's norm)."""
    from klearu_amd.dejavu import rmsnorm
    rng = np.random.default_rng(3)
    for name, x in _rms_rows(rng).items():
        w = rng.uniform(0.5, 1.5, x.size).astype(np.float32)
        got = rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), 1e-5).cpu().numpy()
        want = orc.rmsnorm(x, w, 1e-5)
        print(f"{name}: {int(np.sum(got.view(np.uint32) != want.view(np.uint32)))} differing words")
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32), err_msg=name)
    xb = rng.standard_normal((16, 4096)).astype(np.float32) * rng.uniform(0.1, 10, (16, 1)).astype(np.float32)
    w = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    got = rmsnorm(torch.from_numpy(xb).cuda(), torch.from_numpy(w).cuda(), 1e-6).cpu().numpy()
    for b in range(16):
        np.testing.assert_array_equal(got[b].view(np.uint32), orc.rmsnorm(xb[b], w, 1e-6).view(np.uint32))


@pytest.mark.parametrize("H,I,R,k,layers", [
    (4096, 11008, 256, 1652, 4),   # cfg3 (7B): hidden 4096, 11008 neurons, rank 256, top 15%
    (2048, 5632, 128, 564, 3),     # cfg2 (1.1B): top 10%
    (2048, 5632, 128, 563, 2),     # cfg2, ragged: the last 8-neuron block takes 3
])
def test_mlp_block_chained_exact(kh, orc, H, I, R, k, layers):
    """kh_dejavu_mlp_block chained over several layers against the oracle's
    RmsNorm -> predictor -> select_top_k -> forward_sparse -> residual
    (crates/klearu-llm/src/sparse/mod.rs:115-142).  For each layer, the
    oracle runs on the hidden row the GPU held before the block: the active
    set must equal the oracle's own top-k exactly (no boundary swaps), and the
    updated row must match the oracle's residual, computed from the oracle's
    selection, within the BF16-weight tolerance."""
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block
    rng = np.random.default_rng(31 + H)
    wg, wu, wd, _, _ = _ffn_case(orc, rng, H, I, k, 1)
    mlp = Mlp(wg, wu, wd, max_batch=1)
    hidden = rng.standard_normal(H).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    hd = torch.from_numpy(hidden.copy()).cuda()
    wnd = torch.from_numpy(wn).cuda()
    ws = torch.empty(1, dtype=torch.float32, device="cuda")
    for layer in range(layers):
        w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
        p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
        h_in = hd.cpu().numpy().copy()
        act = mlp_block(p, mlp, hd, wnd, 1e-5, k, norm_ws=ws)
        _check_block(orc, f"layer {layer}", h_in, wn, ws, act, hd, (w1, b1, w2, b2), k, (wg, wu, wd))


def _check_block(orc, what, h_in, wn, ws, act, hd, pred, k, ffn):
    """One kh_dejavu_mlp_block call against the oracle: the RmsNorm scale the
    block wrote (norm_ws) bit-equal to rms_norm.rs:48-52's, the active set
    equal to the oracle's own top-k (no boundary swaps), and the updated row
    within the BF16-weight tolerance of the oracle's residual."""
    inv = orc.rms_inv(h_in, 1e-5)
    got_inv = ws.cpu().numpy()[:1]
    print(f"{what}: norm scale {float(got_inv[0])!r} (oracle {float(inv)!r})")
    np.testing.assert_array_equal(got_inv.view(np.uint32), np.array([inv], np.float32).view(np.uint32),
                                  err_msg=f"{what}: norm scale")
    norm = orc.rmsnorm(h_in, wn, 1e-5)
    scores, _ = orc.predictor_predict(*pred, norm)
    sel = np.sort(orc.select_top_k(scores, k))
    got = act.cpu().numpy()
    print(f"{what}: {np.setxor1d(got, sel).size} ids differ")
    np.testing.assert_array_equal(got, sel, err_msg=what)
    y, _ = orc.sparse_mlp_forward_bf16(*ffn, norm, sel.astype(np.int64))
    want = h_in + y
    out = hd.cpu().numpy()
    scale = float(np.max(np.abs(want)))
    print(f"{what}: max-abs {float(np.max(np.abs(out - want))):.3e} (max |hidden| {scale:.3e})")
    np.testing.assert_allclose(out, want, rtol=RTOL, atol=1e-4 * scale, err_msg=what)


@pytest.mark.parametrize("H,I,R,k", [
    (4096, 11008, 256, 1652),   # cfg3 (7B)
    (2048, 5632, 128, 564),     # cfg2 (1.1B)
])
def test_mlp_block_hard_norm_rows(kh, orc, H, I, R, k):
    """kh_dejavu_mlp_block fed hidden rows whose sum of squares defeats the
    exact sum's speculative windows (ties stuck at 2^24, round-up drift),
    leading zeros, an all-zero row, tiny, huge and wide-range magnitudes: the
    fused predictor kernel's own exact-sum instance must take its sequential
    fallback and still write the reference's RmsNorm scale bit for bit, and
    the selection must stay the oracle's (rms_norm.rs:43-53,
    sparse/mod.rs:115-125)."""
    from hard_rows import hard_hidden_rows
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block
    rng = np.random.default_rng(57 + H)
    wg, wu, wd, _, _ = _ffn_case(orc, rng, H, I, k, 1)
    mlp = Mlp(wg, wu, wd, max_batch=1)
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    wnd = torch.from_numpy(wn).cuda()
    ws = torch.full((1,), float("nan"), dtype=torch.float32, device="cuda")
    for name, row in hard_hidden_rows(rng, H).items():
        hd = torch.from_numpy(row.copy()).cuda()
        ws.fill_(float("nan"))
        act = mlp_block(p, mlp, hd, wnd, 1e-5, k, norm_ws=ws)
        _check_block(orc, name, row, wn, ws, act, hd, (w1, b1, w2, b2), k, (wg, wu, wd))


@pytest.mark.parametrize("case,k", [
    ("tie group", 1652),   # 5000 identical predictor rows: the k-th score is one of 5000 equal keys
    ("saturated", 1652),   # scores pinned at 1.0 for about a third of the neurons
    ("all", 11008),        # every neuron
    ("one", 1),
    ("ragged", 1651),      # the last block takes fewer than 8 neurons
])
def test_mlp_block_selection_edges(kh, orc, case, k):
    """The fused block's FFN kernel selects its own neurons from layer 2's
    scores when its blocks have 8 waves (every block runs the same exact
    selection): ties broken by the lower index when the k-th score sits in a
    group of equal keys larger than the directly ranked bin, saturated sigmoid
    scores, k equal to the whole layer, k = 1 and a partial last block, against
    the oracle's select_top_k (mlp_predictor.rs:128-135)."""
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block
    H, I, R = 2560, 11008, 128
    rng = np.random.default_rng(91)
    wg, wu, wd, _, _ = _ffn_case(orc, rng, H, I, 1, 1)
    mlp = Mlp(wg, wu, wd, max_batch=1)
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    row = rng.standard_normal(H).astype(np.float32)
    if case == "tie group":
        # copy into rows 0..4999 the row of neurons 5000.. that about 1000 of
        # them outscore, so the copies fill ranks ~1000..6000 around k
        s0, _ = orc.predictor_predict(w1, b1, w2, b2, orc.rmsnorm(row, wn, 1e-5))
        r = 5000 + int(np.argsort(-s0[5000:], kind="stable")[1000])
        w2[:5000] = w2[r]
        b2[:5000] = b2[r]
    elif case == "saturated":
        w2 = bf16(orc, orc.bf16_to_f32(w2) * 250.0)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    hd = torch.from_numpy(row.copy()).cuda()
    ws = torch.empty(1, dtype=torch.float32, device="cuda")
    act = mlp_block(p, mlp, hd, torch.from_numpy(wn).cuda(), 1e-5, k, norm_ws=ws)
    if case in ("tie group", "saturated"):
        scores, _ = orc.predictor_predict(w1, b1, w2, b2, orc.rmsnorm(row, wn, 1e-5))
        kth = np.sort(scores)[::-1][k - 1]
        ties = int(np.sum(scores == kth))
        print(f"{case}: {ties} scores equal the k-th ({float(kth)!r})")
        assert ties > 256
    _check_block(orc, case, row, wn, ws, act, hd, (w1, b1, w2, b2), k, (wg, wu, wd))


def test_batched_norm_select_union_exact(kh, orc):
    """The batch-16 decode path: kh_rmsnorm over 16 rows, then the predictor's
    top-k of every row and their union, against the oracle per row (exact)."""
    from klearu_amd.dejavu import SparsityPredictor, rmsnorm
    rng = np.random.default_rng(77)
    H, R, I, k, B = 4096, 256, 11008, 1652, 16
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    x = rng.standard_normal((B, H)).astype(np.float32)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    nd = rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(wn).cuda(), 1e-5)
    ids, uni, cnt = p.select_top_k_union(nd, k)
    uni = uni[:int(cnt.item())]
    want_u = set()
    for b in range(B):
        norm = orc.rmsnorm(x[b], wn, 1e-5)
        scores, _ = orc.predictor_predict(w1, b1, w2, b2, norm)
        sel = np.sort(orc.select_top_k(scores, k))
        np.testing.assert_array_equal(ids[b].cpu().numpy(), sel)
        want_u |= set(sel.tolist())
    np.testing.assert_array_equal(uni.cpu().numpy(), np.array(sorted(want_u), np.int32))


@pytest.mark.parametrize("H,R,I,k,B", [
    (4096, 256, 11008, 1652, 16),  # cfg3 batch 16: union from the marks inside the gate/up kernel
    (512, 64, 1000, 150, 3),       # small, the same path
    (384, 32, 700, 90, 5),         # hidden not a multiple of 512: the union kernel, then the FFN
])
def test_mlp_block_batch_matches_unfused(kh, orc, H, R, I, k, B):
    """kh_dejavu_mlp_block_batch over three chained calls: every row's RmsNorm
    scale and top-k ids equal the oracle's (rms_norm.rs:43-53,
    mlp_predictor.rs:127-132), and the updated rows equal, bit for bit, what
    kh_rmsnorm + kh_predictor_select_top_k_union + kh_sparse_ffn_forward
    produce from the same rows (the same FFN over the same union); the second
    and third calls show the union marks were cleared in between."""
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block_batch, rmsnorm
    rng = np.random.default_rng(H + I + B)
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    wg, wu, wd, x, _ = _ffn_case(orc, rng, H, I, 1, B)
    mlp = Mlp(wg, wu, wd, max_batch=B)
    wn = rng.uniform(0.5, 1.5, H).astype(np.float32)
    wnd = torch.from_numpy(wn).cuda()
    hd = torch.from_numpy(x.copy()).cuda()
    ws = torch.empty(B, dtype=torch.float32, device="cuda")
    for call in range(3):
        h_in = hd.clone()
        ws.fill_(float("nan"))
        act = mlp_block_batch(p, mlp, hd, wnd, 1e-5, k, norm_ws=ws).cpu().numpy()
        # the unfused sequence on the same input rows
        nd = rmsnorm(h_in, wnd, 1e-5)
        ids, uni, cnt = p.select_top_k_union(nd, k)
        want = h_in.clone()
        mlp.forward_sparse_into(nd, uni, want, n_active_dev=cnt, accumulate=True)
        np.testing.assert_array_equal(hd.cpu().numpy(), want.cpu().numpy(), err_msg=f"call {call}: rows")
        hn = h_in.cpu().numpy()
        scales = ws.cpu().numpy()
        for b in range(B):
            inv = np.array([orc.rms_inv(hn[b], 1e-5)], np.float32)
            np.testing.assert_array_equal(scales[b:b + 1].view(np.uint32), inv.view(np.uint32),
                                          err_msg=f"call {call} row {b}: norm scale")
            norm = orc.rmsnorm(hn[b], wn, 1e-5)
            scores, _ = orc.predictor_predict(w1, b1, w2, b2, norm)
            np.testing.assert_array_equal(act[b], np.sort(orc.select_top_k(scores, k)),
                                          err_msg=f"call {call} row {b}: ids")


def test_sparse_ffn_out_of_range_ids_are_reported(kh, orc):
    """An active id outside [0, intermediate) (the reference panics in
    get_weights, crates/klearu-accel/src/memory/mod.rs:87-92) reads no memory
    outside the weights and is reported by the handle's status call, once."""
    from klearu_amd import KlearuError
    from klearu_amd._lib import KH_ERR_ARG
    from klearu_amd.dejavu import Mlp
    rng = np.random.default_rng(4)
    H, I = 512, 300
    wg, wu, wd, x, _ = _ffn_case(orc, rng, H, I, 8, 2)
    for batch in (1, 2):
        mlp = Mlp(wg, wu, wd, max_batch=2)
        mlp.status()
        xd = torch.from_numpy(x[:batch].copy()).cuda()
        for bad in (I, -1, 1 << 30):
            act = torch.tensor([3, bad, 7], dtype=torch.int32, device="cuda")
            y = torch.zeros(batch, H, device="cuda")
            mlp.forward_sparse_into(xd, act, y)
            with pytest.raises(KlearuError) as e:
                mlp.status()
            assert e.value.code == KH_ERR_ARG
            mlp.status()   # the record was cleared
        good = torch.tensor([3, 7], dtype=torch.int32, device="cuda")
        mlp.forward_sparse_into(xd, good, torch.zeros(batch, H, device="cuda"))
        mlp.status()


def test_batched_predictor_wait_give_up_is_reported(kh, orc):
    """The batched layer-1 kernel (7B shape, batch 16) bounds every wait for
    its LDS hand-offs.  With the spin limit forced down to one sleep from the
    host, the consumer gives up waiting for the producers' first stage: the
    kernel still exits, and kh_predictor_status reports the call.  With the
    default limit restored the scores are bit-exact again and the status is
    clean."""
    from klearu_amd import KlearuError
    from klearu_amd._lib import KH_ERR_HIP
    from klearu_amd.dejavu import SparsityPredictor
    rng = np.random.default_rng(12)
    H, R, I, B = 4096, 256, 11008, 16
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    x = rng.standard_normal((B, H)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    p.status()
    p.set_spin_limit(1)
    p.predict(xd)
    with pytest.raises(KlearuError) as e:
        p.status()
    assert e.value.code == KH_ERR_HIP
    p.status()   # the record was cleared
    p.set_spin_limit(1 << 22)
    got = p.predict(xd).cpu().numpy()
    p.status()
    for b in (0, 7, 15):
        want, _ = orc.predictor_predict(w1, b1, w2, b2, x[b])
        np.testing.assert_array_equal(got[b].view(np.uint32), want.view(np.uint32))


def test_predictor_concurrent_streams(kh, orc):
    """SparsityPredictor::select_top_k takes &self: two host threads on their
    own streams select on one predictor at the same time; every selection is
    the oracle's."""
    import threading
    from klearu_amd.dejavu import ORDER_ASCENDING, ORDER_SCORE, SparsityPredictor
    rng = np.random.default_rng(12)
    H, R, I, k = 4096, 256, 11008, 1652
    w1, b1, w2, b2 = make_predictor(orc, rng, H, R, I, bias=True)
    p = SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2)
    xs = [rng.standard_normal((2, H)).astype(np.float32) for _ in range(2)]
    want = []
    for x in xs:
        rows = []
        for b in range(2):
            s, _ = orc.predictor_predict(w1, b1, w2, b2, x[b])
            rows.append(orc.select_top_k(s, k))
        want.append(rows)
    errors = []

    def worker(t):
        try:
            s = torch.cuda.Stream()
            xd = torch.from_numpy(xs[t]).cuda()
            order = ORDER_SCORE if t == 0 else ORDER_ASCENDING
            for _ in range(10):
                with torch.cuda.stream(s):
                    ids = p.select_top_k(xd, k, order, stream=s)
                s.synchronize()
                got = ids.cpu().numpy()
                for b in range(2):
                    w = want[t][b] if order == ORDER_SCORE else np.sort(want[t][b])
                    if not np.array_equal(got[b], w):
                        errors.append((t, b))
                        return
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append((t, repr(e)))

    th = [threading.Thread(target=worker, args=(t,)) for t in range(2)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert not errors, errors


@pytest.mark.parametrize("B", [1, 16])
def test_mlp_block_graph_replays_match_eager_7b(kh, orc, B):
    """The headline step at cfg3's shape (hidden 4096, intermediate 11008, top
    1652; batch 1 and 16): kh_dejavu_mlp_block[_batch] captured in a HIP graph
    as bench.py times it, replayed several times with eager calls of a twin
    (the same weights, its own handles) on the same stream between the replays.
    After every replay the rows, neuron sets and RmsNorm scales equal the eager
    call's bit for bit."""
    from klearu_amd.dejavu import Mlp, SparsityPredictor, mlp_block, mlp_block_batch
    H, I, R, k, calls = 4096, 11008, 256, 1652, 4
    rng = np.random.default_rng(11 + B)
    bf = lambda a: orc.bf16_from_f32(np.asarray(a, np.float32))  # noqa: E731
    w1, w2 = bf(rng.normal(0, 0.02, (R, H))), bf(rng.normal(0, 0.02, (I, R)))
    b1, b2 = rng.normal(0, 0.1, R).astype(np.float32), rng.normal(0, 0.1, I).astype(np.float32)
    wg, wu, wd = bf(rng.normal(0, 0.02, (I, H))), bf(rng.normal(0, 0.02, (I, H))), bf(rng.normal(0, 0.02, (H, I)))
    wn = torch.from_numpy(rng.uniform(0.5, 1.5, H).astype(np.float32)).cuda()
    x0 = torch.from_numpy(rng.standard_normal((B, H)).astype(np.float32)).cuda()

    def twin():
        return dict(p=SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2),
                    mlp=Mlp(wg, wu, wd, max_batch=B), h=x0.clone(),
                    act=torch.full((B, k), -1, dtype=torch.int32, device="cuda"),
                    ws=torch.zeros(B, device="cuda"))

    def call(t, s):
        if B == 1:
            mlp_block(t["p"], t["mlp"], t["h"][0], wn, 1e-5, k, active=t["act"][0], norm_ws=t["ws"], stream=s)
        else:
            mlp_block_batch(t["p"], t["mlp"], t["h"], wn, 1e-5, k, active=t["act"], norm_ws=t["ws"], stream=s)

    def same(te, tg, what):
        for key in ("h", "ws"):
            np.testing.assert_array_equal(tg[key].cpu().numpy().view(np.uint32), te[key].cpu().numpy().view(np.uint32),
                                          err_msg=f"{what}: {key}")
        np.testing.assert_array_equal(tg["act"].cpu().numpy(), te["act"].cpu().numpy(), err_msg=f"{what}: ids")

    te, tg = twin(), twin()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        call(te, s)  # the warm-up call sizes the scratch buffers the capture records
        call(tg, s)
        s.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            call(tg, s)
    torch.cuda.synchronize()
    same(te, tg, "warm-up call")
    for i in range(calls):
        with torch.cuda.stream(s):
            call(te, s)
            s.synchronize()
            g.replay()
        torch.cuda.synchronize()
        print(f"B={B} replay {i}: first ids {tg['act'][0, :4].tolist()}", flush=True)
        same(te, tg, f"replay {i}")
