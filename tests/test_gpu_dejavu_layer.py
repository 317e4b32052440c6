"""GPU parity: the klearu-dejavu transformer layer (f32 Linear with bias,
SparseMlp, SparseAttention) vs the oracle.

Bar: bit-exact.  Every output of the reference is a sequential f32 sum of
rounded products (transformer/mod.rs:114-134, mlp.rs:23-58, attention.rs:18-74)
and the kernels replay it in the same order.  Shapes: the reference tests'
configuration (hidden 64, intermediate 128, 4 heads x 16) and larger ragged
ones; edge cases: repeated and empty selections, out-of-range indices.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def xavier(rng, out_f, in_f):
    return rng.normal(0, np.sqrt(2.0 / (in_f + out_f)), (out_f, in_f)).astype(np.float32)


@pytest.mark.parametrize("in_f,out_f,batch", [(64, 128, 1), (128, 64, 3), (517, 1031, 2)])
def test_linear_bit_exact(kh, orc, in_f, out_f, batch):
    from klearu_amd.dejavu_transformer import Linear
    rng = np.random.default_rng(in_f + out_f)
    w, b = xavier(rng, out_f, in_f), rng.normal(0, 0.1, out_f).astype(np.float32)
    x = rng.standard_normal((batch, in_f)).astype(np.float32)
    lin = Linear(w, b)
    y = lin.forward(torch.from_numpy(x).cuda()).cpu().numpy()
    idx = np.concatenate([rng.choice(out_f, 20, replace=False), [3, 3, out_f - 1]])
    ys = lin.forward_sparse(torch.from_numpy(x).cuda(), idx).cpu().numpy()
    for r in range(batch):
        np.testing.assert_array_equal(bits(y[r]), bits(orc.dejavu_linear_forward(w, b, x[r])))
        np.testing.assert_array_equal(bits(ys[r]), bits(orc.dejavu_linear_forward_sparse(w, b, x[r], idx)))


def test_linear_rejects_out_of_range(kh):
    from klearu_amd import KlearuError
    from klearu_amd.dejavu_transformer import Linear
    lin = Linear(np.ones((4, 3), np.float32))
    with pytest.raises(KlearuError):
        lin.forward_sparse(np.ones(3, np.float32), [1, 4])
    with pytest.raises(KlearuError):
        lin.forward_sparse(np.ones(3, np.float32), [-1])


@pytest.mark.parametrize("H,I,batch", [(64, 128, 1), (512, 1376, 2)])
def test_sparse_mlp_bit_exact(kh, orc, H, I, batch):
    from klearu_amd.dejavu_transformer import Linear, SparseMlp
    rng = np.random.default_rng(H + I)
    wg, wu, wd = xavier(rng, I, H), xavier(rng, I, H), xavier(rng, H, I)
    bg, bu, bd = (rng.normal(0, 0.05, n).astype(np.float32) for n in (I, I, H))
    gate, up, down = Linear(wg, bg), Linear(wu, bu), Linear(wd, bd)
    mlp = SparseMlp(H, I)
    x = rng.standard_normal((batch, H)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    sels = [rng.choice(I, I // 10, replace=False),          # unsorted selection
            np.array([5, 9, 5, 0, I - 1]),                  # repeated neuron
            np.array([], np.int64),                         # nothing selected: bias only
            np.arange(I)]                                   # every neuron
    for sel in sels:
        y = mlp.forward(xd, gate, up, down, sel).cpu().numpy()
        for r in range(batch):
            ref = orc.dejavu_sparse_mlp_forward(wg, bg, wu, bu, wd, bd, x[r], sel)
            np.testing.assert_array_equal(bits(y[r]), bits(ref))


@pytest.mark.parametrize("H,nh,hd,batch", [(64, 4, 16, 1), (512, 8, 64, 3)])
def test_sparse_attention_bit_exact(kh, orc, H, nh, hd, batch):
    from klearu_amd.dejavu_transformer import Linear, SparseAttention
    rng = np.random.default_rng(H + nh)
    ws = [xavier(rng, nh * hd, H) for _ in range(3)] + [xavier(rng, H, nh * hd)]
    bs = [rng.normal(0, 0.05, nh * hd).astype(np.float32) for _ in range(3)] + \
        [rng.normal(0, 0.05, H).astype(np.float32)]
    q, k, v, o = (Linear(w, b) for w, b in zip(ws, bs))
    sa = SparseAttention(H, nh, hd)
    x = (rng.standard_normal((batch, H)) * 0.5).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    args = [a for pair in zip(ws, bs) for a in pair]
    for heads in ([0, 2], list(range(nh)), [], [nh - 1, 1, nh - 1]):
        y = sa.forward(xd, q, k, v, o, heads).cpu().numpy()
        for r in range(batch):
            ref = orc.dejavu_sparse_attention_forward(*args, nh, hd, x[r], heads)
            np.testing.assert_array_equal(bits(y[r]), bits(ref))


def test_sparse_attention_rejects_bad_heads(kh):
    from klearu_amd import KlearuError
    from klearu_amd.dejavu_transformer import Linear, SparseAttention
    w = np.ones((32, 32), np.float32)
    q = Linear(w)
    sa = SparseAttention(32, 2, 16)
    with pytest.raises(KlearuError):
        sa.forward(np.ones(32, np.float32), q, q, q, q, [2])
