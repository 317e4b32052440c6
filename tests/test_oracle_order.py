"""Pins the oracle's summation order with cancellation known answers (CPU).

Every sum on the reference's path is a left-to-right f32 fold: the predictor's
two layers (`.map(|(w, x)| w * x).sum()`, mlp_predictor.rs:106-121), the SLIDE
neuron (neuron.rs:55-61), the SimHash plane dot (simhash.rs:75-86), the sparse
FFN's down projection (`sum += w[neuron] * gate_sparse[idx]` in active-list
order, sparse_mlp.rs:27-34) and RmsNorm's sum of squares (rms_norm.rs:48-51).

The known answers use terms whose exact sum differs from every reordering's:
  2^24 followed by m ones: each `+ 1.0` is a tie between 2^24 and 2^24 + 2 and
  rounds back to 2^24 (ties to even), so the left-to-right sum stays 2^24,
  while any order that adds ones together first (reverse, pairwise, blocked,
  compensated) reaches 2^24 + m;
  2^25 followed by m minus-ones and -2^25: each `- 1.0` also ties back to 2^25,
  so the fold ends at exactly 0 (sign bit set), the exact sum is -m.
A plausible mistake -- a reversed or pairwise order, a wider accumulator, a
fused multiply-add that skips the product's rounding -- changes these results.
Iterator::sum over f32 folds from -0.0 (Rust >= 1.82; the reference's Cargo.lock
is version 4, written by Cargo >= 1.83), visible only when every term is -0.0.
"""
import numpy as np

P24, P25, M = float(2 ** 24), float(2 ** 25), 64


def absorbing_terms():
    """[2^24, 1 x M, -2^24]: left to right 0, exactly M."""
    return np.array([P24] + [1.0] * M + [-P24], np.float32)


def test_neuron_forward_sums_left_to_right(orc):
    w = absorbing_terms()
    x = np.ones_like(w)
    assert orc.neuron_forward(w, 0.5, x) == np.float32(0.5)            # (0 + 0.5); exact: M + 0.5
    idx = np.arange(w.size, dtype=np.uint32)
    assert orc.neuron_forward_sparse(w, 0.5, idx, x) == np.float32(0.5)
    # the fold starts at -0.0: a product of -0.0 plus a -0.0 bias stays -0.0
    z = orc.neuron_forward(np.array([-1.0], np.float32), -0.0, np.array([0.0], np.float32))
    assert np.float32(z).view(np.uint32) == np.uint32(0x80000000)


def test_neuron_forward_products_are_rounded(orc):
    """w * x is rounded before the add (no FMA): (1 + 2^-12)^2 rounds to
    1 + 2^-11, so with -(1 + 2^-11) after it the sum is 0 (an FMA keeps 2^-24)."""
    a = np.float32(1 + 2.0 ** -12)
    w = np.array([a, -(1 + 2.0 ** -11)], np.float32)
    x = np.array([a, 1.0], np.float32)
    assert orc.neuron_forward(w, 0.0, x) == np.float32(0.0)


def test_predictor_layers_sum_left_to_right(orc):
    """Layer 1 (n_in = M + 2): w1 rows are the absorbing terms, x all ones, so
    h = max(0 + b1, 0).  Layer 2 is pinned with n_in = 1 and w1 = v, which makes
    the hidden vector v itself: the logit is the left-to-right sum of v."""
    v = absorbing_terms()
    n = v.size
    w1 = np.tile(v, (3, 1))
    b1 = np.array([0.25, -1.0, 3.0], np.float32)
    w2 = np.ones((2, 3), np.float32)
    b2 = np.zeros(2, np.float32)
    _, h = orc.predictor_predict(w1, b1, w2, b2, np.ones(n, np.float32))
    np.testing.assert_array_equal(h, np.array([0.25, 0.0, 3.0], np.float32))   # exactly M + b1 otherwise
    w1b = v.reshape(n, 1)
    w2b = np.ones((1, n), np.float32)
    s, h = orc.predictor_predict(w1b, np.zeros(n, np.float32), w2b, np.zeros(1, np.float32),
                                 np.ones(1, np.float32))
    np.testing.assert_array_equal(h, np.maximum(v, 0))
    # h = [2^24, 1 x M, 0]: left to right the logit is 2^24, so sigmoid = 1 ...
    assert s[0] == np.float32(1.0)
    # ... and with -2^24 appended through a second unit the logit is 0: sigmoid(0) = 0.5
    w1c = np.concatenate([v.reshape(n, 1), np.full((1, 1), 1.0, np.float32)])
    w2c = np.concatenate([np.ones((1, n), np.float32), np.full((1, 1), -P24, np.float32)], axis=1)
    s, _ = orc.predictor_predict(w1c, np.zeros(n + 1, np.float32), w2c, np.zeros(1, np.float32),
                                 np.ones(1, np.float32))
    assert s[0] == np.float32(0.5)                                   # exactly: sigmoid(M) != 0.5


def test_simhash_plane_dot_sums_left_to_right(orc):
    """A plane of all +1 over x = [2^25, -1 x M, -2^25]: left to right the sum
    is +0 (bit set, s >= 0), exactly -M (bit clear).  Appending one more -1
    makes it -1 (bit clear), while a reversed fold would give 0 (bit set)."""
    x1 = np.array([P25] + [-1.0] * M + [-P25], np.float32)
    x2 = np.append(x1, np.float32(-1.0))
    for x, bit in ((x1, 1), (x2, 0)):
        planes = np.ones((1, 1, x.size), np.int8)
        assert orc.hash_dense(planes, x, 0) == bit
        idx = np.arange(x.size, dtype=np.uint32)
        assert orc.hash_sparse(planes, idx, x, 0) == bit
    # a -1 plane entry subtracts (sum -= x): the mirror image gives the same bits
    planes = -np.ones((1, 1, x1.size), np.int8)
    assert orc.hash_dense(planes, -x1, 0) == 1


def test_sparse_mlp_down_sums_in_active_order(orc):
    """The down projection adds w[neuron] * h in active-list order.  Gate rows
    give g = 32 (silu(32) = 32 exactly: exp(-32) vanishes against 1) and up
    rows u = v / 32, so h = v: [2^24, 1 x M, -2^24] in list order.  With the
    down weights 1 the output is 0 left to right (M exactly), and the reversed
    list gives 0 as well while a list with -2^24 first gives M."""
    v = absorbing_terms()
    n = v.size
    H = 2
    wg = np.zeros((n, H), np.float32)
    wg[:, 0] = 32.0
    wu = np.zeros((n, H), np.float32)
    wu[:, 0] = v / 32.0
    wd = np.ones((H, n), np.float32)
    bf = orc.bf16_from_f32
    x = np.array([1.0, 0.0], np.float32)
    act = np.arange(n, dtype=np.int64)
    y, h = orc.sparse_mlp_forward_bf16(bf(wg), bf(wu), bf(wd), x, act)
    np.testing.assert_array_equal(h, v)
    np.testing.assert_array_equal(y, np.zeros(H, np.float32))
    # order matters: -2^24 first, then 2^24, then the ones -> M
    act2 = np.concatenate([[n - 1, 0], np.arange(1, n - 1)]).astype(np.int64)
    y2, _ = orc.sparse_mlp_forward_bf16(bf(wg), bf(wu), bf(wd), x, act2)
    np.testing.assert_array_equal(y2, np.full(H, float(M), np.float32))


def test_rmsnorm_sum_of_squares_left_to_right(orc):
    """x = [4096, 1 x M]: the squares are [2^24, 1 x M]; left to right the sum
    stays 2^24 (each + 1.0 ties back), exactly 2^24 + M.  The outputs are those
    of the scale from 2^24 and differ from those of the exact sum."""
    x = np.array([4096.0] + [1.0] * M, np.float32)
    w = np.ones_like(x)
    n = np.float32(x.size)
    eps = np.float32(1e-5)
    got = orc.rmsnorm(x, w, 1e-5)

    def with_sum(ss):
        inv = np.float32(1.0) / np.sqrt(np.float32(ss) / n + eps)
        return (x * inv) * w

    np.testing.assert_array_equal(got, with_sum(P24))
    assert not np.array_equal(got, with_sum(P24 + M))
