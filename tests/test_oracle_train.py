"""Pins for the oracle's SLIDE training restatement (CPU only).

Each check is one the reference's own tests state (known values), a closed
form the mathematics fixes, or a cancellation case that only the reference's
left-to-right f32 order reproduces, so that a dropped term, a swapped operand
or a reordered sum fails here.
"""
import math

import numpy as np
import pytest

import oracle as orc

F = np.float32


# ----------------------------------------------------------------- f32::powi
@pytest.mark.parametrize("b", [0.9, 0.999, 0.5, 1.7])
def test_powi_closed_forms(b):
    b = F(b)
    assert orc.powi_f32(b, 0) == 1.0
    assert orc.powi_f32(b, 1) == b
    assert orc.powi_f32(b, 2) == F(b * b)
    assert orc.powi_f32(b, 3) == F(b * F(b * b))        # low bit first: mul = b, then b*(b*b)
    assert orc.powi_f32(b, 4) == F(F(b * b) * F(b * b))
    assert orc.powi_f32(b, -2) == F(F(1.0) / F(b * b))
    # large exponents stay within f32 rounding of the exact power
    assert orc.powi_f32(b, 100) == pytest.approx(float(b) ** 100, rel=1e-5)


# ----------------------------------------------------------------- Sgd (sgd.rs tests)
def test_sgd_reference_values():
    w = np.array([1.0, 2.0, 3.0], F)
    b, _ = orc.sgd_update(w, [0.1, 0.2, 0.3], 0.5, 0.05, 0.01, momentum=0.0)
    np.testing.assert_allclose(w, [1.0 - 0.01 * 0.1, 2.0 - 0.01 * 0.2, 3.0 - 0.01 * 0.3], atol=1e-6)
    assert abs(b - (0.5 - 0.01 * 0.05)) < 1e-6
    # momentum 0.9 (sgd.rs:96-117): 0.9, 1.9, bias 0.4; then 0.71, 1.71, 0.21
    w = np.array([1.0, 2.0], F)
    mw = np.zeros(2, F)
    b, mb = orc.sgd_update(w, [1.0, 1.0], 0.5, 1.0, 0.1, momentum=0.9, mw=mw, mb=0.0)
    np.testing.assert_allclose(w, [0.9, 1.9], atol=1e-6)
    assert abs(b - 0.4) < 1e-6
    b, mb = orc.sgd_update(w, [1.0, 1.0], b, 1.0, 0.1, momentum=0.9, mw=mw, mb=mb)
    np.testing.assert_allclose(w, [0.9 - 0.19, 1.9 - 0.19], atol=1e-6)
    assert abs(b - (0.4 - 0.19)) < 1e-6


def test_sgd_exact_binary_fractions():
    # lr and gradients that are exact in f32: every result is exact
    w = np.array([1.0, -2.0], F)
    mw = np.array([0.5, -0.25], F)
    b, mb = orc.sgd_update(w, [2.0, 4.0], 0.0, 8.0, 0.5, momentum=0.5, mw=mw, mb=1.0)
    # v = 0.5*m - 0.5*g
    np.testing.assert_array_equal(mw, [0.25 - 1.0, -0.125 - 2.0])
    np.testing.assert_array_equal(w, [1.0 - 0.75, -2.0 - 2.125])
    assert (b, mb) == (0.5 - 4.0, 0.5 - 4.0)


# ----------------------------------------------------------------- Adam (adam.rs)
@pytest.mark.parametrize("g", [1.0, -1.0, 2.0, -8.0, 0.5])
def test_adam_first_step_moves_by_lr(g):
    """Step 1: m/c1 = g and v/c2 = g^2 exactly (m = (1-b1) g is the same
    rounding as c1 = 1 - b1^1 times g), so w moves by lr * sign(g)."""
    w = np.array([3.0], F)
    m, v = np.zeros(1, F), np.zeros(1, F)
    b, mb, vb = orc.adam_update(w, [g], 1.0, g, 0.001, 1, m, v, 0.0, 0.0)
    step = -math.copysign(1.0, g) * F(0.001)
    assert w[0] == F(F(3.0) + F(step))
    assert b == F(F(1.0) + F(step))
    assert m[0] == F(F(1.0 - F(0.9)) * F(g))


def test_adam_step_zero_counts_as_one_and_reference_signs():
    w0, w1 = np.array([0.0], F), np.array([0.0], F)
    z = [np.zeros(1, F) for _ in range(4)]
    orc.adam_update(w0, [1.0], 0.0, 1.0, 0.01, 0, z[0], z[1], 0.0, 0.0)
    orc.adam_update(w1, [1.0], 0.0, 1.0, 0.01, 1, z[2], z[3], 0.0, 0.0)
    assert w0[0] == w1[0]
    # zero gradient: no move (adam.rs:177-192); negative gradient: increase (:194-208)
    w = np.array([1.0, 2.0], F)
    b, _, _ = orc.adam_update(w, [0.0, 0.0], 0.5, 0.0, 0.001, 1, np.zeros(2, F), np.zeros(2, F), 0.0, 0.0)
    np.testing.assert_array_equal(w, [1.0, 2.0])
    assert b == 0.5
    w = np.array([0.0], F)
    b, _, _ = orc.adam_update(w, [-1.0], 0.0, -1.0, 0.001, 1, np.zeros(1, F), np.zeros(1, F), 0.0, 0.0)
    assert w[0] > 0 and b > 0


def test_adam_constant_gradient_closed_form():
    """With a constant gradient g, m_t / c1_t = g and v_t / c2_t = g^2 exactly
    in real arithmetic, so each step moves w by about lr; f32 keeps it within 1e-5."""
    w = np.array([0.0], F)
    m, v = np.zeros(1, F), np.zeros(1, F)
    b = mb = vb = 0.0
    prev = 0.0
    for step in range(1, 31):
        b, mb, vb = orc.adam_update(w, [0.25], b, 0.25, 0.01, step, m, v, mb, vb)
        assert (prev - w[0]) == pytest.approx(0.01, rel=1e-4)
        prev = float(w[0])
        # moments: m_t = 0.25 (1 - 0.9^t), v_t = 0.0625 (1 - 0.999^t)
        assert m[0] == pytest.approx(0.25 * (1 - 0.9 ** step), rel=1e-5)
        assert v[0] == pytest.approx(0.0625 * (1 - 0.999 ** step), rel=1e-4)


# ----------------------------------------------------------------- activation derivatives (layer.rs:477-505)
def test_activation_derivatives_reference_values():
    d = lib_d = orc.lib.or_activation_derivative
    assert d(1.0, 1.0, 0) == 1.0 and d(-1.0, 0.0, 0) == 0.0 and d(0.0, 0.0, 0) == 0.0
    assert abs(d(0.0, 0.5, 1) - 0.25) < 1e-6
    assert abs(d(0.0, 0.0, 2) - 1.0) < 1e-6
    assert d(3.0, 7.0, 4) == 1.0 and lib_d(3.0, 7.0, 3) == 1.0
    # sigmoid uses post*(1-post), tanh 1-post^2: post = 0.75 -> 0.1875, 0.4375 (exact)
    assert d(9.0, 0.75, 1) == 0.1875 and d(9.0, 0.75, 2) == 0.4375


# ----------------------------------------------------------------- softmax Jacobian
def test_softmax_local_grads_cancellation_order():
    """For i = 0: terms 2^24 (i == j), 64 terms of +1 (each lost against 2^24
    in round-to-nearest-even), then -2^24.  Left to right gives exactly 0; a
    pairwise or reversed order gives 64."""
    n = 66
    s = np.full(n, 0.5, F)
    go = np.full(n, -4.0, F)       # i != j: go * (-0.5 * 0.5) = +1
    go[0] = 2.0 ** 26              # i == j: 2^26 * 0.5 * 0.5 = 2^24
    go[-1] = 2.0 ** 26             # -> 2^26 * (-0.25) = -2^24
    lg = orc.softmax_local_grads(s, go)
    assert lg[0] == 0.0
    # row 1: the diagonal is -4 * 0.25 = -1, off-diagonal j=0: 2^26 * -0.25 = -2^24 ...
    # the whole row in float64 is the reference's value up to the lost ones
    exact = [sum(float(go[j]) * (float(s[j]) * (1 - float(s[j])) if i == j else -float(s[i]) * float(s[j]))
                 for j in range(n)) for i in range(n)]
    assert abs(float(lg[1]) - exact[1]) <= 64


def test_softmax_local_grads_identity():
    """sum_j J_ij go_j = s_i (go_i - sum_j s_j go_j) for s a softmax."""
    rng = np.random.default_rng(3)
    z = rng.standard_normal(300).astype(F)
    s = orc.layer_activate(z, "softmax")
    go = rng.standard_normal(300).astype(F)
    lg = orc.softmax_local_grads(s, go).astype(np.float64)
    s64, g64 = s.astype(np.float64), go.astype(np.float64)
    want = s64 * (g64 - np.dot(s64, g64))
    np.testing.assert_allclose(lg, want, rtol=1e-4, atol=1e-6)


# ----------------------------------------------------------------- loss (net.rs:404-494)
def test_compute_loss_reference_values():
    act = np.array([0.1, 0.7, 0.2], F)
    assert abs(orc.compute_loss(act, [0, 1, 2], [1]) - (-math.log(0.7))) < 1e-4
    act = np.array([0.3, 0.5, 0.2], F)
    want = (-math.log(0.3) - math.log(0.5)) / 2
    assert abs(orc.compute_loss(act, [0, 1, 2], [0, 1]) - want) < 1e-4
    assert orc.compute_loss(np.array([0.5, 0.5], F), [0, 1], []) == 0.0
    act = np.array([0.5, 0.5, 0.0], F)
    assert abs(orc.compute_loss(act, [0, 1], [2]) - (-math.log(1e-7))) < 1e-3
    # an active label with probability 0 also takes eps
    assert orc.compute_loss(np.array([0.0, 1.0], F), [0, 1], [0]) == orc.compute_loss(act, [0, 1], [2])


def test_compute_loss_gradient_reference_values():
    act = np.array([0.2, 0.5, 0.3], F)
    g = orc.compute_loss_gradient(act, [0, 1, 2], [1], 3)
    assert abs(g[1] + 0.5) < 1e-6 and abs(g[0] - 0.2) < 1e-6 and abs(g[2] - 0.3) < 1e-6
    # repeated labels subtract once per occurrence; labels past the output are skipped;
    # an inactive label gets -1/|labels|; no labels -> all zero
    g = orc.compute_loss_gradient(act, [0, 2], [2, 2, 1, 9], 3)
    np.testing.assert_array_equal(g, [F(0.2), F(-0.25), F(F(F(0.3) - F(0.25)) - F(0.25))])
    np.testing.assert_array_equal(orc.compute_loss_gradient(act, [0, 1, 2], [], 3), np.zeros(3, F))


# ----------------------------------------------------------------- Layer::backward
def _planes(L, k, dim, seed):
    return orc.simhash_planes(dim, k, L, seed)


def test_layer_backward_grad_in_order_and_pre_update_weights():
    """grad_in[j] is a sequential sum over the active list of lg * w (weights
    before the update): rows 2^24, 64 x 1, -2^24 with lg = 1 give 0."""
    dim, n = 4, 66
    W = np.ones((n, dim), F)
    W[0] = 2.0 ** 24
    W[n - 1] = -(2.0 ** 24)
    b = np.zeros(n, F)
    active = np.arange(n, dtype=np.uint32)
    pre = np.ones(n, F)          # relu' = 1
    dense = np.ones(n, F)
    go = np.ones(n, F)
    x = np.array([1.0, 0.0, -1.0, 2.0], F)
    gi = np.zeros(dim, F)
    st = [np.zeros(n * dim, F), np.zeros(n * dim, F), np.zeros(n, F), np.zeros(n, F)]
    Wf = W.reshape(-1).copy()
    orc.lib.or_layer_backward(Wf, b, dim, n, 0, x, active, n, pre, dense, go, n, orc.SGD, 0.0, 0.9, 0.999,
                              1e-8, *st, 0.5, 1, gi.ctypes.data)
    np.testing.assert_array_equal(gi, np.zeros(dim, F))
    # vanilla SGD: w -= 0.5 * (1 * x)
    np.testing.assert_array_equal(Wf.reshape(n, dim)[1], F(1.0) - F(0.5) * x)
    np.testing.assert_array_equal(b, np.full(n, -0.5, F))
    # reversed active order: -2^24 first, and -2^24 + 1 is exact, so the ones survive: 64
    Wf = W.reshape(-1).copy()
    orc.lib.or_layer_backward(Wf, np.zeros(n, F), dim, n, 0, x, active[::-1].copy(), n, pre, dense, go, n,
                              orc.SGD, 0.0, 0.9, 0.999, 1e-8, *st, 0.5, 1, gi.ctypes.data)
    np.testing.assert_array_equal(gi, np.full(dim, 64.0, F))


def test_layer_backward_relu_masks_and_grad_out_length():
    dim, n = 3, 4
    W = np.arange(12, dtype=F).reshape(n, dim)
    b = np.zeros(n, F)
    active = np.array([2, 0, 3], np.uint32)
    pre = np.array([1.0, -1.0, 2.0], F)       # neuron 0 inactive in relu terms
    dense = np.array([0.0, 0.0, 1.0, 2.0], F)
    go = np.array([1.0, 1.0, 4.0], F)         # grad_out shorter than n: id 3 reads 0
    x = np.array([1.0, 2.0, 3.0], F)
    gi = np.zeros(dim, F)
    st = [np.zeros(n * dim, F), np.zeros(n * dim, F), np.zeros(n, F), np.zeros(n, F)]
    Wf = W.reshape(-1).copy()
    orc.lib.or_layer_backward(Wf, b, dim, n, 0, x, active, 3, pre, dense, go, 3, orc.SGD, 0.0, 0.9, 0.999,
                              1e-8, *st, 0.25, 1, gi.ctypes.data)
    # only neuron 2 has a nonzero local grad (4 * 1): grad_in = 4 * W[2]
    np.testing.assert_array_equal(gi, F(4.0) * W[2])
    Wn = Wf.reshape(n, dim)
    np.testing.assert_array_equal(Wn[2], W[2] - F(0.25) * (F(4.0) * x))
    np.testing.assert_array_equal(Wn[[0, 1, 3]], W[[0, 1, 3]])


# ----------------------------------------------------------------- RebuildScheduler (maintenance.rs tests)
def test_scheduler_reference_tests():
    s = orc.RebuildScheduler(10, 0.0)
    assert [s.step() for _ in range(10)] == [False] * 9 + [True]
    s = orc.RebuildScheduler(5, 0.0)
    got = [s.current_step for _ in range(30) if s.step()]
    assert got == [5, 10, 15, 20, 25, 30]
    s = orc.RebuildScheduler(10, 0.0)
    assert s.next_rebuild_step == 10
    for _ in range(10):
        s.step()
    assert s.next_rebuild_step == 20
    s = orc.RebuildScheduler(1, 0.0)
    assert s.step() and s.step()
    s = orc.RebuildScheduler(5, 2.0)
    assert sum(s.step() for _ in range(10000)) >= 1


def test_scheduler_closed_form():
    """rebuild_i_at = sum_{j=0}^{i} floor(base * e^(lambda j)) (maintenance.rs:6-9)."""
    base, lam = 10, 0.5
    s = orc.RebuildScheduler(base, lam)
    got = [s.current_step for _ in range(2000) if s.step()]
    want, acc = [], 0
    for j in range(len(got)):
        acc += math.floor(base * math.exp(lam * j))
        want.append(acc)
    assert got == want and len(got) >= 6
    # should_rebuild jumps: a late call rebuilds once and schedules from there
    s = orc.RebuildScheduler(10, 0.0)
    assert not s.should_rebuild(9) and s.should_rebuild(25) and s.next_rebuild_step == 35


# ----------------------------------------------------------------- forward order and network
def test_forward_ordered_lists_topk_by_count_then_id():
    rng = np.random.default_rng(11)
    L, k, dim, n, cap = 8, 3, 16, 40, 64
    planes = _planes(L, k, dim, 5)
    W = rng.standard_normal((n, dim)).astype(F)
    net = orc.SlideNetOracle([dict(planes=planes, cap=cap, bucket_type=orc.FIFO, W=W, b=np.zeros(n, F),
                                   sampling=1, top_k=12, threshold=1, act="relu")])
    l = net.layers[0]
    for _ in range(5):
        x = rng.standard_normal(dim).astype(F)
        ids, pre, dense = net.layer_forward(l, x)
        qids, qcnt = l["index"].query(orc.hash_dense_batch(planes, x[None]))
        cnt = dict(zip(qids.tolist(), qcnt.tolist()))
        keys = [(-cnt[i], i) for i in ids.tolist()]
        assert keys == sorted(keys) and len(ids) == min(12, len(qids))
        # the same set as the ascending-order forward
        (a_ids, a_pre, _), = orc.slide_layer_oracle(planes, cap, orc.FIFO, W, np.zeros(n, F), x[None],
                                                    sampling=1, top_k=12, threshold=1, act="relu",
                                                    index=l["index"])[0]
        assert sorted(ids.tolist()) == a_ids.tolist()
        np.testing.assert_array_equal(pre[np.argsort(ids)], a_pre)


def _tiny_net(opt=orc.SGD, sampling=1):
    rng = np.random.default_rng(42)
    specs = [dict(planes=_planes(3, 4, 4, 1), cap=128, bucket_type=orc.FIFO,
                  W=rng.normal(0, math.sqrt(2 / 4), (8, 4)).astype(F), b=np.zeros(8, F),
                  sampling=sampling, top_k=8, threshold=1, act="relu"),
             dict(planes=_planes(3, 4, 8, 2), cap=128, bucket_type=orc.FIFO,
                  W=rng.normal(0, math.sqrt(2 / 8), (4, 8)).astype(F), b=np.zeros(4, F),
                  sampling=sampling, top_k=4, threshold=1, act="softmax")]
    return orc.SlideNetOracle(specs, optimizer=opt)


@pytest.mark.parametrize("opt", [orc.SGD, orc.ADAM])
def test_network_train_step_reference_behaviour(opt):
    """net.rs:339-400: finite non-negative loss, step increments, empty batch
    returns 0 and changes nothing, and 20 steps do not double the loss."""
    net = _tiny_net(opt)
    X = np.eye(4, dtype=F)[:3]
    labels = [[0], [1], [2]]
    w0 = [l["W"].copy() for l in net.layers]
    assert net.train_step(np.zeros((0, 4), F), [], 0.1) == 0.0 and net.step == 0
    for a, l in zip(w0, net.layers):
        np.testing.assert_array_equal(a, l["W"])
    first = net.train_step(X, labels, 0.1)
    assert math.isfinite(first) and first >= 0 and net.step == 1
    last = first
    for _ in range(20):
        last = net.train_step(X, labels, 0.1)
    assert net.step == 21 and math.isfinite(last) and last < 2 * first


def test_network_forward_is_layer_chain():
    net = _tiny_net()
    x = np.array([1.0, 0.5, -0.3, 0.2], F)
    outs = net.forward(x)
    ids1, pre1, dense1 = net.layer_forward(net.layers[1], outs[0][2])
    np.testing.assert_array_equal(outs[1][2], dense1)
    assert outs[1][2].shape == (4,) and abs(float(outs[1][2].sum()) - 1.0) < 1e-6
