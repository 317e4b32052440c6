"""GPU parity: SLIDE training (Layer::backward, Network::train_step / predict,
index rebuilds) against the oracle's restatement.

Bar: weights, biases, grad_input and predictions bit-exact (every f32
operation of the path is the reference's, in its order, and the activations
used here are ReLU / identity / softmax / sigmoid, whose GPU forms are exact);
the loss within 1e-5 relative (the GPU's logf is not glibc's).  Top-k layers
list active neurons by count, then id, as the reference's sampler does; the
other samplers use ascending ids on both sides (the reference's HashMap order
is not reproducible).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

F = np.float32
SAMP = {"Vanilla": 0, "TopK": 1, "Threshold": 2}
ACTS = {"Relu": "relu", "Sigmoid": "sigmoid", "Tanh": "tanh", "Softmax": "softmax", "Identity": "identity"}


def build(orc, specs, optimizer="Sgd", momentum=0.9, rebuild_base=100, rebuild_decay=0.1):
    """specs: dicts(dim, n, k, L, cap, sampling, top_k, threshold, act, W, b, seed).
    Returns (gpu Network, gpu layers, oracle net)."""
    from klearu_amd.lsh import HashFamily, LshConfig, LshIndex
    from klearu_amd.slide import Layer, LayerConfig, Network
    layers, ospecs = [], []
    for s in specs:
        planes = orc.simhash_planes(s["dim"], s["k"], s["L"], s["seed"])
        fam = HashFamily.from_planes(planes)
        idx = LshIndex(fam, orc.FIFO, s["cap"])
        cfg = LayerConfig(s["dim"], s["n"], s["act"], LshConfig(num_tables=s["L"], num_hashes=s["k"],
                                                               bucket_capacity=s["cap"]),
                          s["sampling"], s["threshold"], s["top_k"])
        layers.append(Layer(cfg, s["W"], s["b"], 0, index=idx))
        ospecs.append(dict(planes=planes, cap=s["cap"], bucket_type=orc.FIFO, W=s["W"], b=s["b"],
                           sampling=SAMP[s["sampling"]], top_k=s["top_k"], threshold=s["threshold"],
                           act=ACTS[s["act"]]))
    net = Network(layers, optimizer, momentum=momentum, rebuild_base=rebuild_base, rebuild_decay=rebuild_decay)
    onet = orc.SlideNetOracle(ospecs, optimizer=orc.SGD if optimizer == "Sgd" else orc.ADAM, momentum=momentum,
                              rebuild_base=rebuild_base, rebuild_decay=rebuild_decay)
    return net, layers, onet


def spec(rng, dim, n, act, sampling="TopK", top_k=None, k=4, L=6, cap=32, scale=None, seed=7, threshold=2):
    sc = scale if scale is not None else np.sqrt(2.0 / dim)
    return dict(dim=dim, n=n, k=k, L=L, cap=cap, sampling=sampling, top_k=n if top_k is None else top_k,
                threshold=threshold, act=act, W=rng.normal(0, sc, (n, dim)).astype(F),
                b=rng.normal(0, 0.01, n).astype(F), seed=seed)


def check_same(layers, onet, what):
    for i, (l, ol) in enumerate(zip(layers, onet.layers)):
        w, b = l.weights()
        np.testing.assert_array_equal(w, ol["W"], err_msg=f"{what}: layer {i} weights")
        np.testing.assert_array_equal(b, ol["b"], err_msg=f"{what}: layer {i} bias")


def run_steps(net, layers, onet, X, labels, lr, steps, bs):
    for s in range(steps):
        lo = (s * bs) % X.shape[0]
        xb, lb = X[lo:lo + bs], labels[lo:lo + bs]
        got = net.train_step(xb, lb, lr)
        want = onet.train_step(xb, lb, lr)
        print(f"step {s}: loss gpu {got:.7g} oracle {want:.7g}")
        assert got == pytest.approx(want, rel=1e-5, abs=1e-6)
        check_same(layers, onet, f"after step {s}")
        assert net.step == onet.step


def data(rng, n, dim, n_out, density=0.3, max_labels=2):
    X = (rng.random((n, dim)) * (rng.random((n, dim)) < density)).astype(F)
    labels = [sorted(rng.choice(n_out, rng.integers(1, max_labels + 1), replace=False).tolist()) for _ in range(n)]
    return X, labels


@pytest.mark.parametrize("optimizer", ["Sgd", "Adam"])
def test_reference_bench_shape_train_steps(kh, orc, optimizer):
    """The reference's train-step benchmark net (benches/benchmarks.rs:238-270):
    128 -> 64 ReLU -> 10 softmax, top-k = all, 10 tables of 6 bits."""
    rng = np.random.default_rng(1 + (optimizer == "Adam"))
    specs = [spec(rng, 128, 64, "Relu", k=6, L=10, cap=128, seed=11),
             spec(rng, 64, 10, "Softmax", k=6, L=10, cap=128, seed=12)]
    net, layers, onet = build(orc, specs, optimizer)
    X, labels = data(rng, 24, 128, 10)
    run_steps(net, layers, onet, X, labels, 0.01, 4, 8)


def test_sparse_topk_layers_and_rebuilds(kh, orc):
    """Top-k below the candidate count (count order matters), a rebuild every
    two steps, SGD with momentum; predictions after training."""
    rng = np.random.default_rng(5)
    specs = [spec(rng, 96, 160, "Relu", top_k=40, k=5, L=8, cap=24, seed=21),
             spec(rng, 160, 120, "Softmax", top_k=30, k=5, L=8, cap=24, seed=22)]
    net, layers, onet = build(orc, specs, "Sgd", rebuild_base=2, rebuild_decay=0.0)
    X, labels = data(rng, 40, 96, 120, max_labels=3)
    run_steps(net, layers, onet, X, labels, 0.05, 6, 10)
    sched = net.scheduler()
    assert (sched.rebuild_count, sched.next_rebuild_step) == (onet.scheduler.rebuild_count,
                                                            onet.scheduler.next_rebuild_step)
    # indices after the rebuilds equal the oracle's (rebuilt from the same weights)
    for l, ol in zip(layers, onet.layers):
        data_, ln, _ = l.index.buckets()
        np.testing.assert_array_equal(ln.reshape(-1), ol["index"].len)
        cap = ol["cap"]
        od = ol["index"].data.reshape(ln.shape[0], ln.shape[1], cap)
        for t in range(ln.shape[0]):
            for bk in range(ln.shape[1]):
                np.testing.assert_array_equal(data_[t, bk, :ln[t, bk]], od[t, bk, :ln[t, bk]])
    got = net.predict_batch(X[:6]).cpu().numpy()
    for i in range(6):
        np.testing.assert_array_equal(got[i], onet.predict(X[i]))


def test_vanilla_threshold_sigmoid_identity(kh, orc):
    rng = np.random.default_rng(9)
    specs = [spec(rng, 64, 80, "Sigmoid", sampling="Vanilla", k=4, L=5, cap=16, seed=31),
             spec(rng, 80, 48, "Identity", sampling="Threshold", threshold=2, k=4, L=5, cap=16, seed=32),
             spec(rng, 48, 30, "Softmax", sampling="TopK", top_k=12, k=4, L=5, cap=16, seed=33)]
    net, layers, onet = build(orc, specs, "Adam")
    X, labels = data(rng, 16, 64, 30)
    run_steps(net, layers, onet, X, labels, 0.01, 3, 8)


def test_label_edge_cases_and_empty_batch(kh, orc):
    rng = np.random.default_rng(13)
    specs = [spec(rng, 32, 40, "Relu", top_k=20, seed=41), spec(rng, 40, 16, "Softmax", top_k=8, seed=42)]
    net, layers, onet = build(orc, specs, "Sgd", momentum=0.0)
    assert net.train_step(np.zeros((0, 32), F), [], 0.1) == 0.0 and net.step == 0
    X, _ = data(rng, 5, 32, 16)
    # no labels, a repeated label, a label past the output, an inactive-or-not label
    labels = [[], [3, 3], [15, 99], [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11], [7]]
    got = net.train_step(X, labels, 0.2)
    want = onet.train_step(X, labels, 0.2)
    assert got == pytest.approx(want, rel=1e-5)
    check_same(layers, onet, "label edge cases")


def test_layer_backward_entry_matches_oracle(kh, orc):
    """kh_slide_layer_backward on a softmax layer and a ReLU layer, given the
    oracle's own LayerOutput (active list in the sampler's order)."""
    rng = np.random.default_rng(17)
    for act in ("Softmax", "Relu"):
        s = spec(rng, 48, 64, act, top_k=20, seed=51)
        net, layers, onet = build(orc, [s], "Adam")
        l, ol = layers[0], onet.layers[0]
        x = (rng.random(48) * (rng.random(48) < 0.5)).astype(F)
        ids, pre, dense = onet.layer_forward(ol, x)
        g = rng.standard_normal(64).astype(F)
        from klearu_amd.slide import LayerOutput
        out = LayerOutput(dense, ids, pre)
        gi = l.backward(x, out, g[:50], 0.01, 3)          # a shorter grad_output reads 0 past it
        onet.step = 3
        ogi = onet.layer_backward(ol, x, (ids, pre, dense), g[:50], 0.01)
        np.testing.assert_array_equal(gi, ogi)
        check_same(layers, onet, f"layer backward {act}")


def test_cfg1_shaped_network(kh, orc):
    """cfg1's hidden layer (784 -> 1024 ReLU, SimHash K6 L50 FIFO 128, inputs 80%
    zeros) under a 1024 -> 32 softmax head, top-k sampling, batch 16."""
    rng = np.random.default_rng(23)
    specs = [spec(rng, 784, 1024, "Relu", top_k=256, k=6, L=50, cap=128, scale=0.01, seed=42),
             spec(rng, 1024, 32, "Softmax", top_k=32, k=6, L=50, cap=128, seed=43)]
    net, layers, onet = build(orc, specs, "Sgd")
    X = (rng.random((32, 784)) * (rng.random((32, 784)) < 0.2)).astype(F)
    labels = [[int(v)] for v in rng.integers(0, 32, 32)]
    run_steps(net, layers, onet, X, labels, 0.01, 2, 16)


def test_rebuild_scheduler_and_index_rebuild(kh, orc):
    from klearu_amd.lsh import HashFamily, LshIndex
    planes = orc.simhash_planes(40, 4, 6, 3)
    idx = LshIndex(HashFamily.from_planes(planes), orc.FIFO, 8)
    rng = np.random.default_rng(2)
    W = rng.standard_normal((50, 40)).astype(F)
    idx.insert_batch(np.arange(50, dtype=np.uint32), W)
    ids = rng.permutation(30).astype(np.uint32)
    idx.rebuild([(int(i), W[i]) for i in ids])
    ref = orc.LshIndex(6, 4, 8, orc.FIFO)
    ref.insert_many(ids, orc.hash_dense_batch(planes, W[ids]))
    d, ln, cnt = idx.buckets()
    np.testing.assert_array_equal(ln.reshape(-1), ref.len)
    np.testing.assert_array_equal(cnt.reshape(-1), ref.count)
    od = ref.data.reshape(d.shape)
    for t in range(d.shape[0]):
        for b in range(d.shape[1]):
            np.testing.assert_array_equal(d[t, b, :ln[t, b]], od[t, b, :ln[t, b]])
    idx.rebuild([])
    assert idx.buckets()[1].sum() == 0


def test_sparse_examples_match_dense_training(kh, orc):
    """train_step_sparse densifies each example as SparseVector::to_dense does
    (unsorted entries, repeated indices: the later value wins, explicit zeros):
    the same weights as training on the dense rows."""
    from klearu_amd.lsh import SparseVector
    rng = np.random.default_rng(31)
    specs = [spec(rng, 200, 64, "Relu", top_k=48, k=5, L=6, cap=32, seed=61),
             spec(rng, 64, 40, "Softmax", top_k=16, k=5, L=6, cap=32, seed=62)]
    net, layers, onet = build(orc, specs, "Adam")
    B = 12
    vecs, X = [], np.zeros((B, 200), F)
    for r in range(B):
        idx = rng.choice(200, 30, replace=False)
        val = rng.random(30).astype(F)
        val[:3] = 0.0
        idx = np.concatenate([idx, idx[5:9]])          # repeats: these later values win
        val = np.concatenate([val, rng.random(4).astype(F)])
        for i, v in zip(idx, val):
            X[r, i] = v
        vecs.append(SparseVector(idx.astype(np.uint32), val, 200))
    labels = [[int(rng.integers(0, 40))] for _ in range(B)]
    for step in range(2):
        got = net.train_step_sparse(vecs, labels, 0.01)
        want = onet.train_step(X, labels, 0.01)
        assert got == pytest.approx(want, rel=1e-5)
        check_same(layers, onet, f"sparse step {step}")
    p = net.predict_sparse(vecs[:4]).cpu().numpy()
    for i in range(4):
        np.testing.assert_array_equal(p[i], onet.predict(X[i]))
