"""Pins the oracle's buckets, LSH index, sampling and SLIDE neuron (CPU only).

Known answers come from the reference's own tests:
  FIFO  crates/klearu-core/src/bucket/fifo.rs:74-161
  Reservoir bucket/reservoir.rs:110-225 (cap bound, determinism, fairness)
  index lsh/index.rs:401-693 (self query count == L, duplicates, rebuild/clear)
  TopK  sampling/topk.rs:41-98;  Threshold sampling/threshold.rs:50-125
SplitMix64 (bucket/reservoir.rs:40-47) is pinned by its published output stream
for seed 0.  Neuron sums are pinned by exact integer arithmetic and by float64
bounds.
"""
import numpy as np
import pytest

FIFO, RES = 0, 1


def bucket_seq(orc, cap, typ, ids):
    idx = orc.LshIndex(1, 1, cap, typ)
    idx.insert_many(ids, np.zeros(len(ids), np.uint32))
    return list(idx.bucket(0, 0)), int(idx.count[0])


def test_fifo_kats(orc):
    assert bucket_seq(orc, 4, FIFO, [1, 2, 3])[0] == [1, 2, 3]
    assert bucket_seq(orc, 3, FIFO, [10, 20, 30, 40])[0] == [20, 30, 40]
    assert bucket_seq(orc, 2, FIFO, [1, 2, 3])[0] == [2, 3]
    assert bucket_seq(orc, 2, FIFO, [1, 2, 3, 4])[0] == [3, 4]
    assert bucket_seq(orc, 2, FIFO, [1, 2, 3, 4, 5])[0] == [4, 5]
    assert bucket_seq(orc, 1, FIFO, [10])[0] == [10]
    assert bucket_seq(orc, 1, FIFO, [10, 20])[0] == [20]


def test_splitmix64_stream(orc):
    # SplitMix64 from state 0: outputs are mix(k * golden) for k = 1, 2, 3.
    g = 0x9E3779B97F4A7C15
    mask = (1 << 64) - 1
    expect = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    for k, e in enumerate(expect):
        assert orc.lib.or_reservoir_rand((k * g) & mask, mask) == e


def test_reservoir_kats(orc):
    seq, cnt = bucket_seq(orc, 4, RES, [1, 2, 3])
    assert seq == [1, 2, 3] and cnt == 3
    seq, cnt = bucket_seq(orc, 3, RES, list(range(100)))
    assert len(seq) <= 3 and cnt == 100
    assert bucket_seq(orc, 4, RES, list(range(50))) == bucket_seq(orc, 4, RES, list(range(50)))
    assert len(bucket_seq(orc, 1, RES, [10] + list(range(11, 100)))[0]) == 1


def test_reservoir_fairness(orc):
    # reservoir.rs:196-225: ids i + 1000*trial, cap 5, 10 inserts, 10000 trials.
    counts = np.zeros(10)
    for trial in range(10000):
        seq, _ = bucket_seq(orc, 5, RES, [i + trial * 1000 for i in range(10)])
        for v in seq:
            counts[v - trial * 1000] += 1
    ratio = counts / 5000.0
    assert np.all((ratio >= 0.5) & (ratio <= 1.5)), ratio


def test_reservoir_replacement_rule(orc):
    # Brute-force the replacement rule against the SplitMix64 stream above:
    # after cap inserts, insert number c (1-based) with id v replaces slot
    # r(seed+1) % cap iff r(seed) % c < cap, seed = c * 0x517cc1b727220a95 + v.
    mask = (1 << 64) - 1
    cap = 4
    ids = [7, 9, 11, 13, 1000, 2000, 3000, 4000, 5000, 6000, 77, 88]
    state = []
    for c, v in enumerate(ids, start=1):
        if len(state) < cap:
            state.append(v)
            continue
        seed = (c * 0x517CC1B727220A95 + v) & mask
        j = orc.lib.or_reservoir_rand(seed, c)
        if j < cap:
            state[orc.lib.or_reservoir_rand((seed + 1) & mask, cap)] = v
    assert bucket_seq(orc, cap, RES, ids)[0] == state


@pytest.mark.parametrize("typ", [FIFO, RES])
def test_self_query_count_equals_L(orc, typ):
    # lsh/index.rs:417-434 (L=4, K=3, cap 32, dim 8, weights below)
    L, K = 4, 3
    planes = orc.simhash_planes(8, K, L, 42)
    w = np.array([1.0, 0.5, -0.3, 0.0, 2.0, -1.0, 0.1, 0.7], np.float32)
    codes = orc.hash_dense_batch(planes, w)
    idx = orc.LshIndex(L, K, 32, typ)
    idx.insert_many([100], codes)
    ids, cnt = idx.query(codes[0])
    assert list(ids) == [100] and list(cnt) == [L]
    # index.rs:657 duplicate insert -> counted once per occurrence
    idx.insert_many([100], codes)
    ids, cnt = idx.query(codes[0])
    assert list(ids) == [100] and list(cnt) == [2 * L]


def test_query_union_is_bucket_union(orc):
    L, K, cap = 6, 4, 8
    rng = np.random.default_rng(2)
    idx = orc.LshIndex(L, K, cap, FIFO)
    codes = rng.integers(0, 1 << K, (300, L)).astype(np.uint32)
    idx.insert_many(np.arange(300, dtype=np.uint32), codes)
    q = rng.integers(0, 1 << K, L).astype(np.uint32)
    ids, cnt = idx.query(q)
    allv = np.concatenate([idx.bucket(t, int(q[t])) for t in range(L)])
    u, c = np.unique(allv, return_counts=True)
    np.testing.assert_array_equal(ids, u)
    np.testing.assert_array_equal(cnt, c)
    # every FIFO bucket holds the last <= cap ids inserted into it, in order
    for t in range(L):
        for b in range(1 << K):
            expect = [i for i in range(300) if codes[i, t] == b][-cap:]
            assert list(idx.bucket(t, b)) == expect


def test_empty_index_query(orc):
    idx = orc.LshIndex(4, 3, 32, FIFO)
    ids, cnt = idx.query(np.zeros(4, np.uint32))
    assert ids.size == 0


def test_topk_kats(orc):
    tk = lambda c, k: list(orc.sample_topk([a for a, _ in c], [b for _, b in c], k))
    assert tk([(0, 3), (1, 5), (2, 1), (3, 4)], 2) == [1, 3]
    assert tk([(0, 1), (1, 2)], 10) == [1, 0]
    assert tk([(10, 5), (20, 3), (30, 1)], 3) == [10, 20, 30]
    assert tk([], 5) == []
    assert tk([(0, 5), (1, 3)], 0) == []
    assert tk([(5, 3), (2, 3), (8, 3), (1, 3)], 2) == [1, 2]
    assert tk([(42, 10)], 5) == [42]


def test_threshold_kats(orc):
    th = lambda c, t: list(orc.sample_threshold([a for a, _ in c], [b for _, b in c], t))
    assert th([(0, 5), (1, 2), (2, 3), (3, 1)], 3) == [0, 2]
    assert th([(0, 5), (1, 2), (2, 3)], 1) == [0, 1, 2]
    assert th([(0, 3), (1, 5), (2, 1)], 10) == [1]
    assert th([(5, 3), (2, 3), (8, 3)], 100) == [2]
    assert th([], 1) == []
    assert th([(42, 1)], 1) == [42]
    assert th([(42, 2)], 5) == [42]
    assert th([(0, 0), (1, 0), (2, 0)], 0) == [0, 1, 2]


def test_neuron_forward_exact_and_sparse(orc):
    rng = np.random.default_rng(4)
    w = rng.integers(-30, 31, 784).astype(np.float32)
    x = rng.integers(0, 5, 784).astype(np.float32)
    x[rng.random(784) < 0.8] = 0.0
    exact = float(w.astype(np.int64) @ x.astype(np.int64)) + 3.0
    assert orc.neuron_forward(w, 3.0, x) == exact
    nz = np.nonzero(x)[0].astype(np.uint32)
    assert orc.neuron_forward_sparse(w, 3.0, nz, x[nz]) == exact
    # float inputs: dense == sparse bit for bit (zero terms do not change a
    # sequential sum), and within the sequential-sum error bound of float64
    wf = rng.normal(0, 0.01, 784).astype(np.float32)
    xf = rng.random(784).astype(np.float32)
    xf[rng.random(784) < 0.8] = 0.0
    nz = np.nonzero(xf)[0].astype(np.uint32)
    d = orc.neuron_forward(wf, 0.0, xf)
    assert d.tobytes() == orc.neuron_forward_sparse(wf, 0.0, nz, xf[nz]).tobytes()
    ref = float(wf.astype(np.float64) @ xf.astype(np.float64))
    bound = 784 * 2 ** -23 * float(np.abs(wf.astype(np.float64)) @ np.abs(xf))
    assert abs(float(d) - ref) <= bound


def test_activations(orc):
    pre = np.array([-2.0, -0.5, 0.0, 0.5, 3.0], np.float32)
    np.testing.assert_array_equal(orc.layer_activate(pre, "relu"), np.maximum(pre, 0))
    sm = orc.layer_activate(pre, "softmax")
    ref = np.exp(pre.astype(np.float64) - 3.0)
    np.testing.assert_allclose(sm, ref / ref.sum(), rtol=1e-6)
    assert abs(float(sm.sum()) - 1.0) < 1e-6
    np.testing.assert_allclose(orc.layer_activate(pre, "sigmoid"), 1 / (1 + np.exp(-pre.astype(np.float64))),
                               rtol=1e-6)
    np.testing.assert_allclose(orc.layer_activate(pre, "tanh"), np.tanh(pre.astype(np.float64)), rtol=1e-6)
    # all -inf: exp(-inf - -inf) is NaN, the sum is not > 0, so the
    # reference falls back to the uniform distribution (layer.rs:301-307)
    u = orc.layer_activate(np.full(4, -np.inf, np.float32), "softmax")
    np.testing.assert_array_equal(u, np.full(4, 0.25, np.float32))


def _union_below(idx, codes, n):
    """Brute-force active set of Layer::forward under Vanilla sampling
    (layer.rs:67-86): the union of the L query buckets; all neurons when the
    union is empty; then ids >= n dropped."""
    allv = np.concatenate([idx.bucket(t, int(codes[t])) for t in range(idx.L)])
    u = np.unique(allv)
    if u.size == 0:
        return np.arange(n, dtype=np.uint32)
    return u[u < n]


def test_slide_forward_invariants(orc):
    """or_slide_forward against its parts checked independently: the active
    set is the brute-force bucket union (empty -> all neurons, ids >= n
    dropped after the fallback), pre-activations lie within the sequential-sum
    error bound of float64 W x + b, ReLU is max(pre, 0), softmax matches the
    float64 softmax over the active set and sums to 1; TopK sampling keeps the
    sample_topk KATs' order."""
    rng = np.random.default_rng(11)
    L, K, dim, n, cap = 6, 4, 32, 40, 6
    planes = rng.choice(np.array([-1, 0, 1], np.int8), size=(L, K, dim), p=[1 / 6, 2 / 3, 1 / 6])
    W = rng.normal(0, 0.1, (n, dim)).astype(np.float32)
    b = rng.normal(0, 0.1, n).astype(np.float32)
    X = rng.random((8, dim)).astype(np.float32)
    X[rng.random(X.shape) < 0.5] = 0.0
    idx = orc.LshIndex(L, K, cap, FIFO)
    idx.insert_many(np.arange(n, dtype=np.uint32), orc.hash_dense_batch(planes, W))
    # ids beyond the layer share buckets too and must be filtered out
    idx.insert_many(np.arange(n, n + 12, dtype=np.uint32), orc.hash_dense_batch(planes, X[:4].repeat(3, 0)))
    codes = orc.hash_dense_batch(planes, X)
    for act in ("relu", "softmax"):
        out, _ = orc.slide_layer_oracle(planes, cap, FIFO, W, b, X, act=act, index=idx)
        for r, (ids, pre, a) in enumerate(out):
            np.testing.assert_array_equal(ids, _union_below(idx, codes[r], n))
            ref = W[ids].astype(np.float64) @ X[r].astype(np.float64) + b[ids]
            bound = (dim + 1) * 2 ** -23 * (np.abs(W[ids].astype(np.float64)) @ np.abs(X[r]) + np.abs(b[ids]))
            assert np.all(np.abs(pre - ref) <= bound + 1e-30)
            if act == "relu":
                np.testing.assert_array_equal(a, np.maximum(pre, 0))
            else:
                e = np.exp(pre.astype(np.float64) - pre.max())
                np.testing.assert_allclose(a, e / e.sum(), rtol=1e-5, atol=1e-7)
                assert abs(float(a.astype(np.float64).sum()) - 1.0) < 1e-5
    # TopK sampling: the k best by (count desc, id asc), then ids >= n dropped
    out, _ = orc.slide_layer_oracle(planes, cap, FIFO, W, b, X, sampling=1, top_k=5, index=idx)
    for r, (ids, _, _) in enumerate(out):
        u, c = idx.query(codes[r])
        sel = orc.sample_topk(u, c, 5)
        sel = np.arange(n, dtype=np.uint32) if sel.size == 0 else sel
        np.testing.assert_array_equal(ids, np.sort(sel[sel < n]))
    # empty index: every neuron is active
    empty = orc.LshIndex(L, K, cap, FIFO)
    out, _ = orc.slide_layer_oracle(planes, cap, FIFO, W, b, X[:2], index=empty)
    for ids, _, _ in out:
        np.testing.assert_array_equal(ids, np.arange(n, dtype=np.uint32))


def _one_bucket(orc, cap, typ):
    return orc.LshIndex(1, 1, cap, typ)


@pytest.mark.parametrize("typ", [FIFO, RES])
def test_remove_kats(orc, typ):
    """Bucket::remove (fifo.rs:117-139, reservoir.rs:148-170): an existing id
    goes, a missing id or an empty bucket changes nothing; the slot is filled
    by the last entry as Vec::swap_remove documents (the removed element is
    replaced by the last one), and the insertion count stays."""
    z = lambda n: np.zeros(n, np.uint32)  # noqa: E731 -- every vector in bucket 0
    b = _one_bucket(orc, 4, typ)
    b.insert_many([1, 2, 3], z(3))
    b.remove_many([2], z(1))
    assert list(b.bucket(0, 0)) == [1, 3] and 2 not in b.bucket(0, 0)
    b = _one_bucket(orc, 4, typ)
    b.insert_many([1], z(1))
    b.remove_many([99], z(1))
    assert list(b.bucket(0, 0)) == [1]
    b = _one_bucket(orc, 4, typ)
    b.remove_many([1], z(1))
    assert list(b.bucket(0, 0)) == []
    # swap_remove: [1, 2, 3, 4] without 2 is [1, 4, 3]; only the first of two
    # equal entries goes
    b = _one_bucket(orc, 6, typ)
    b.insert_many([1, 2, 3, 4, 2], z(5))
    b.remove_many([2], z(1))
    assert list(b.bucket(0, 0)) == [1, 2, 3, 4]
    b = _one_bucket(orc, 4, typ)
    b.insert_many([1, 2, 3, 4], z(4))
    cnt = int(b.count[0])
    b.remove_many([2], z(1))
    assert list(b.bucket(0, 0)) == [1, 4, 3] and int(b.count[0]) == cnt


def test_fifo_eviction_after_remove(orc):
    """After a removal the FIFO appends while it has room and then evicts its
    first entry (fifo.rs:27-33): [1,2,3,4] - 2 -> [1,4,3] + 5 -> [1,4,3,5]
    + 6 -> [4,3,5,6]."""
    z = lambda n: np.zeros(n, np.uint32)  # noqa: E731
    b = _one_bucket(orc, 4, FIFO)
    b.insert_many([1, 2, 3, 4], z(4))
    b.remove_many([2], z(1))
    b.insert_many([5], z(1))
    assert list(b.bucket(0, 0)) == [1, 4, 3, 5]
    b.insert_many([6], z(1))
    assert list(b.bucket(0, 0)) == [4, 3, 5, 6]


def test_reservoir_refills_after_remove(orc):
    """A full reservoir bucket that loses an entry pushes the next insert
    (len < cap) whatever its count (reservoir.rs:51-58)."""
    z = lambda n: np.zeros(n, np.uint32)  # noqa: E731
    b = _one_bucket(orc, 3, RES)
    b.insert_many(list(range(10, 30)), z(20))
    full = list(b.bucket(0, 0))
    assert len(full) == 3 and int(b.count[0]) == 20
    b.remove_many([full[0]], z(1))
    b.insert_many([99], z(1))
    assert list(b.bucket(0, 0)) == [full[2], full[1], 99] and int(b.count[0]) == 21


@pytest.mark.parametrize("typ", [FIFO, RES])
def test_remove_all_matches_targeted_remove(orc, typ):
    """remove (every bucket, lsh/index.rs:278-280) leaves the same tables as
    remove_with_weights (lsh/index.rs:271-276) for ids that live only in the
    buckets their own codes name, and removed ids appear nowhere
    (index.rs:455-483)."""
    rng = np.random.default_rng(7)
    L, k, cap, n = 6, 3, 8, 120
    codes = rng.integers(0, 1 << k, (n, L)).astype(np.uint32)
    ids = np.arange(n, dtype=np.uint32)
    a, b = orc.LshIndex(L, k, cap, typ), orc.LshIndex(L, k, cap, typ)
    a.insert_many(ids, codes)
    b.insert_many(ids, codes)
    gone = rng.choice(n, 30, replace=False).astype(np.uint32)
    a.remove_many(gone, codes[gone])
    b.remove_all(gone)
    np.testing.assert_array_equal(a.len, b.len)
    for t in range(L):
        for bb in range(1 << k):
            assert list(a.bucket(t, bb)) == list(b.bucket(t, bb))
            assert not set(a.bucket(t, bb).tolist()) & set(gone.tolist())
