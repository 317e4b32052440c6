"""GPU parity: WTA / DWTA / MinHash families (hash/wta.rs, dwta.rs, minhash.rs)
against the oracle.  Codes bit-exact (the low 32 bits the C ABI returns);
windows and permutations equal to the oracle's restatement of the rand 0.8.5
draws (the composed stream is parity unpinned); LSH indices over these
families bit-exact against the oracle's insert / query."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F = np.float32


def codes_dense(fam, X):
    return fam.hash_dense_batch(X).cpu().numpy().view(np.uint32)


def rows_sparse(rng, n, dim, nnz, zeros=False):
    from klearu_amd.lsh import SparseVector
    out = []
    for _ in range(n):
        idx = np.sort(rng.choice(dim, nnz, replace=False)).astype(np.uint32)
        val = rng.uniform(-1, 1, nnz).astype(F)
        if zeros:
            val[::4] = 0.0
        out.append(SparseVector(idx, val, dim))
    return out


@pytest.mark.parametrize("dim,k,L,ws,seed", [(64, 4, 3, 8, 42), (784, 6, 50, 8, 7), (300, 3, 10, 5, 1),
                                             (20, 8, 4, 8, 9), (16, 24, 2, 1, 3)])
def test_wta_dwta_windows_and_dense_codes(kh, orc, dim, k, L, ws, seed):
    from klearu_amd.lsh import DwtaHash, WtaHash
    rng = np.random.default_rng(seed)
    X = rng.uniform(-1, 1, (40, dim)).astype(F)
    X[::5, :3] = np.nan
    X[1] = -np.inf
    X[2] = rng.integers(-2, 2, dim)     # ties
    ow = orc.wta_windows(dim, k, L, ws, seed)
    for make in (WtaHash, DwtaHash):
        fam = make(dim, k, L, ws, seed)
        np.testing.assert_array_equal(fam.tables(), ow)
        got = codes_dense(fam, X)
        want = np.array([[orc.wta_hash_dense(ow, x, t) & 0xFFFFFFFF for t in range(L)] for x in X], np.uint32)
        np.testing.assert_array_equal(got, want)


def test_wta_sparse_is_to_dense_and_dwta_sparse_rules(kh, orc):
    from klearu_amd.lsh import DwtaHash, SparseVector, WtaHash
    rng = np.random.default_rng(5)
    dim, k, L, ws = 200, 4, 8, 8
    rows = rows_sparse(rng, 30, dim, 20, zeros=True)
    rows.append(SparseVector(np.zeros(0, np.uint32), np.zeros(0, F), dim))    # empty row
    ow = orc.wta_windows(dim, k, L, ws, 11)
    wta, dwta = WtaHash(dim, k, L, ws, 11), DwtaHash(dim, k, L, ws, 11)
    gw = wta.hash_sparse_batch(rows).cpu().numpy().view(np.uint32)
    gd = dwta.hash_sparse_batch(rows).cpu().numpy().view(np.uint32)
    for r, row in enumerate(rows):
        dense = np.zeros(dim, F)
        dense[row.indices] = row.values
        for t in range(L):
            assert gw[r, t] == orc.wta_hash_dense(ow, dense, t) & 0xFFFFFFFF
            assert gd[r, t] == orc.dwta_hash_sparse(ow, row.indices, row.values, t) & 0xFFFFFFFF


@pytest.mark.parametrize("dim,k,L,seed", [(64, 4, 3, 42), (784, 6, 50, 7), (1000, 24, 5, 2), (10, 4, 2, 3),
                                          (16384, 8, 3, 9), (20000, 8, 3, 5)])
def test_minhash_permutations_and_codes(kh, orc, dim, k, L, seed):
    """Dense rows up to 16384 dims stage their nonzeros in LDS (one block per
    row; at 16384 with every dimension nonzero the staging takes 64 KiB of
    dynamic LDS plus the static bins); wider rows (20000) take the
    per-(row, table) kernel."""
    from klearu_amd.lsh import MinHash
    rng = np.random.default_rng(seed)
    fam = MinHash(dim, k, L, seed)
    op = orc.minhash_perms(dim, L, seed)
    np.testing.assert_array_equal(fam.tables(), op)
    X = (rng.uniform(-1, 1, (30, dim)) * (rng.random((30, dim)) < 0.1)).astype(F)
    X[0] = 0.0                      # all bins empty
    X[1, 3] = -0.0
    X[2] = 1.0                      # every dimension nonzero
    got = codes_dense(fam, X)
    want = np.array([[orc.minhash_hash_dense(op, k, t, x) for t in range(L)] for x in X], np.uint32)
    np.testing.assert_array_equal(got, want)
    rows = rows_sparse(rng, 20, dim, min(15, dim), zeros=True)
    gs = fam.hash_sparse_batch(rows).cpu().numpy().view(np.uint32)
    for r, row in enumerate(rows):
        for t in range(L):   # every stored index counts, stored zeros included
            assert gs[r, t] == orc.minhash_hash(op, k, t, row.indices)


@pytest.mark.parametrize("family", ["WtaHash", "DwtaHash", "MinHash"])
def test_index_over_rank_families_matches_oracle(kh, orc, family):
    from klearu_amd.lsh import LshConfig, create_lsh_index
    rng = np.random.default_rng(17)
    dim, k, L, cap, n = 96, 5, 12, 16, 500
    cfg = LshConfig(hash_function=family, num_tables=L, num_hashes=k, bucket_capacity=cap)
    idx = create_lsh_index(cfg, dim, 123)
    W = rng.uniform(-1, 1, (n, dim)).astype(F)
    if family == "MinHash":
        W *= rng.random((n, dim)) < 0.2
    idx.insert_batch(np.arange(n, dtype=np.uint32), W)
    fam = idx.hash_family
    tabs = fam.tables()
    if family == "MinHash":
        hw = np.array([[orc.minhash_hash_dense(tabs, k, t, w) for t in range(L)] for w in W], np.uint32)
    else:
        hw = np.array([[orc.wta_hash_dense(tabs, w, t) & 0xFFFFFFFF for t in range(L)] for w in W], np.uint32)
    ref = orc.LshIndex(L, k, cap, orc.FIFO)
    ref.insert_many(np.arange(n, dtype=np.uint32), hw & ((1 << k) - 1))
    d, ln, _ = idx.buckets()
    np.testing.assert_array_equal(ln.reshape(-1), ref.len)
    X = W[:8] + rng.normal(0, 0.05, (8, dim)).astype(F)
    for x in X:
        got = sorted(idx.query(x), key=lambda c: c.neuron_id)
        if family == "MinHash":
            q = np.array([orc.minhash_hash_dense(tabs, k, t, x) for t in range(L)], np.uint32)
        else:
            q = np.array([orc.wta_hash_dense(tabs, x, t) & 0xFFFFFFFF for t in range(L)], np.uint32)
        rids, rcnt = ref.query(q & ((1 << k) - 1))
        assert [c.neuron_id for c in got] == rids.tolist()
        assert [c.count for c in got] == rcnt.tolist()


def test_lsh_sparsity_predictor(kh, orc):
    """lsh_predictor.rs:33-43 and its own test (:61-95): well-separated
    observations predict their ids; against the oracle: query counts sorted
    by count descending, ties by id, first top_k."""
    from klearu_amd.lsh import LshConfig, LshSparsityPredictor
    dim = 16
    p = LshSparsityPredictor(LshConfig(num_tables=10, num_hashes=4), dim, 3, 42)
    assert p.predict(np.ones(dim, F)) == []          # empty index
    obs = [(np.full(dim, v, F), [0, 1]) for v in (1.0, 0.9, 0.8)] + \
          [(np.full(dim, v, F), [5, 6]) for v in (-1.0, -0.9, -0.8)]
    p.build_from_observations(obs)
    assert set(p.predict(np.full(dim, 0.95, F))) <= {0, 1} and p.predict(np.full(dim, 0.95, F))
    assert set(p.predict(np.full(dim, -0.95, F))) <= {5, 6}
    # random observations, oracle check of the ordering
    rng = np.random.default_rng(3)
    p = LshSparsityPredictor(LshConfig(num_tables=20, num_hashes=3, bucket_capacity=64), 32, 7, 9)
    obs = [(rng.standard_normal(32).astype(F), rng.choice(40, 4, replace=False).tolist()) for _ in range(60)]
    p.build_from_observations(obs)
    planes = p.index.hash_family.planes()
    ref = orc.LshIndex(20, 3, 64, orc.FIFO)
    ids = np.array([i for _, imp in obs for i in imp], np.uint32)
    rows = np.stack([x for x, imp in obs for _ in imp])
    ref.insert_many(ids, orc.hash_dense_batch(planes, rows))
    X = rng.standard_normal((10, 32)).astype(F)
    got = p.predict_batch(X)
    for x, g in zip(X, got):
        rid, rc = ref.query(orc.hash_dense_batch(planes, x[None]))
        order = sorted(zip(rid.tolist(), rc.tolist()), key=lambda t: (-t[1], t[0]))[:7]
        assert g == [i for i, _ in order]


@pytest.mark.parametrize("relu", [True, False])
def test_sparse_inference_engine(kh, orc, relu):
    """sparse_inference.rs:36-111: top effective_k candidates by count, dot + bias
    (+ ReLU), no fallback; against the oracle's pieces."""
    from klearu_amd.lsh import LshConfig
    from klearu_amd.slide import Layer, LayerConfig, SparseInferenceEngine
    rng = np.random.default_rng(8)
    dim, n, L, k = 64, 300, 12, 4
    W = rng.standard_normal((n, dim)).astype(F) * F(0.1)
    b = rng.standard_normal(n).astype(F) * F(0.1)
    layer = Layer(LayerConfig(dim, n, "Relu", LshConfig(num_tables=L, num_hashes=k, bucket_capacity=32), "TopK", 2, 50),
                  W, b, 5)
    eng = SparseInferenceEngine(1.5)
    planes = layer.index.hash_family.planes()
    d, ln, _ = layer.index.buckets()
    ref = orc.LshIndex(L, k, 32, orc.FIFO)
    ref.data[:] = d.reshape(-1)
    ref.len[:] = ln.reshape(-1)
    X = (rng.standard_normal((12, dim)) * (rng.random((12, dim)) < 0.7)).astype(F)
    got = eng.infer_batch(X, layer, 20, relu)
    eff = int(np.float32(20) * np.float32(1.5))
    for x, g in zip(X, got):
        rid, rc = ref.query(orc.hash_dense_batch(planes, x[None]))
        order = sorted(zip(rid.tolist(), rc.tolist()), key=lambda t: (-t[1], t[0]))[:eff]
        assert [i for i, _ in g] == [i for i, _ in order]
        for i, a in g:
            z = orc.neuron_forward(W[i], b[i], x)
            assert np.float32(a) == (np.float32(max(z, 0.0)) if relu else np.float32(z))
    # multiplier 0 -> nothing; an index query with no candidates -> nothing (no fallback)
    assert SparseInferenceEngine(0.0).infer(X[0], layer, 20) == []
