"""GPU parity: SimHash/SRP hashing, LSH index build + query, SLIDE layer forward.

Bars (north_star): hash codes, bucket contents, candidate sets, hit counts and
active sets bit-exact against the oracle; fp32 pre-activations bit-exact (the
kernel replays the reference's sequential sum); softmax/tanh within 1e-5
relative.  Shapes: cfg1 (784-d inputs, 1024 neurons, SimHash K6 L50, FIFO cap
128, batch 128, 80% zeros), a scaled cfg5 (128-d hidden, K9 L50 reservoir cap
128, sparse inputs) and small edge cases (empty buckets, duplicates, all-zero
inputs, cleared index).
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

FIFO, RESERVOIR = 0, 1


def cfg1_inputs(rng, batch, dim=784):
    x = rng.uniform(0, 1, (batch, dim)).astype(np.float32)
    x[rng.uniform(0, 1, (batch, dim)) < 0.8] = 0.0
    return x


def sparse_rows(rng, batch, dim, nnz_mean, empty_every=0):
    from klearu_amd.lsh import SparseVector
    rows = []
    for b in range(batch):
        nnz = 0 if (empty_every and b % empty_every == 0) else int(rng.integers(1, 2 * nnz_mean))
        idx = np.sort(rng.choice(dim, size=min(nnz, dim), replace=False)).astype(np.uint32)
        rows.append(SparseVector(idx, rng.uniform(0, 1, idx.size).astype(np.float32), dim))
    return rows


# ----------------------------------------------------------------------------- families
@pytest.mark.parametrize("dim,k,L,seed", [(784, 6, 50, 42), (128, 9, 50, 1_000_042), (33, 24, 3, 0),
                                          (5, 1, 1, 7)])
def test_simhash_planes_match_stdrng(kh, orc, dim, k, L, seed):
    from klearu_amd.lsh import SimHash
    fam = SimHash(dim, k, L, seed)
    assert (fam.k(), fam.input_dim(), fam.num_tables()) == (k, dim, L)
    np.testing.assert_array_equal(fam.planes(), orc.simhash_planes(dim, k, L, seed))


@pytest.mark.parametrize("dim,k,L,sp,seed", [(128, 9, 50, 1.0 / 3.0, 42), (784, 6, 10, 0.1, 3),
                                             (64, 4, 2, 1.0, 9), (64, 4, 2, 0.0, 9)])
def test_srp_planes_match_stdrng(kh, orc, dim, k, L, sp, seed):
    from klearu_amd.lsh import SparseRandomProjection
    fam = SparseRandomProjection(dim, k, L, sp, seed)
    np.testing.assert_array_equal(fam.planes(), orc.srp_planes(dim, k, L, sp, seed))


@pytest.mark.parametrize("dim,k,L,batch", [(784, 6, 50, 128), (128, 9, 50, 300), (33, 24, 3, 5),
                                           (4096, 16, 8, 3)])
def test_hash_dense_bit_exact(kh, orc, dim, k, L, batch):
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(dim + k)
    fam = SimHash(dim, k, L, 42)
    x = cfg1_inputs(rng, batch, dim)
    x[0] = 0.0                       # all-zero input: every bit set (dot 0 >= 0)
    if batch > 2:
        x[1] = -x[1]                 # negative values
    got = fam.hash_dense_batch(x).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, orc.hash_dense_batch(fam.planes(), x))
    assert np.all(got[0] == (1 << k) - 1)
    assert fam.hash_dense(x[2], L - 1) == orc.hash_dense(fam.planes(), x[2], L - 1)


def _hard_rows(rng, batch, dim):
    """Rows for the matrix-core hashing path (batches of >= 1024 rows): most are
    N(0,1); the rest force its exact fallback -- small integers (many sums
    exactly zero), zero and -0.0 rows, denormals, tiny and huge magnitudes,
    overflowing sums, inf and NaN."""
    x = rng.standard_normal((batch, dim)).astype(np.float32)
    q = batch // 8
    x[:q] = rng.integers(-2, 3, (q, dim)).astype(np.float32)
    x[q] = 0.0
    x[q + 1] = -0.0
    x[q + 2] = rng.standard_normal(dim).astype(np.float32) * np.float32(1e-41)
    x[q + 3] = rng.standard_normal(dim).astype(np.float32) * np.float32(1e-30)
    x[q + 4] = rng.standard_normal(dim).astype(np.float32) * np.float32(1e36)
    x[q + 5, ::3] = np.float32(3e38)
    x[q + 6, dim // 2] = np.inf
    x[q + 7, dim // 3] = np.nan
    x[q + 8] = 1.0
    x[q + 8, ::2] = -1.0
    return x


@pytest.mark.parametrize("dim,k,L,batch,srp", [(128, 9, 50, 4096, False), (100, 6, 7, 1500, False),
                                               (784, 6, 50, 2048, False), (128, 9, 50, 1024, True),
                                               (4096, 16, 8, 1100, False), (33, 24, 3, 1030, False)])
def test_hash_dense_matrix_core_path_bit_exact(kh, orc, dim, k, L, batch, srp):
    """Batches of >= 1024 rows hash on the matrix cores: a sign is taken from the
    MFMA sum only where it exceeds the error bound, every other (row, plane)
    replays the sequential sum.  Codes must equal the oracle's replay."""
    from klearu_amd.lsh import SimHash, SparseRandomProjection
    rng = np.random.default_rng(dim * 31 + k)
    fam = SparseRandomProjection(dim, k, L, 1.0 / 3.0, 7) if srp else SimHash(dim, k, L, 42)
    x = _hard_rows(rng, batch, dim)
    got = fam.hash_dense_batch(x).cpu().numpy().view(np.uint32)
    want = orc.hash_dense_batch(fam.planes(), x)
    np.testing.assert_array_equal(got, want)
    q = batch // 8
    assert np.all(got[q] == (1 << k) - 1) and np.all(got[q + 1] == (1 << k) - 1)


@pytest.mark.parametrize("dim,k,L,batch", [(784, 6, 50, 200), (2048, 9, 50, 40), (2049, 6, 50, 20),
                                           (1, 1, 256, 17), (33, 24, 50, 30), (100, 7, 37, 64),
                                           (257, 1, 3, 9), (512, 16, 256, 12)])
def test_hash_dense_lds_path_bit_exact(kh, orc, dim, k, L, batch):
    """Batches below 1024 rows with dim <= 2048 hash from LDS-staged 2-bit signs
    over the row's compacted nonzero values (2049 takes the per-plane kernel):
    group splits (k 24 -> 10 tables per block, k 1 -> 256), one-dimensional and
    odd widths, fully dense rows, the hard rows of the matrix-core test."""
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(dim * 7 + k)
    fam = SimHash(dim, k, L, 9)
    x = _hard_rows(rng, batch, dim) if batch >= 10 else rng.standard_normal((batch, dim)).astype(np.float32)
    x[-1] = rng.uniform(0.5, 1.0, dim).astype(np.float32)  # no zero value
    if batch > 12:
        x[-2] = cfg1_inputs(rng, 1, dim)[0]
    got = fam.hash_dense_batch(x).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, orc.hash_dense_batch(fam.planes(), x))


def test_hash_sparse_matches_dense(kh, orc):
    from klearu_amd.lsh import SparseVector, SimHash
    rng = np.random.default_rng(5)
    fam = SimHash(2000, 9, 50, 11)
    rows = sparse_rows(rng, 64, 2000, 40, empty_every=17)
    got = fam.hash_sparse_batch(rows).cpu().numpy().view(np.uint32)
    planes = fam.planes()
    for b, r in enumerate(rows):
        ref = [orc.hash_sparse(planes, r.indices, r.values, t) for t in range(50)]
        np.testing.assert_array_equal(got[b], np.array(ref, np.uint32))
        np.testing.assert_array_equal(got[b], orc.hash_dense_batch(planes, r.to_dense())[0])
    assert fam.hash_sparse(rows[3], 7) == int(got[3, 7])
    assert fam.hash_sparse(SparseVector([], [], 2000), 0) == (1 << 9) - 1


def test_family_from_planes_and_errors(kh, orc):
    from klearu_amd._lib import KlearuError
    from klearu_amd.lsh import HashFamily, SimHash
    p = orc.simhash_planes(40, 5, 4, 123)
    fam = HashFamily.from_planes(p)
    np.testing.assert_array_equal(fam.planes(), p)
    x = np.random.default_rng(0).standard_normal((7, 40)).astype(np.float32)
    np.testing.assert_array_equal(fam.hash_dense_batch(x).cpu().numpy().view(np.uint32),
                                  orc.hash_dense_batch(p, x))
    bad = p.copy()
    bad[0, 0, 0] = 2
    with pytest.raises(KlearuError):
        HashFamily.from_planes(bad)
    with pytest.raises(KlearuError):
        SimHash(10, 25, 2, 0)      # K > 24
    with pytest.raises(ValueError):
        fam.hash_dense(np.zeros(39, np.float32), 0)


# ----------------------------------------------------------------------------- index build
def build_pair(kh, orc, fam, bucket_type, cap, W, ids=None, chunks=1):
    from klearu_amd.lsh import LshIndex
    idx = LshIndex(fam, bucket_type, cap)
    ref = orc.LshIndex(fam.num_tables(), fam.k(), cap, bucket_type)
    n = W.shape[0]
    ids = np.arange(n, dtype=np.uint32) if ids is None else ids
    planes = fam.planes()
    for part in np.array_split(np.arange(n), chunks):
        idx.insert_batch(ids[part], W[part])
        ref.insert_many(ids[part], orc.hash_dense_batch(planes, W[part]))
    return idx, ref


def assert_buckets_equal(idx, ref):
    data, ln, cnt = idx.buckets()
    L, nb, cap = data.shape
    rl = ref.len.reshape(L, nb)
    np.testing.assert_array_equal(ln, rl)
    np.testing.assert_array_equal(cnt, ref.count.reshape(L, nb))
    rd = ref.data.reshape(L, nb, cap)
    mask = np.arange(cap)[None, None, :] < rl[:, :, None]
    np.testing.assert_array_equal(np.where(mask, data, 0), np.where(mask, rd, 0))


@pytest.mark.parametrize("chunks", [1, 3])
def test_fifo_index_cfg1_bit_exact(kh, orc, chunks):
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(1)
    fam = SimHash(784, 6, 50, 42 + 1_000_000)
    W = rng.normal(0, 0.01, (1024, 784)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, FIFO, 128, W, chunks=chunks)
    assert_buckets_equal(idx, ref)
    # a second pass over the same neurons overflows buckets: FIFO evicts the front
    idx.insert_batch(np.arange(1024, dtype=np.uint32)[::-1].copy(), W[::-1].copy())
    ref.insert_many(np.arange(1024, dtype=np.uint32)[::-1].copy(), orc.hash_dense_batch(fam.planes(), W[::-1]))
    assert_buckets_equal(idx, ref)


@pytest.mark.parametrize("n,k,L,cap,chunks", [(20000, 4, 8, 16, 1), (20000, 4, 8, 16, 4),
                                              (40000, 9, 50, 128, 2), (3000, 2, 3, 5, 7)])
def test_reservoir_index_bit_exact(kh, orc, n, k, L, cap, chunks):
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(n + k)
    fam = SimHash(128, k, L, 99)
    W = rng.normal(0, 0.01, (n, 128)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, RESERVOIR, cap, W, chunks=chunks)
    assert_buckets_equal(idx, ref)


def test_insert_codes_duplicates_and_clear(kh, orc):
    from klearu_amd.lsh import LshIndex, SimHash
    rng = np.random.default_rng(3)
    fam = SimHash(16, 3, 4, 5)
    for bt in (FIFO, RESERVOIR):
        idx = LshIndex(fam, bt, 6)
        ref = orc.LshIndex(4, 3, 6, bt)
        ids = rng.integers(0, 50, 400).astype(np.uint32)           # repeated ids
        codes = rng.integers(0, 8, (400, 4)).astype(np.uint32)
        idx.insert_codes(ids, codes)
        ref.insert_many(ids, codes)
        assert_buckets_equal(idx, ref)
        idx.clear()
        data, ln, cnt = idx.buckets()
        assert ln.sum() == 0 and cnt.sum() == 0
        idx.insert_codes(ids[:10], codes[:10])
        ref2 = orc.LshIndex(4, 3, 6, bt)
        ref2.insert_many(ids[:10], codes[:10])
        assert_buckets_equal(idx, ref2)


# ----------------------------------------------------------------------------- queries
def test_query_cfg1_bit_exact(kh, orc):
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(11)
    fam = SimHash(784, 6, 50, 42 + 1_000_000)
    W = rng.normal(0, 0.01, (1024, 784)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, FIFO, 128, W)
    X = cfg1_inputs(rng, 128)
    off, ids, cnt = idx.query_batch(X)
    off = off.cpu().numpy()
    ids = ids.cpu().numpy().view(np.uint32)
    cnt = cnt.cpu().numpy().view(np.uint32)
    codes = orc.hash_dense_batch(fam.planes(), X)
    for b in range(128):
        ri, rc = ref.query(codes[b])
        np.testing.assert_array_equal(ids[off[b]:off[b + 1]], ri)
        np.testing.assert_array_equal(cnt[off[b]:off[b + 1]], rc)
    # the per-vector mirror and union-only variant
    q = idx.query(X[5])
    ri, rc = ref.query(codes[5])
    assert [c.neuron_id for c in q] == ri.tolist() and [c.count for c in q] == rc.tolist()
    assert idx.query_union(X[5]) == ri.tolist()


def test_query_large_ids_sort_path(kh, orc):
    """Ids beyond the LDS counting range take the sort-based dedup path."""
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(12)
    fam = SimHash(128, 9, 50, 77)
    n = 30000
    W = rng.normal(0, 0.01, (n, 128)).astype(np.float32)
    ids = (np.arange(n, dtype=np.uint64) * 131 + 5).astype(np.uint32)   # sparse id space
    idx, ref = build_pair(kh, orc, fam, RESERVOIR, 128, W, ids=ids)
    X = rng.standard_normal((40, 128)).astype(np.float32)
    off, gi, gc = idx.query_batch(X)
    off = off.cpu().numpy()
    gi = gi.cpu().numpy().view(np.uint32)
    gc = gc.cpu().numpy().view(np.uint32)
    codes = orc.hash_dense_batch(fam.planes(), X)
    for b in range(40):
        ri, rc = ref.query(codes[b])
        np.testing.assert_array_equal(gi[off[b]:off[b + 1]], ri)
        np.testing.assert_array_equal(gc[off[b]:off[b + 1]], rc)


@pytest.mark.parametrize("max_id,path", [(924_000, "bitmap"), (924_700, "bitmap"),
                                          (925_000, "sort"), (670_090, "bitmap")])
def test_query_bitmap_limits(kh, orc, max_id, path):
    """Ids above 12288 are deduplicated with an LDS bitmap while its
    ceil(bound/32) * 9/8 words plus L*cap counts fit in 152 KB (L=50, cap=128:
    ids < 924_672), else by sorting.  Ids sit on both sides of that limit and
    in the bitmap's last word; unions are checked with and without counts."""
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(max_id % 1000)
    fam = SimHash(64, 9, 50, 31)
    n = 6000
    ids = np.sort(rng.choice(max_id, n - 1, replace=False)).astype(np.uint32)
    ids = np.append(ids, np.uint32(max_id))  # id_bound = max_id + 1
    W = rng.normal(0, 0.01, (n, 64)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, RESERVOIR, 128, W, ids=ids)
    words = (max_id + 1 + 31) // 32
    fits = 4 * (words + (words + 7) // 8 + 50 * 128) <= 152 * 1024
    assert fits == (path == "bitmap")
    X = np.concatenate([rng.standard_normal((12, 64)), W[-3:]]).astype(np.float32)
    codes = orc.hash_dense_batch(fam.planes(), X)
    off, gi, gc = idx.query_batch(X)
    off2, gi2, _ = idx.query_batch(X, counts=False)
    off, off2 = off.cpu().numpy(), off2.cpu().numpy()
    gi, gi2 = gi.cpu().numpy().view(np.uint32), gi2.cpu().numpy().view(np.uint32)
    gc = gc.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(off, off2)
    for b in range(X.shape[0]):
        ri, rc = ref.query(codes[b])
        np.testing.assert_array_equal(gi[off[b]:off[b + 1]], ri)
        np.testing.assert_array_equal(gc[off[b]:off[b + 1]], rc)
        np.testing.assert_array_equal(gi2[off[b]:off[b + 1]], ri)
    # the rows that hash like the last inserted vector find the largest id
    assert np.uint32(max_id) in gi[off[-2]:off[-1]]


@pytest.mark.parametrize("L,k,n", [(100, 4, 3000), (256, 3, 600), (200, 7, 20000)])
def test_query_many_tables(kh, orc, L, k, n):
    """More than 64 tables (up to the 256 an index may hold): dense hashing
    with one plane per thread over more than 256 planes, and both query paths
    (LDS counting below 12288 ids, sort-based dedup above)."""
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(L + k)
    fam = SimHash(96, k, L, 5 + L)
    W = rng.normal(0, 0.01, (n, 96)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, FIFO, 16, W)
    assert_buckets_equal(idx, ref)
    X = rng.standard_normal((9, 96)).astype(np.float32)
    np.testing.assert_array_equal(fam.hash_dense_batch(X).cpu().numpy().view(np.uint32),
                                  orc.hash_dense_batch(fam.planes(), X))
    off, gi, gc = idx.query_batch(X)
    off = off.cpu().numpy()
    gi = gi.cpu().numpy().view(np.uint32)
    gc = gc.cpu().numpy().view(np.uint32)
    codes = orc.hash_dense_batch(fam.planes(), X)
    for b in range(9):
        ri, rc = ref.query(codes[b])
        np.testing.assert_array_equal(gi[off[b]:off[b + 1]], ri)
        np.testing.assert_array_equal(gc[off[b]:off[b + 1]], rc)


def test_query_sparse_and_capacity(kh, orc):
    from klearu_amd._lib import KlearuError
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(13)
    fam = SimHash(500, 5, 12, 8)
    W = rng.normal(0, 0.01, (700, 500)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, FIFO, 32, W)
    rows = sparse_rows(rng, 20, 500, 30, empty_every=7)
    off, gi, gc = idx.query_sparse_batch(rows)
    off = off.cpu().numpy()
    gi = gi.cpu().numpy().view(np.uint32)
    gc = gc.cpu().numpy().view(np.uint32)
    for b, r in enumerate(rows):
        ri, rc = ref.query(orc.hash_dense_batch(fam.planes(), r.to_dense())[0])
        np.testing.assert_array_equal(gi[off[b]:off[b + 1]], ri)
        np.testing.assert_array_equal(gc[off[b]:off[b + 1]], rc)
    with pytest.raises(KlearuError):
        idx.query_sparse_batch(rows, capacity=3)


def test_empty_index_query(kh, orc):
    from klearu_amd.lsh import LshIndex, SimHash
    fam = SimHash(20, 4, 6, 1)
    idx = LshIndex(fam, FIFO, 8)
    off, ids, cnt = idx.query_batch(np.ones((3, 20), np.float32))
    assert off.cpu().numpy().tolist() == [0, 0, 0, 0]
    assert idx.query(np.ones(20, np.float32)) == []


# ----------------------------------------------------------------------------- SLIDE layer
def slide_pair(kh, orc, dim, n, k, L, cap, bt, sampling, top_k, thr, act, rng, seed=42):
    from klearu_amd.lsh import LshConfig
    from klearu_amd.slide import Layer, LayerConfig
    lsh = LshConfig(num_tables=L, num_hashes=k, bucket_capacity=cap,
                    bucket_type="Fifo" if bt == FIFO else "Reservoir")
    cfg = LayerConfig(dim, n, act, lsh, sampling, thr, top_k)
    W = rng.normal(0, 0.01, (n, dim)).astype(np.float32)
    b = rng.normal(0, 0.01, n).astype(np.float32) if act != "Relu" else np.zeros(n, np.float32)
    layer = Layer(cfg, W, b, seed)
    planes = layer.index.hash_family.planes()
    np.testing.assert_array_equal(planes, orc.simhash_planes(dim, k, L, seed + 1_000_000))
    return layer, planes, W, b


SAMP = {"Vanilla": 0, "TopK": 1, "Threshold": 2}
ACTS = {"Relu": "relu", "Sigmoid": "sigmoid", "Tanh": "tanh", "Softmax": "softmax", "Identity": "identity"}


def check_slide(orc, layer, planes, W, b, X, got, exact_act):
    cfg = layer.config
    ref, _ = orc.slide_layer_oracle(planes, cfg.lsh.bucket_capacity,
                                    FIFO if cfg.lsh.bucket_type == "Fifo" else RESERVOIR, W, b, X,
                                    SAMP[cfg.sampling], cfg.top_k, cfg.sampling_threshold,
                                    ACTS[cfg.activation])
    off, ids, pre, act = (t.cpu().numpy() for t in got)
    ids = ids.view(np.uint32)
    for r, (ri, rp, ra) in enumerate(ref):
        s = slice(off[r], off[r + 1])
        np.testing.assert_array_equal(ids[s], ri)
        np.testing.assert_array_equal(pre[s], rp)
        if exact_act:
            np.testing.assert_array_equal(act[s], ra)
        else:
            np.testing.assert_allclose(act[s], ra, rtol=1e-5, atol=1e-7)
    return ref


def test_slide_cfg1_vanilla_relu(kh, orc):
    """cfg1 exactly: 1024x784 N(0,0.01), bias 0, batch 128, 80% zeros, K6 L50 FIFO 128, seed 42."""
    rng = np.random.default_rng(42)
    layer, planes, W, b = slide_pair(kh, orc, 784, 1024, 6, 50, 128, FIFO, "Vanilla", 0, 2, "Relu", rng)
    X = cfg1_inputs(rng, 128)
    ref = check_slide(orc, layer, planes, W, b, X, layer.forward_batch(X), True)
    assert np.mean([len(r[0]) for r in ref]) > 10
    out = layer.forward(X[3])
    dense = np.zeros(1024, np.float32)
    dense[ref[3][0]] = ref[3][2]
    np.testing.assert_array_equal(out.activations, dense)
    np.testing.assert_array_equal(out.active_neurons, ref[3][0])


@pytest.mark.parametrize("sampling,top_k,thr,act", [
    ("TopK", 102, 2, "Relu"), ("TopK", 5, 2, "Sigmoid"), ("Threshold", 2, 2, "Relu"),
    ("Threshold", 1000, 1000, "Identity"),   # nobody passes -> single best candidate
    ("TopK", 0, 2, "Relu"),                  # take(0) -> empty -> every neuron
    ("Vanilla", 0, 2, "Tanh"), ("TopK", 300, 2, "Softmax")])
def test_slide_sampling_modes(kh, orc, sampling, top_k, thr, act):
    rng = np.random.default_rng(top_k + thr)
    layer, planes, W, b = slide_pair(kh, orc, 784, 1024, 6, 50, 128, FIFO, sampling, top_k, thr, act, rng)
    X = cfg1_inputs(rng, 48)
    check_slide(orc, layer, planes, W, b, X, layer.forward_batch(X), act in ("Relu", "Sigmoid", "Identity"))


def test_slide_empty_index_falls_back_to_all(kh, orc):
    rng = np.random.default_rng(4)
    layer, planes, W, b = slide_pair(kh, orc, 64, 300, 8, 4, 16, FIFO, "Vanilla", 0, 2, "Relu", rng)
    layer.index.clear()
    X = rng.standard_normal((5, 64)).astype(np.float32)
    off, ids, pre, act = (t.cpu().numpy() for t in layer.forward_batch(X))
    for r in range(5):
        s = slice(off[r], off[r + 1])
        np.testing.assert_array_equal(ids[s], np.arange(300))
        ref = np.array([orc.neuron_forward(W[i], b[i], X[r]) for i in range(300)], np.float32)
        np.testing.assert_array_equal(pre[s], ref)


def test_slide_sparse_input_matches_dense(kh, orc):
    from klearu_amd.lsh import SparseVector
    rng = np.random.default_rng(8)
    layer, planes, W, b = slide_pair(kh, orc, 784, 1024, 6, 50, 128, FIFO, "Vanilla", 0, 2, "Relu", rng)
    X = cfg1_inputs(rng, 32)
    rows = [SparseVector.from_dense(x) for x in X]
    dense = [t.cpu().numpy() for t in layer.forward_batch(X)]
    sparse = [t.cpu().numpy() for t in layer.forward_sparse_batch(rows)]
    np.testing.assert_array_equal(dense[0], sparse[0])
    total = int(dense[0][-1])
    for a, c in zip(dense[1:], sparse[1:]):
        np.testing.assert_array_equal(a[:total], c[:total])


def test_dense_layer_sparse_inputs(kh, orc):
    from klearu_amd.slide import DenseLayer
    rng = np.random.default_rng(9)
    W = rng.normal(0, 0.01, (128, 5000)).astype(np.float32)
    b = rng.normal(0, 0.01, 128).astype(np.float32)
    rows = sparse_rows(rng, 33, 5000, 75, empty_every=11)
    y = DenseLayer(W, b, "Relu").forward_sparse(rows).cpu().numpy()
    for r, v in enumerate(rows):
        pre = np.array([orc.neuron_forward_sparse(W[o], b[o], v.indices, v.values) for o in range(128)],
                       np.float32)
        np.testing.assert_array_equal(y[r], np.maximum(pre, 0))


def test_xc_network_scaled_cfg5(kh, orc):
    """cfg5 at reduced width: sparse 20000-d inputs (~75 nnz) -> DenseLayer 128 ReLU ->
    SLIDE softmax output layer (K9 L50 reservoir cap 128) over 60000 labels."""
    from klearu_amd.lsh import LshConfig
    from klearu_amd.slide import DenseLayer, Layer, LayerConfig
    rng = np.random.default_rng(2024)
    W1 = rng.normal(0, 0.01, (128, 20000)).astype(np.float32)
    b1 = np.zeros(128, np.float32)
    hidden = DenseLayer(W1, b1, "Relu")
    n = 60000
    W2 = rng.normal(0, 0.01, (n, 128)).astype(np.float32)
    b2 = np.zeros(n, np.float32)
    cfg = LayerConfig(128, n, "Softmax", LshConfig(num_tables=50, num_hashes=9, bucket_capacity=128,
                                                   bucket_type="Reservoir"), "Vanilla", 2, 0, True)
    out = Layer(cfg, W2, b2, 7)
    rows = sparse_rows(rng, 24, 20000, 75)
    h = hidden.forward_sparse(rows)
    got = out.forward_batch(h)
    hh = h.cpu().numpy()
    ref = check_slide(orc, out, out.index.hash_family.planes(), W2, b2, hh, got, False)
    sizes = [len(r[0]) for r in ref]
    assert min(sizes) > 100
    act = got[3].cpu().numpy()
    o = got[0].cpu().numpy()
    for r in range(24):
        assert abs(act[o[r]:o[r + 1]].astype(np.float64).sum() - 1.0) < 1e-4


# ----------------------------------------------------------------------------- mutators
@pytest.mark.parametrize("bt", [FIFO, RESERVOIR])
def test_remove_and_reinsert_bit_exact(kh, orc, bt):
    """insert -> remove_with_weights -> insert -> remove (every bucket) ->
    insert_sparse, each against the oracle's replay of the reference's bucket
    rules (swap_remove, counts kept, refills after removal): buckets, lengths
    and insertion counts bit-exact.  The removal lists hold repeated ids and
    ids that were never inserted."""
    from klearu_amd.lsh import LshIndex, SimHash, SparseVector
    rng = np.random.default_rng(5 + bt)
    dim, k, L, cap = 64, 4, 8, 12
    fam = SimHash(dim, k, L, 17)
    planes = fam.planes()
    idx = LshIndex(fam, bt, cap)
    ref = orc.LshIndex(L, k, cap, bt)
    W = rng.normal(0, 0.01, (600, dim)).astype(np.float32)
    ids = np.arange(600, dtype=np.uint32)
    idx.insert_batch(ids[:400], W[:400])
    ref.insert_many(ids[:400], orc.hash_dense_batch(planes, W[:400]))
    gone = np.concatenate([rng.choice(400, 80, replace=False), [5, 5, 599, 450]]).astype(np.uint32)
    idx.remove_with_weights_batch(gone, W[gone])
    ref.remove_many(gone, orc.hash_dense_batch(planes, W[gone]))
    assert_buckets_equal(idx, ref)
    idx.insert_batch(ids[400:], W[400:])
    ref.insert_many(ids[400:], orc.hash_dense_batch(planes, W[400:]))
    all_gone = np.concatenate([rng.choice(600, 50, replace=False), [7, 7, 12345]]).astype(np.uint32)
    idx.remove_batch(all_gone)
    ref.remove_all(all_gone)
    assert_buckets_equal(idx, ref)
    rows = [SparseVector(np.sort(rng.choice(dim, 9, replace=False)).astype(np.uint32),
                         rng.normal(0, 1, 9).astype(np.float32), dim) for _ in range(40)]
    sids = np.arange(1000, 1040, dtype=np.uint32)
    idx.insert_sparse_batch(sids, rows)
    dense = np.zeros((40, dim), np.float32)
    for i, r in enumerate(rows):
        dense[i, r.indices] = r.values
    ref.insert_many(sids, orc.hash_dense_batch(planes, dense))
    assert_buckets_equal(idx, ref)


def test_index_rejects_ids_at_or_above_2_31(kh, orc):
    """Ids must be below 2^31 (id + 1 bounds and bitmap sizes cannot wrap);
    such an insert is refused before anything changes."""
    from klearu_amd import KlearuError
    from klearu_amd._lib import KH_ERR_ARG
    from klearu_amd.lsh import LshIndex, SimHash
    fam = SimHash(16, 3, 4, 5)
    idx = LshIndex(fam, FIFO, 6)
    codes = np.zeros((3, 4), np.uint32)
    for bad in (0x80000000, 0xFFFFFFFF):
        with pytest.raises(KlearuError) as e:
            idx.insert_codes(np.array([1, bad, 2], np.uint32), codes)
        assert e.value.code == KH_ERR_ARG
    _, ln, cnt = idx.buckets()
    assert ln.sum() == 0 and cnt.sum() == 0


def test_concurrent_queries_two_streams_two_threads(kh, orc):
    """The reference's LshIndex is Send + Sync and query takes &self: two host
    threads, each on its own stream, query one index (and one SLIDE layer)
    many times while the other does; every result matches the oracle."""
    import threading
    from klearu_amd.lsh import SimHash
    rng = np.random.default_rng(23)
    fam = SimHash(784, 6, 50, 42 + 1_000_000)
    W = rng.normal(0, 0.01, (1024, 784)).astype(np.float32)
    idx, ref = build_pair(kh, orc, fam, FIFO, 128, W)
    X = [cfg1_inputs(rng, 32) for _ in range(2)]
    codes = [orc.hash_dense_batch(fam.planes(), x) for x in X]
    want = [[ref.query(c[b]) for b in range(32)] for c in codes]
    errors = []

    def worker(t):
        try:
            s = torch.cuda.Stream()
            xd = torch.from_numpy(X[t]).cuda()
            for _ in range(20):
                with torch.cuda.stream(s):
                    off, ids, cnt = idx.query_batch(xd, stream=s)
                s.synchronize()
                o = off.cpu().numpy()
                i = ids.cpu().numpy().view(np.uint32)
                c = cnt.cpu().numpy().view(np.uint32)
                for b in range(32):
                    if not (np.array_equal(i[o[b]:o[b + 1]], want[t][b][0]) and
                            np.array_equal(c[o[b]:o[b + 1]], want[t][b][1])):
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


def test_xc_network_full_cfg5(kh, orc):
    """cfg5 at its BASELINE size: sparse 135909-d inputs (50-100 nnz, U[0,1]) ->
    DenseLayer 128 ReLU -> SLIDE softmax output layer of 670091 neurons
    (N(0, 0.01) weights, SimHash K9 L50, reservoir cap 128), batch 256.
      - hash codes of a random sample of 4096 neurons are bit-exact against the
        oracle's hash_dense (simhash.rs:103-114);
      - every bucket (contents, lengths, insertion counts) is bit-exact against
        the oracle's insert replay (reservoir.rs:50-67, neurons 0..n-1 in order)
        from the GPU's codes of all 670091 neurons;
      - for 16 of the 256 samples: hidden activations, active sets and
        pre-activations bit-exact, softmax within 1e-5, against
        Layer::forward (layer.rs:65-120) on the oracle's index.
    |A| is reported: with untrained N(0, 0.01) weights every bucket is full
    (670091 / 512 = 1309 inserts per bucket) and the 50 buckets of a query
    rarely share a neuron, so |A| is close to 50 x 128 = 6400."""
    from klearu_amd.lsh import LshConfig, SparseVector
    from klearu_amd.slide import DenseLayer, Layer, LayerConfig
    D_in, Hd, n, B, L, K, cap = 135909, 128, 670091, 256, 50, 9, 128
    rng = np.random.default_rng(670091)
    W1 = rng.normal(0, 0.01, (Hd, D_in)).astype(np.float32)
    b1 = np.zeros(Hd, np.float32)
    W2 = rng.normal(0, 0.01, (n, Hd)).astype(np.float32)
    b2 = np.zeros(n, np.float32)
    hidden = DenseLayer(W1, b1, "Relu")
    cfg = LayerConfig(Hd, n, "Softmax", LshConfig(num_tables=L, num_hashes=K, bucket_capacity=cap,
                                                  bucket_type="Reservoir"), "Vanilla", 2, 0, True)
    out = Layer(cfg, W2, b2, 42)
    fam = out.index.hash_family
    planes = fam.planes()
    # 1. codes of every neuron on the GPU; a sample against the oracle
    codes = fam.hash_dense_batch(torch.from_numpy(W2).cuda()).cpu().numpy().view(np.uint32).reshape(n, L)
    sample = np.sort(rng.choice(n, 4096, replace=False))
    np.testing.assert_array_equal(codes[sample], orc.hash_dense_batch(planes, W2[sample]))
    # 2. buckets against the oracle's replay of the inserts from those codes
    ref = orc.LshIndex(L, K, cap, RESERVOIR)
    ref.insert_many(np.arange(n, dtype=np.uint32), codes)
    assert_buckets_equal(out.index, ref)
    # 3. the network on 256 samples; 16 checked against the oracle
    rows = []
    for _ in range(B):
        nnz = int(rng.integers(50, 101))
        idx = np.sort(rng.choice(D_in, nnz, replace=False)).astype(np.uint32)
        rows.append(SparseVector(idx, rng.uniform(0, 1, nnz).astype(np.float32), D_in))
    h = hidden.forward_sparse(rows)
    got = out.forward_batch(h)
    hh = h.cpu().numpy()
    off = got[0].cpu().numpy()
    A = np.diff(off)
    print(f"|A| mean {A.mean():.0f} min {A.min()} max {A.max()} (config: ~2-4k with trained weights)")
    pick = np.sort(rng.choice(B, 16, replace=False))
    for r in pick:
        pre_h = np.array([orc.neuron_forward_sparse(W1[o], b1[o], rows[r].indices, rows[r].values)
                          for o in range(Hd)], np.float32)
        want_h = orc.layer_activate(pre_h, "relu")
        np.testing.assert_array_equal(hh[r], want_h)
    refrows, _ = orc.slide_layer_oracle(planes, cap, RESERVOIR, W2, b2, hh[pick], 0, 0, 2, "softmax", index=ref)
    ids = got[1].cpu().numpy().view(np.uint32)
    pre = got[2].cpu().numpy()
    act = got[3].cpu().numpy()
    for j, r in enumerate(pick):
        s = slice(off[r], off[r + 1])
        ri, rp, ra = refrows[j]
        np.testing.assert_array_equal(ids[s], ri)
        np.testing.assert_array_equal(pre[s], rp)
        np.testing.assert_allclose(act[s], ra, rtol=1e-5, atol=1e-9)
