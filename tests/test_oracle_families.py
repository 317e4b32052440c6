"""Pins for the oracle's WTA / DWTA / MinHash restatement (CPU only).

The window and permutation draws come from rand 0.8.5 (a dependency absent
from the reference tree): its gen_range / shuffle steps are pinned here by
closed forms on the oracle's own ChaCha stream, and the composed draws stay
parity unpinned.  The hash functions are pinned by brute force, the
reference's own tests (hash/wta.rs:154-215, dwta.rs, minhash.rs) and the
SipHash paper's vectors for the fallback hasher's round function.
"""
import math

import numpy as np
import pytest

import oracle as orc

F = np.float32
KEY = (0x0706050403020100, 0x0F0E0D0C0B0A0908)


def test_siphash_round_function_reference_vectors():
    # SipHash-2-4, key 00..0f, message 00..(n-1) (Aumasson & Bernstein, reference vectors)
    assert orc.siphash(2, 4, *KEY, bytes(range(15))) == 0xA129CA6149BE45E5
    assert orc.siphash(2, 4, *KEY, b"") == 0x726FDB47DD0E0E31
    assert orc.siphash(2, 4, *KEY, bytes([0])) == 0x74F839C593DC67FD
    assert orc.siphash(2, 4, *KEY, bytes([0, 1])) == 0x0D6C8009D9A94F5A


def test_dwta_fallback_is_siphash13_of_two_words():
    for t, f, ws in [(0, 0, 8), (3, 5, 8), (49, 8, 7), (1 << 40, 2, 5)]:
        msg = t.to_bytes(8, "little") + f.to_bytes(8, "little")
        assert orc.lib.or_dwta_fallback(t, f, ws) == orc.siphash(1, 3, 0, 0, msg) % ws


def test_gen_range_closed_forms():
    """(draw * n) >> 32 of the first draw whose low word is <= zone, zone =
    (n << lzcnt(n)) - 1: for n = 2^s that is 2^31 - 1, so half the draws are
    rejected even for powers of two (rand's conservative zone)."""
    for n in (2, 6, 8, 1000, 12345, (1 << 31) + 5):
        zone = ((n << (32 - n.bit_length())) - 1) & 0xFFFFFFFF
        a, b = orc.StdRng(3 + n), orc.StdRng(3 + n)
        for _ in range(200):
            while True:
                m = b.next_u32() * n
                if (m & 0xFFFFFFFF) <= zone:
                    want = m >> 32
                    break
            assert a.gen_range(n) == want < n


def test_shuffle_is_fisher_yates_from_the_end():
    # two elements: one draw j = gen_range(2); swap(1, j)
    a, b = orc.StdRng(11), orc.StdRng(11)
    for _ in range(20):
        j = b.gen_range(2)
        got = a.shuffle([0, 1]).tolist()
        assert got == ([1, 0] if j == 0 else [0, 1])
    # three elements: j1 = gen_range(3) swaps with 2, then j2 = gen_range(2) with 1
    a, b = orc.StdRng(12), orc.StdRng(12)
    for _ in range(20):
        v = [0, 1, 2]
        j1 = b.gen_range(3)
        v[2], v[j1] = v[j1], v[2]
        j2 = b.gen_range(2)
        v[1], v[j2] = v[j2], v[1]
        assert a.shuffle([0, 1, 2]).tolist() == v
    # a permutation, reproducible from the seed
    p = orc.StdRng(5).shuffle(np.arange(1000))
    assert sorted(p.tolist()) == list(range(1000))
    assert np.array_equal(p, orc.StdRng(5).shuffle(np.arange(1000)))


def test_windows_and_permutations_shapes():
    w = orc.wta_windows(50, 4, 3, 8, 42)
    assert w.shape == (3, 4, 8)
    for t in range(3):
        for f in range(4):
            assert len(set(w[t, f].tolist())) == 8 and w[t, f].max() < 50
    p = orc.minhash_perms(30, 4, 9)
    for t in range(4):
        assert sorted(p[t].tolist()) == list(range(30))


def _brute_wta(windows, x, table):
    L, k, ws = windows.shape
    bits = 1 if ws <= 1 else math.ceil(math.log2(ws))
    h = 0
    for f in range(k):
        best, bv = 0, -math.inf
        for p, d in enumerate(windows[table, f]):
            if x[d] > bv:          # NaN compares false: never wins
                best, bv = p, x[d]
        h |= best << (bits * f)
    return h


def test_wta_hash_brute_force_ties_nan_inf():
    rng = np.random.default_rng(0)
    w = orc.wta_windows(40, 5, 4, 8, 1)
    for trial in range(50):
        x = rng.integers(-3, 3, 40).astype(F)        # many ties
        if trial % 5 == 0:
            x[rng.integers(0, 40, 6)] = np.nan
        if trial % 7 == 0:
            x[:] = -np.inf
        for t in range(4):
            assert orc.wta_hash_dense(w, x, t) == _brute_wta(w, x, t)
    # bits per window: ceil(log2(ws)); ws 5 -> 3 bits, ws 1 -> 1 bit
    assert [orc.lib.or_wta_bits(v) for v in (1, 2, 5, 8, 9)] == [1, 1, 3, 3, 4]


def test_wta_invariant_to_positive_scaling():
    """hash/wta.rs:202-215: argmax positions do not change under x -> c x, c > 0."""
    rng = np.random.default_rng(2)
    w = orc.wta_windows(64, 4, 3, 8, 42)
    x = rng.uniform(-1, 1, 64).astype(F)
    for c in (0.5, 3.0, 1e3):
        for t in range(3):
            assert orc.wta_hash_dense(w, x, t) == orc.wta_hash_dense(w, (x * F(c)).astype(F), t)


def test_dwta_sparse_rules():
    w = orc.wta_windows(64, 4, 3, 8, 42)
    rng = np.random.default_rng(4)
    x = rng.uniform(-1, 1, 64).astype(F)
    idx = np.arange(64, dtype=np.uint32)
    for t in range(3):   # every dimension stored: the dense argmax
        assert orc.dwta_hash_sparse(w, idx, x, t) == orc.wta_hash_dense(w, x, t)
    # nothing stored: every window takes its fallback
    for t in range(3):
        want = sum(orc.lib.or_dwta_fallback(t, f, 8) << (3 * f) for f in range(4))
        assert orc.dwta_hash_sparse(w, [], [], t) == want
    # a stored negative value still beats an absent dimension (absent != 0)
    win = w[0, 0]
    idx1 = np.array(sorted([int(win[5])]), np.uint32)
    h = orc.dwta_hash_sparse(w, idx1, np.array([-7.0], F), 0)
    assert h & 7 == 5


def test_minhash_closed_form():
    P = 0x517CC1B727220A95
    perms = np.arange(8, dtype=np.uint32)[None, :]          # identity, dim 8
    k = 4                                                    # bin size 2
    # nonzero dims {1, 4, 5}: bins [1, -, 4, -] -> densified [1, 4, 4, 1]
    h = orc.minhash_hash(perms, k, 0, [1, 4, 5])
    want = (1 + 4 * P + 4 * P * P + 1 * P ** 3) % (1 << 64) & ((1 << k) - 1)
    assert h == want
    assert orc.minhash_hash(perms, k, 0, []) == 0            # all empty -> zeros
    # dense form takes x != 0 (a stored -0.0 is zero); sparse takes every stored index
    x = np.zeros(8, F)
    x[[1, 4, 5]] = [1.0, -2.0, 3.0]
    x[6] = -0.0
    assert orc.minhash_hash_dense(perms, k, 0, x) == h
    # dim not divisible by k: bin size ceil(10/4) = 3, bins 0..3 cover 0..11
    p10 = np.arange(10, dtype=np.uint32)[None, :]
    h = orc.minhash_hash(p10, 4, 0, [9])
    want = (9 + 9 * P + 9 * P * P + 9 * P ** 3) % (1 << 64) & 15
    assert h == want


def test_cpu_baseline_drivers_match_the_pinned_functions():
    """bench.py's CPU legs time one batch call each (or_cpu_rank_hash_batch,
    or_cpu_bolt_batch, or_cpu_lsh_topk_batch); each must compute exactly what
    the pinned per-row functions give: WTA / MinHash codes, bolt's top
    candidates by (count desc, id asc) with dot + bias + ReLU and no fallback
    (sparse_inference.rs:36-74), and the LSH predictor's top ids
    (lsh_predictor.rs:15-43)."""
    rng = np.random.default_rng(21)
    dim, k, L, ws, B = 96, 4, 7, 8, 9
    X = (rng.uniform(0, 1, (B, dim)) * (rng.random((B, dim)) < 0.4)).astype(F)
    X[0] = 0.0
    win = orc.wta_windows(dim, k, L, ws, 3)
    got = np.zeros(B * L, np.uint64)
    orc.lib.or_cpu_rank_hash_batch(0, np.ascontiguousarray(win, np.uint32).reshape(-1), dim, k, ws, L, X, B, got)
    want = [orc.wta_hash_dense(win, x, t) for x in X for t in range(L)]
    np.testing.assert_array_equal(got, np.array(want, np.uint64))
    perms = orc.minhash_perms(dim, L, 4)
    orc.lib.or_cpu_rank_hash_batch(2, np.ascontiguousarray(perms, np.uint32).reshape(-1), dim, k, 0, L, X, B, got)
    want = [orc.minhash_hash_dense(perms, k, t, x) for x in X for t in range(L)]
    np.testing.assert_array_equal(got, np.array(want, np.uint64))
    # a FIFO index over n neurons, then bolt and the predictor's top ids
    n, cap, topk = 120, 16, 11
    planes = orc.simhash_planes(dim, k, L, 5)
    W = rng.normal(0, 0.1, (n, dim)).astype(F)
    bias = rng.normal(0, 0.1, n).astype(F)
    idx = orc.LshIndex(L, k, cap, orc.FIFO)
    idx.insert_many(np.arange(n, dtype=np.uint32), orc.hash_dense_batch(planes, W).reshape(-1))
    pl = np.ascontiguousarray(planes, np.int8).reshape(-1)
    n_out = np.zeros(B, np.int64)
    act = np.zeros(B * topk, F)
    tot = orc.lib.or_cpu_bolt_batch(pl, dim, k, L, cap, idx.data, idx.len, W.reshape(-1), bias, X, B, topk, 1,
                                    n_out, act)
    ids = np.zeros(B * topk, np.uint32)
    n_ids = np.zeros(B, np.int64)
    orc.lib.or_cpu_lsh_topk_batch(pl, dim, k, L, cap, idx.data, idx.len, X, B, topk, n_ids, ids)
    pos = 0
    for r, x in enumerate(X):
        rid, rc = idx.query(orc.hash_dense_batch(planes, x[None]))
        sel = [i for i, _ in sorted(zip(rid.tolist(), rc.tolist()), key=lambda t: (-t[1], t[0]))[:topk]]
        assert n_out[r] == len(sel) and n_ids[r] == len(sel)
        assert ids[r * topk: r * topk + len(sel)].tolist() == sel
        for j, i in enumerate(sel):
            z = orc.neuron_forward(W[i], bias[i], x)
            assert act[pos + j] == F(max(z, 0.0))
        pos += len(sel)
    assert tot == pos
    assert b"clang" in orc.lib.or_compiler_version() or b"." in orc.lib.or_compiler_version()
