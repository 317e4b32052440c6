"""Pins the oracle's StdRng restatement and SimHash/SRP hashing (CPU only).

rand 0.8.5 / rand_chacha 0.3.1 / rand_core 0.6.4 are third-party crates absent
from the reference tree (no Rust toolchain here).  What is pinned:
  * the ChaCha block function, by RFC 7539 test vectors (20 rounds; the 12-round
    StdRng uses the same code with a different round count);
  * the PCG32 XSH-RR output function and LCG multiplier, by the PCG reference
    demo vector (pcg32_srandom_r(42, 54));
  * the ternary distribution test of crates/klearu-core/src/hash/simhash.rs:191-215.
The composed seed -> hyperplane stream stays "parity unpinned": no reference test
holds a drawn value.

Hashing is pinned by simhash.rs:232-240 (zero vector -> all ones), dense == sparse
(simhash.rs:173, :218; srp.rs:241-273) and an exact-arithmetic closed form.
"""
import numpy as np


def _words(hexstr):
    return np.array([int(w, 16) for w in hexstr.split()], np.uint32)


def test_chacha20_rfc7539_block(orc):
    # RFC 7539 section 2.3.2: key 00..1f, counter 1, nonce 00000009 0000004a 00000000
    inp = _words("61707865 3320646e 79622d32 6b206574 03020100 07060504 0b0a0908 0f0e0d0c "
                 "13121110 17161514 1b1a1918 1f1e1d1c 00000001 09000000 4a000000 00000000")
    exp = _words("e4e7f110 15593bd1 1fdd0f50 c47120a3 c7f4d1c7 0368c033 9aaa2204 4e6cd4c3 "
                 "466482d2 09aa9f07 05d7c214 a2028bd9 d19c12b5 b94e16de e883d0cb 4e3c50a2")
    np.testing.assert_array_equal(orc.chacha_block(inp, 20), exp)


def test_chacha20_zero_key_keystream(orc):
    # RFC 7539 appendix A.1 test vector #1 (all-zero key, nonce and counter).
    inp = np.zeros(16, np.uint32)
    inp[:4] = [0x61707865, 0x3320646e, 0x79622d32, 0x6b206574]
    exp = _words("ade0b876 903df1a0 e56a5d40 28bd8653 b819d2bd 1aed8da0 ccef36a8 c70d778b "
                 "7c5941da 8d485751 3fe02477 374ad8b8 f4b8436a 1ca11815 69b687c3 8665eeb2")
    np.testing.assert_array_equal(orc.chacha_block(inp, 20), exp)


def test_pcg32_demo_vector(orc):
    mult = 6364136223846793005
    mask = (1 << 64) - 1
    inc = (54 << 1) | 1
    state = 0
    state = (state * mult + inc) & mask
    state = (state + 42) & mask
    state = (state * mult + inc) & mask
    out = []
    for _ in range(6):
        old = state
        state = (old * mult + inc) & mask
        out.append(int(orc.lib.or_pcg32_output(old)))
    assert out == [0xa15c02b7, 0x7b47f409, 0xba1d3330, 0x83d2f293, 0xbfa4784b, 0xcbed606e]


def test_ternary_distribution(orc):
    # simhash.rs:191-215: StdRng::seed_from_u64(0), 60000 draws, within 0.02.
    p = orc.simhash_planes(60000, 1, 1, 0).ravel()
    for v, frac in ((-1, 1 / 6), (0, 2 / 3), (1, 1 / 6)):
        assert abs(np.mean(p == v) - frac) < 0.02


def test_f64_draws_uniform(orc):
    import ctypes

    r = orc.lib
    st = (ctypes.c_uint8 * 512)()
    r.or_stdrng_seed_from_u64.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
    r.or_stdrng_gen_f64.argtypes = [ctypes.c_void_p]
    r.or_stdrng_gen_f64.restype = ctypes.c_double
    r.or_stdrng_seed_from_u64(ctypes.addressof(st), 42)
    v = np.array([r.or_stdrng_gen_f64(ctypes.addressof(st)) for _ in range(20000)])
    assert v.min() >= 0.0 and v.max() < 1.0
    assert abs(v.mean() - 0.5) < 0.01 and abs(v.var() - 1 / 12) < 0.005


def test_srp_density(orc):
    # srp.rs:241 sparsity 0 -> all zero planes (hash all ones); :252 sparsity 1 -> no zeros
    assert np.all(orc.srp_planes(64, 4, 3, 0.0, 7) == 0)
    assert np.all(orc.srp_planes(64, 4, 3, 1.0, 7) != 0)
    p = orc.srp_planes(3000, 2, 2, 1.0 / 3.0, 9)
    assert abs(np.mean(p != 0) - 1 / 3) < 0.02


def test_zero_vector_hashes_to_all_ones(orc):
    planes = orc.simhash_planes(128, 8, 4, 42)
    for t in range(4):
        assert orc.hash_dense(planes, np.zeros(128, np.float32), t) == (1 << 8) - 1
    srp0 = orc.srp_planes(128, 8, 4, 0.0, 42)
    x = np.random.default_rng(0).uniform(-1, 1, 128).astype(np.float32)
    for t in range(4):
        assert orc.hash_dense(srp0, x, t) == (1 << 8) - 1


def test_dense_equals_sparse(orc):
    rng = np.random.default_rng(11)
    planes = orc.simhash_planes(128, 8, 4, 42)
    for trial in range(20):
        x = rng.uniform(-1, 1, 128).astype(np.float32)
        x[rng.random(128) < 0.7] = 0.0
        idx = np.nonzero(x)[0].astype(np.uint32)
        for t in range(4):
            assert orc.hash_dense(planes, x, t) == orc.hash_sparse(planes, idx, x[idx], t)


def test_hash_bits_exact_on_integers(orc):
    # With integer inputs every partial sum is exact, so bit b must equal
    # [sum_d plane[t][b][d] * x[d] >= 0] computed in exact integer arithmetic.
    rng = np.random.default_rng(12)
    L, K, D = 5, 9, 300
    planes = orc.simhash_planes(D, K, L, 1234)
    for _ in range(30):
        x = rng.integers(-50, 51, D).astype(np.float32)
        for t in range(L):
            s = planes[t].astype(np.int64) @ x.astype(np.int64)
            expect = sum(1 << b for b in range(K) if s[b] >= 0)
            assert orc.hash_dense(planes, x, t) == expect
    codes = orc.hash_dense_batch(planes, rng.integers(-5, 6, (3, D)).astype(np.float32))
    assert codes.shape == (3, L) and codes.max() < (1 << K)
