"""Pins the oracle's klearu-accel restatement (CPU only).

Sources of truth:
  * the reference's own known-answer tests (crates/klearu-accel/src/simd/mod.rs:365-470,
    bf16/mod.rs:153-287), restated with their inputs and expected values;
  * the AVX2 intrinsic build (oracle_avx2.c), which issues the reference's own
    instruction sequence: the portable emulation must match it bit for bit;
  * closed forms: integer-valued inputs make every f32 operation exact, so any
    dropped, duplicated or misplaced term changes the exact integer result;
  * torch's bfloat16 conversion (round to nearest even) as an independent library routine.
"""
import numpy as np
import pytest
import torch


def test_sparse_dot_kats(orc):
    # simd/mod.rs:365 and :378
    d = np.array([1, 2, 3, 4, 5], np.float32)
    assert orc.sparse_dot_dense_scalar([0, 2, 4], [1, 1, 1], d) == 9.0
    assert orc.sparse_dot_dense([0, 2, 4], [1, 1, 1], d) == 9.0
    d2 = np.array([10, 20, 30, 40], np.float32)
    assert orc.sparse_dot_dense([1, 3], [0.5, 0.25], d2) == 20.0
    # :404 empty, :415 exact chunk of 8
    assert orc.sparse_dot_dense([], [], np.array([1, 2, 3], np.float32)) == 0.0
    dense = np.arange(16, dtype=np.float32)
    assert orc.sparse_dot_dense(list(range(8)), [1.0] * 8, dense) == 28.0


def test_dense_dot_kats(orc):
    # simd/mod.rs:428 and :443
    assert orc.dense_dot_scalar([1, 2, 3], [4, 5, 6]) == 32.0
    assert orc.dense_dot([1, 2, 3], [4, 5, 6]) == 32.0
    assert orc.dense_dot([], []) == 0.0
    # :435 simd ~ scalar on the reference's own ramp inputs
    a = np.array([i * 0.3 - 15.0 for i in range(100)], np.float32)
    b = np.array([i * 0.7 + 2.0 for i in range(100)], np.float32)
    assert abs(orc.dense_dot(a, b) - orc.dense_dot_scalar(a, b)) < 1e-2


def test_scatter_add_kats(orc):
    # simd/mod.rs:451
    out = orc.scatter_add([1, 3, 5], [1, 2, 3], np.zeros(8, np.float32), 2.0)
    assert out[1] == 2.0 and out[3] == 4.0 and out[5] == 6.0 and out[0] == 0.0
    # :463 simd == scalar on the reference's inputs (duplicates accumulate)
    idx = [(i * 5) % 256 for i in range(50)]
    val = [i * 0.1 for i in range(50)]
    out = orc.scatter_add(idx, val, np.ones(256, np.float32), 0.5)
    ref = np.ones(256, np.float64)
    for i, v in zip(idx, val):
        ref[i] += np.float32(v) * 0.5
    np.testing.assert_allclose(out, ref, rtol=1e-6)


@pytest.mark.parametrize("n", list(range(0, 70)) + [127, 128, 129, 1000, 4096, 4099])
def test_dense_dot_emulation_matches_avx2_build(orc, n):
    rng = np.random.default_rng(n)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    e, v = orc.dense_dot(a, b), orc.dense_dot_avx2(a, b)
    assert e.tobytes() == v.tobytes(), (n, e, v)


@pytest.mark.parametrize("nnz", list(range(0, 40)) + [75, 157, 1000])
def test_sparse_dot_emulation_matches_avx2_build(orc, nnz):
    rng = np.random.default_rng(1000 + nnz)
    dense = rng.standard_normal(2048).astype(np.float32)
    idx = np.sort(rng.choice(2048, nnz, replace=False)).astype(np.uint32)
    val = rng.random(nnz).astype(np.float32)
    e, v = orc.sparse_dot_dense(idx, val, dense), orc.sparse_dot_dense_avx2(idx, val, dense)
    assert e.tobytes() == v.tobytes()


def test_dots_exact_on_integers(orc):
    # Small integers: every product and partial sum is exact in f32, so the
    # result must equal the exact integer dot product in any summation order.
    rng = np.random.default_rng(7)
    for n in (1, 7, 8, 15, 16, 17, 33, 100, 513):
        a = rng.integers(-20, 21, n).astype(np.float32)
        b = rng.integers(-20, 21, n).astype(np.float32)
        exact = float(np.dot(a.astype(np.int64), b.astype(np.int64)))
        assert orc.dense_dot(a, b) == exact
        assert orc.dense_dot_scalar(a, b) == exact
        idx = np.arange(n, dtype=np.uint32)
        assert orc.sparse_dot_dense(idx, a, b) == exact


def test_dense_dot_order_is_not_sequential(orc):
    # Guards against the emulation degenerating into a plain sequential sum:
    # with 16 lanes, 1e8 and -1e8 in different lanes cancel only in the hsum.
    a = np.zeros(32, np.float32)
    a[0], a[16], a[1] = 1e8, -1e8, 1.0
    b = np.ones(32, np.float32)
    # lane 0 accumulates 1e8 then -1e8 -> 0; lane 1 holds 1 -> total exactly 1
    assert orc.dense_dot(a, b) == 1.0


def test_bf16_round_trip_and_rne(orc):
    x = np.array([0.0, -0.0, 1.0, -2.5, 3.140625, 65504.0, 1e-40, np.inf, -np.inf], np.float32)
    b = orc.bf16_from_f32(x)
    np.testing.assert_array_equal(orc.bf16_to_f32(b)[:7], np.array(
        torch.from_numpy(x[:7]).to(torch.bfloat16).float()))
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1.0
    t = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8], np.float32)
    np.testing.assert_array_equal(orc.bf16_to_f32(orc.bf16_from_f32(t)),
                                  np.array([1.0, 1.0 + 2.0 ** -6], np.float32))
    # NaN stays NaN and quiet
    nb = orc.bf16_from_f32(np.array([np.nan], np.float32))
    assert np.isnan(orc.bf16_to_f32(nb))[0] and (int(nb[0]) & 0x0040)


def test_bf16_matches_torch_on_random(orc):
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(100000) * np.exp(rng.uniform(-30, 30, 100000))).astype(np.float32)
    ours = orc.bf16_from_f32(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_bf16_weights_tolerances(orc):
    # bf16/mod.rs:170 round trip rel < 0.02; :273 dot within 1% of f32 dot
    rng = np.random.default_rng(5)
    w = rng.uniform(-1, 1, 256).astype(np.float32)
    x = rng.uniform(-1, 1, 256).astype(np.float32)
    rt = orc.bf16_to_f32(orc.bf16_from_f32(w))
    nz = np.abs(w) > 1e-3
    assert np.all(np.abs(rt[nz] - w[nz]) / np.abs(w[nz]) < 0.02)
    bw = orc.bf16_from_f32(w)
    d_bf = orc.bf16_dot_f32(bw, x)
    d_f = float(np.dot(w.astype(np.float64), x))
    assert abs(d_bf - d_f) <= 0.01 * max(1.0, abs(d_f))
    # full mode on exact small integers is exact
    ai = orc.bf16_from_f32(np.arange(-8, 8, dtype=np.float32))
    assert orc.bf16_full_dot(ai, ai) == float(sum(i * i for i in range(-8, 8)))
    # update_from_f32 = RNE(w + delta)
    upd = orc.bf16_update_from_f32(orc.bf16_from_f32(np.array([1.0], np.float32)),
                                   np.array([0.25], np.float32))
    assert orc.bf16_to_f32(upd)[0] == 1.25
