"""GPU parity for the klearu-accel entry points: bit-exact vs the oracle's
restatement of the AVX2 path (crates/klearu-accel/src/simd/mod.rs:145-236) and
the sequential BF16 dots (bf16/mod.rs:64-134)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("n", [0, 1, 7, 8, 15, 16, 17, 24, 31, 100, 4096, 4099, 11008])
def test_dense_dot_bit_exact(kh, orc, n):
    from klearu_amd.accel import dense_dot_dense_simd
    rng = np.random.default_rng(n)
    A = rng.standard_normal((5, n)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    got = dense_dot_dense_simd(torch.from_numpy(A).cuda(), torch.from_numpy(b).cuda()).cpu().numpy()
    ref = np.array([orc.dense_dot(A[r], b) for r in range(5)], np.float32)
    np.testing.assert_array_equal(bits(got), bits(ref))


def test_dense_dot_kats(kh):
    from klearu_amd.accel import dense_dot_dense_simd
    assert float(dense_dot_dense_simd([1.0, 2.0, 3.0], [4.0, 5.0, 6.0])) == 32.0


@pytest.mark.parametrize("nnz", [0, 3, 8, 9, 75, 157, 1000])
def test_sparse_dot_bit_exact(kh, orc, nnz):
    from klearu_amd.accel import sparse_dot_dense_simd
    rng = np.random.default_rng(100 + nnz)
    dense = rng.standard_normal(4096).astype(np.float32)
    idx = np.sort(rng.choice(4096, nnz, replace=False)).astype(np.uint32)
    val = rng.random(nnz).astype(np.float32)
    got = float(sparse_dot_dense_simd(idx, val, torch.from_numpy(dense).cuda()))
    assert np.float32(got).tobytes() == orc.sparse_dot_dense(idx, val, dense).tobytes()
    if nnz == 3:
        d = np.array([1, 2, 3, 4, 5], np.float32)
        assert float(sparse_dot_dense_simd([0, 2, 4], [1, 1, 1], torch.from_numpy(d).cuda())) == 9.0


@pytest.mark.parametrize("n", [3, 50, 1024, 5000])
def test_scatter_add_bit_exact_with_duplicates(kh, orc, n):
    from klearu_amd.accel import scatter_add_simd
    rng = np.random.default_rng(n)
    idx = rng.integers(0, 64, n).astype(np.uint32)  # many duplicates
    val = rng.standard_normal(n).astype(np.float32)
    d0 = rng.standard_normal(64).astype(np.float32)
    got = scatter_add_simd(idx, val, torch.from_numpy(d0).cuda(), 0.37).cpu().numpy()
    np.testing.assert_array_equal(bits(got), bits(orc.scatter_add(idx, val, d0, 0.37)))


def test_bf16_ops(kh, orc):
    from klearu_amd.accel import Bf16Weights, bf16_full_dot
    rng = np.random.default_rng(5)
    w = rng.uniform(-1, 1, 4099).astype(np.float32)
    x = rng.standard_normal(4099).astype(np.float32)
    bw = Bf16Weights.from_f32(torch.from_numpy(w).cuda())
    ref_bits = orc.bf16_from_f32(w)
    np.testing.assert_array_equal(bw.data.cpu().numpy().view(np.uint16), ref_bits)
    np.testing.assert_array_equal(bw.to_f32().cpu().numpy(), orc.bf16_to_f32(ref_bits))
    assert np.float32(float(bw.dot_f32(torch.from_numpy(x).cuda()))).tobytes() == \
        orc.bf16_dot_f32(ref_bits, x).tobytes()
    other = torch.from_numpy(orc.bf16_from_f32(x).view(np.int16)).cuda()
    assert np.float32(float(bf16_full_dot(bw.data, other))).tobytes() == \
        orc.bf16_full_dot(ref_bits, orc.bf16_from_f32(x)).tobytes()
    delta = (rng.standard_normal(4099) * 0.01).astype(np.float32)
    bw.update_from_f32(torch.from_numpy(delta).cuda())
    np.testing.assert_array_equal(bw.data.cpu().numpy().view(np.uint16),
                                  orc.bf16_update_from_f32(ref_bits, delta))


def test_expf_matches_glibc(kh, orc):
    """The device exp equals glibc expf (Rust's f32::exp) bit for bit: a strided
    sweep over all 2^32 bit patterns plus every pattern in windows around 0,
    the overflow / underflow thresholds and the subnormal results."""
    from klearu_amd.accel import exp_f32
    u = np.arange(0, 1 << 32, 251, dtype=np.uint64).astype(np.uint32)
    windows = []
    for centre in (0.0, 1.0, -1.0, 88.72283, 88.72284, -103.97208, -87.33655, -100.0, 1e-8, -1e-8):
        c = int(np.array([centre], np.float32).view(np.uint32)[0])
        windows.append(np.arange(max(c - (1 << 16), 0), min(c + (1 << 16), (1 << 32) - 1), dtype=np.uint64))
    u = np.concatenate([u.astype(np.uint64)] + windows).astype(np.uint32)
    x = u.view(np.float32)
    x = x[~np.isnan(x)]
    print(f"expf sweep: {x.size} inputs", flush=True)
    got = exp_f32(torch.from_numpy(x).cuda()).cpu().numpy()
    ref = orc.expf(x)
    bad = np.nonzero(bits(got) != bits(ref))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first x={x[bad[0]]!r} got={got[bad[0]]!r} ref={ref[bad[0]]!r}"
