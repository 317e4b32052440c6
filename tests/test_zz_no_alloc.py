"""GPU: kh_predictor_select_top_k_noalloc (scratch from a static device array,
no allocation) against kh_predictor_select_top_k, through the C ABI.

Bar: top-k selections are integer results, so bit-exact: the same ids in the
same order, for both orders, on consecutive calls whose second input is
smaller, plus the oracle's own selection for the first row; a request larger
than the static scratch is refused with KH_ERR_CAPACITY.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _predictor(orc, rng, ind, hid, out):
    from klearu_amd.dejavu import SparsityPredictor
    bf = lambda a: orc.bf16_from_f32(np.asarray(a, np.float32))  # noqa: E731
    w1 = bf(rng.normal(0, 0.02, (hid, ind)))
    w2 = bf(rng.normal(0, 0.02 if hid > 64 else 0.1, (out, hid)))
    b1 = rng.normal(0, 0.1, hid).astype(np.float32)
    b2 = rng.normal(0, 0.1, out).astype(np.float32)
    return SparsityPredictor(orc.bf16_to_f32(w1), b1, orc.bf16_to_f32(w2), b2), (w1, b1, w2, b2)


@pytest.mark.parametrize("ind,hid,out,k", [
    (4096, 256, 11008, 1652),   # cfg3 neuron predictor (top-k kernel)
    (4096, 128, 32, 16),        # cfg4 head predictor (top-k inside layer 2)
])
def test_noalloc_matches_select_top_k(kh, orc, ind, hid, out, k):
    from klearu_amd import _lib
    from klearu_amd._dev import ptr
    from klearu_amd.dejavu import ORDER_ASCENDING, ORDER_SCORE
    rng = np.random.default_rng(ind + out)
    p, (w1, b1, w2, b2) = _predictor(orc, rng, ind, hid, out)
    kk = min(k, out)
    for order in (ORDER_SCORE, ORDER_ASCENDING):
        for batch in (4, 2):   # the second call smaller than the first
            x = rng.standard_normal((batch, ind)).astype(np.float32)
            xd = torch.from_numpy(x).cuda()
            ref = torch.full((batch, kk), -1, dtype=torch.int32, device="cuda")
            got = torch.full((batch, kk), -7, dtype=torch.int32, device="cuda")
            _lib.call("kh_predictor_select_top_k", p._h, ptr(xd), batch, k, order, ptr(ref), None)
            _lib.call("kh_predictor_select_top_k_noalloc", p._h, ptr(xd), batch, k, order, ptr(got), None)
            torch.cuda.synchronize()
            print(f"order {order} batch {batch}: {int((got != ref).sum())} ids differ")
            np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
            scores, _ = orc.predictor_predict(w1, b1, w2, b2, x[0])
            want = orc.select_top_k(scores, kk)
            if order == ORDER_ASCENDING:
                want = np.sort(want)
            np.testing.assert_array_equal(got[0].cpu().numpy(), want)


def test_noalloc_rejects_oversized_request(kh, orc):
    from klearu_amd import KlearuError, _lib
    from klearu_amd._lib import KH_ERR_CAPACITY
    from klearu_amd._dev import ptr
    from klearu_amd.dejavu import ORDER_SCORE
    rng = np.random.default_rng(9)
    p, _ = _predictor(orc, rng, 512, 64, 11008)
    batch = 128   # 128 x 11008 scores alone are 5.6 MB, above the 4 MiB scratch
    x = torch.zeros(batch, 512, device="cuda")
    ids = torch.empty(batch, 100, dtype=torch.int32, device="cuda")
    with pytest.raises(KlearuError) as e:
        _lib.call("kh_predictor_select_top_k_noalloc", p._h, ptr(x), batch, 100, ORDER_SCORE, ptr(ids), None)
    assert e.value.code == KH_ERR_CAPACITY
