"""CPU tests of the native LibSVM loader (kh_libsvm_*, host only).

Known answers are the reference's own tests (crates/klearu-core/src/data/
libsvm.rs:203-400) plus the from_pairs rules (tensor/sparse.rs:36-57) and
Rust's FromStr number grammar."""
import math

import numpy as np
import pytest

from klearu_amd import KlearuError
from klearu_amd.formats import LibSvmDataset


def load(s, fd, nl):
    return LibSvmDataset.load_from_bytes(s, fd, nl)


def test_reference_single_label_0based():
    ds = load("0 0:1.0 2:3.5\n1 1:2.0\n", 4, 2)
    assert (len(ds), ds.feature_dim, ds.num_labels) == (2, 4, 2)
    i, v, l = ds.get(0)
    assert (i.tolist(), v.tolist(), l) == ([0, 2], [1.0, 3.5], [0])
    i, v, l = ds.get(1)
    assert (i.tolist(), v.tolist(), l) == ([1], [2.0], [1])


def test_reference_1based_autodetect_and_mixed():
    ds = load("0 1:1.0 3:2.0\n1 2:5.0\n", 4, 2)
    assert ds.get(0)[0].tolist() == [0, 2] and ds.get(0)[1].tolist() == [1.0, 2.0]
    assert ds.get(1)[0].tolist() == [1]
    assert load("0 0:1.0 5:2.0\n", 10, 1).get(0)[0].tolist() == [0, 5]
    # the detection is over the whole file: one 0 index anywhere keeps 0-based
    assert load("0 1:1.0\n1 0:2.0\n", 4, 2).get(0)[0].tolist() == [1]
    # smallest index 2 (no 0, no 1): no shift
    assert load("0 2:1.0 3:1.0\n", 5, 1).get(0)[0].tolist() == [2, 3]


def test_reference_labels_comments_blanks_empty():
    assert load("0,3,7 0:1.0 1:2.0\n", 5, 10).get(0)[2] == [0, 3, 7]
    assert load("0,1,2,3,4,5,6,7,8,9 0:1.0\n", 5, 10).get(0)[2] == list(range(10))
    i, v, l = load("5\n", 10, 6).get(0)
    assert l == [5] and i.size == 0
    assert len(load("# This is a comment\n\n0 0:1.0\n   \n1 1:2.0\n", 5, 2)) == 2
    assert load("0 0:1.0 1:2.0 # this is a comment\n", 5, 2).get(0)[0].size == 2
    assert len(load("", 10, 5)) == 0
    # CRLF line ends and tabs
    ds = load("0\t0:1.0 1:2.0\r\n1 2:3.0\r\n", 5, 2)
    assert len(ds) == 2 and ds.get(1)[0].tolist() == [2]


@pytest.mark.parametrize("text,msg", [
    ("abc 0:1.0\n", "invalid label"),
    ("0 badformat\n", "expected 'index:value'"),
    ("0 abc:1.0\n", "invalid feature index"),
    ("0 0:not_a_number\n", "invalid feature value"),
    ("0,,1 0:1.0\n", "invalid label"),
    ("-1 0:1.0\n", "invalid label"),
    ("4294967296 0:1.0\n", "invalid label"),
    ("0 0:1.0\n1 0:1e\n", "line 2: invalid feature value"),
    ("0 0:.\n", "invalid feature value"),
    ("0 0:nan(1)\n", "invalid feature value"),
])
def test_reference_errors(text, msg):
    with pytest.raises(KlearuError) as e:
        load(text, 10, 5)
    assert msg in str(e.value)


def test_reference_sorted_clamped_negative():
    i, v, _ = load("0 3:1.0 1:2.0 0:3.0\n", 10, 1).get(0)
    assert i.tolist() == [0, 1, 3] and v.tolist() == [3.0, 2.0, 1.0]
    i, _, _ = load("0 0:1.0 999:2.0\n", 10, 1).get(0)
    assert i.tolist() == [0, 9]
    assert load("0 0:-1.5 2:3.0\n", 5, 1).get(0)[1].tolist() == [-1.5, 3.0]


def test_from_pairs_accumulates_repeats_in_order():
    # 2 appears three times (after sorting, in input order): ((a + b) + c) in f32
    a, b, c = 1e8, 1.0, -1e8
    i, v, _ = load(f"0 0:9 2:{a} 1:5 2:{b} 2:{c}\n", 4, 1).get(0)
    assert i.tolist() == [0, 1, 2]
    want = np.float32(np.float32(np.float32(a) + np.float32(b)) + np.float32(c))
    assert v[2] == want and want == 0.0   # the 1.0 is lost against 1e8 in f32
    # clamping can create repeats: 999 and 998 both land on 9
    i, v, _ = load("0 0:1 999:2 998:3\n", 10, 1).get(0)
    assert i.tolist() == [0, 9] and v.tolist() == [1.0, 5.0]


def test_f32_grammar_and_rounding():
    vals = ["+1.5", "1.", ".5", "1e3", "1E-3", "-0", "inf", "-Infinity", "NaN", "3.4028235e38",
            "3.4028236e38", "1e39", "1e-46", "1.4e-45", "0.1", "16777217", "123456789012345678901234567890"]
    text = "0 " + " ".join(f"{k}:{s}" for k, s in enumerate(vals)) + "\n"
    _, v, _ = load(text, 64, 1).get(0)
    want = [1.5, 1.0, 0.5, 1000.0, np.float32(1e-3), -0.0, math.inf, -math.inf, math.nan,
            np.float32(3.4028235e38), math.inf, math.inf, 0.0, np.float32(1.4e-45), np.float32(0.1),
            16777216.0, np.float32(123456789012345678901234567890.0)]
    for got, w, s in zip(v, want, vals):
        if isinstance(w, float) and math.isnan(w):
            assert math.isnan(got), s
        else:
            assert np.float32(got) == np.float32(w), s
    assert math.copysign(1.0, v[5]) == -1.0   # "-0" keeps its sign


def test_file_load_and_csr(tmp_path):
    p = tmp_path / "d.txt"
    p.write_text("1,4 1:0.5 3:0.25\n2 2:1.0\n")
    ds = LibSvmDataset.load(p, 3, 5)
    assert ds.off.tolist() == [0, 2, 3] and ds.idx.tolist() == [0, 2, 1]
    assert ds.label_off.tolist() == [0, 2, 3] and ds.labels.tolist() == [1, 4, 2]
    with pytest.raises(KlearuError):
        LibSvmDataset.load(tmp_path / "missing.txt", 3, 5)
