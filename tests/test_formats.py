"""On-disk formats on the host (CPU): predictor JSON and safetensors.

The predictor files are the serde layout of SparsityPredictor
(crates/klearu-dejavu/src/predictor/mlp_predictor.rs:10-26, save/load :87-98)
in a PredictorStore directory (crates/klearu-llm/src/sparse/predictor_store.rs:
59-89); the fixture is tests/golden/predictor_store (make_predictor_store.py).
serde_json reads an f32 as the f32 nearest the f64 nearest the decimal, which
Python's float() (correctly rounded) followed by np.float32 restates.
The safetensors files are written with the safetensors package (the format's
own writer) and by hand for malformed cases; the reader mirrors
crates/klearu-llm/src/weight/safetensors.rs:37-159 and loader.rs:30-49.
"""
import ctypes as C
import json
import os
import struct

import numpy as np
import pytest

from klearu_amd import _lib
from klearu_amd._lib import KH_ERR_ARG, KH_ERR_CAPACITY, KH_ERR_UNSUPPORTED, KlearuError
from klearu_amd.formats import SafeTensorsFile

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "predictor_store")


def hp(a):
    return a.ctypes.data_as(C.c_void_p)


def read_json(path):
    din, dh, dout = C.c_int(), C.c_int(), C.c_int()
    _lib.call("kh_predictor_read_json", os.fsencode(path), C.byref(din), C.byref(dh), C.byref(dout),
              None, None, None, None)
    w1 = np.empty((dh.value, din.value), np.float32)
    b1 = np.empty(dh.value, np.float32)
    w2 = np.empty((dout.value, dh.value), np.float32)
    b2 = np.empty(dout.value, np.float32)
    _lib.call("kh_predictor_read_json", os.fsencode(path), C.byref(din), C.byref(dh), C.byref(dout),
              hp(w1), hp(b1), hp(w2), hp(b2))
    return w1, b1, w2, b2


def write_json(path, w1, b1, w2, b2):
    w1, b1, w2, b2 = (np.ascontiguousarray(a, np.float32) for a in (w1, b1, w2, b2))
    _lib.call("kh_predictor_write_json", os.fsencode(path), w1.shape[1], w1.shape[0], w2.shape[0],
              hp(w1), hp(b1), hp(w2), hp(b2))


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("name", ["layer_0_head", "layer_0_neuron", "layer_2_neuron"])
def test_predictor_fixture_reads_bit_exact(name):
    exp = np.load(os.path.join(GOLD, "expected.npz"))
    got = read_json(os.path.join(GOLD, name + ".json"))
    for k, g in zip(("w1", "b1", "w2", "b2"), got):
        np.testing.assert_array_equal(bits(g), bits(exp[f"{name}.{k}"]), err_msg=k)


def test_predictor_writer_spelling(tmp_path):
    """Edge values are written as serde_json (ryu) spells them: shortest digits,
    positional for 1e-6 <= |v| < 1e13, else d.ddde<exp> ("1e-7", "1.5e13")."""
    exp = np.load(os.path.join(GOLD, "expected.npz"))
    edge = exp["edge"]
    p = tmp_path / "p.json"
    write_json(p, np.ones((edge.size, 1)), edge, np.ones((1, edge.size)), np.zeros(1))
    text = p.read_text()
    assert '"b1":[' + ",".join(exp["edge_text"]) + "]" in text
    assert text.startswith('{"w1":[[1.0],') and text.endswith('"input_dim":1,"hidden_dim":17,"output_dim":1}')


def test_predictor_roundtrip_random_bit_patterns(tmp_path):
    """Every finite f32 (normals, subnormals, both zeros) survives write -> read,
    and the text reads back the same way through the decimal -> f64 -> f32 path."""
    rng = np.random.default_rng(7)
    u = rng.integers(0, 2 ** 32, 40000, dtype=np.uint64).astype(np.uint32)
    u[:2000] &= 0x807FFFFF                                             # subnormals and zeros
    u = u[np.isfinite(u.view(np.float32))]
    n = u.size - u.size % 100
    w1 = u[:n].view(np.float32).reshape(100, n // 100)
    p = tmp_path / "p.json"
    write_json(p, w1, np.zeros(100), np.zeros((1, 100)), np.zeros(1))
    got = read_json(p)[0]
    np.testing.assert_array_equal(bits(got), bits(w1))
    d = json.loads(p.read_text())
    np.testing.assert_array_equal(bits(np.array(d["w1"], np.float64).astype(np.float32)), bits(w1))


def test_predictor_reader_accepts_any_field_order_and_unknown_fields(tmp_path):
    p = tmp_path / "p.json"
    p.write_text(' { "output_dim" : 1, "b2": [ -0.0 ], "extra": {"a": [1, {"b": null}], "s": "x\\u00e9\\"y"},'
                 '"w2": [[1E0, 2, 0]], "hidden_dim": 3, "b1": [1e-400, -1e-400, 0], "input_dim": 1,'
                 '"w1": [[0.1], [3.4028234663852886e38], [3.4028235677973366e38]] }\n')
    w1, b1, w2, b2 = read_json(p)
    # the f64 halfway between f32 max and 2^128 rounds (to even) to infinity, as Rust's `as f32`
    np.testing.assert_array_equal(bits(w1.ravel()), bits([0.1, 3.4028235e38, np.inf]))
    np.testing.assert_array_equal(bits(b1), bits([0.0, -0.0, 0.0]))   # underflow reads as a signed zero
    np.testing.assert_array_equal(w2, [[1.0, 2.0, 0.0]])
    assert bits(b2)[0] == 0x80000000


@pytest.mark.parametrize("text", [
    '{"w1":[[1]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1}',          # missing field
    '{"w1":[[1],[2,3]],"b1":[0,0],"w2":[[1,1]],"b2":[0],"input_dim":1,"hidden_dim":2,"output_dim":1}',
    '{"w1":[[1]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":2,"hidden_dim":1,"output_dim":1}',
    '{"w1":[[1e400]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1,"output_dim":1}',
    '{"w1":[[null]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1,"output_dim":1}',
    '{"w1":[[01]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1,"output_dim":1}',
    '{"w1":[[1]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1,"output_dim":1} x',
    '{"w1":[[1]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1.5,"hidden_dim":1,"output_dim":1}',
    '{"w1":[[1]],"b1":[0],"w2":[[1]],"b2":[0],"input_dim":1,"hidden_dim":1,"output_dim":1',
])
def test_predictor_reader_rejects_malformed(tmp_path, text):
    p = tmp_path / "p.json"
    p.write_text(text)
    with pytest.raises(KlearuError) as e:
        read_json(p)
    assert e.value.code == KH_ERR_ARG


def test_predictor_writer_rejects_non_finite(tmp_path):
    with pytest.raises(KlearuError):
        write_json(tmp_path / "p.json", [[np.nan]], [0], [[1]], [0])


# ---- safetensors ------------------------------------------------------------

def st_write(path, tensors, metadata=None):
    """Writes a safetensors file by hand: u64 LE header length, JSON header padded
    with spaces to 8 bytes, then the tensors' bytes (spec of the format)."""
    hdr, blobs, off = {}, [], 0
    for name, (dtype, shape, raw) in tensors.items():
        hdr[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    if metadata is not None:
        hdr["__metadata__"] = metadata
    h = json.dumps(hdr).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)) + h + b"".join(blobs))


def test_safetensors_written_by_the_format_library(tmp_path):
    torch = pytest.importorskip("torch")
    st_torch = pytest.importorskip("safetensors.torch")
    g = torch.Generator().manual_seed(3)
    t = {"model.layers.0.mlp.gate_proj.weight": torch.randn(6, 4, generator=g).to(torch.bfloat16),
         "model.norm.weight": torch.randn(4, generator=g).to(torch.float16),
         "lm_head.weight": torch.randn(2, 3, 2, generator=g)}
    path = str(tmp_path / "m.safetensors")
    st_torch.save_file(t, path, metadata={"format": "pt"})
    with SafeTensorsFile(path) as st:
        assert st.names() == sorted(t)
        infos = st.tensors()
        assert infos["model.norm.weight"].dtype == "F16" and infos["model.norm.weight"].shape == (4,)
        assert infos["lm_head.weight"].dtype == "F32" and infos["lm_head.weight"].shape == (2, 3, 2)
        for name, ref in t.items():
            np.testing.assert_array_equal(st.tensor_to_f32(name), ref.float().numpy())
        raw = st.tensor_data("model.layers.0.mlp.gate_proj.weight")
        assert raw.dtype == np.uint16
        np.testing.assert_array_equal(raw, t["model.layers.0.mlp.gate_proj.weight"].view(torch.int16).numpy()
                                      .view(np.uint16))
        assert st.layer_name(0, "mlp.gate_proj.weight") == "model.layers.0.mlp.gate_proj.weight"


def test_safetensors_f16_conversion_is_exact(tmp_path):
    """Every binary16 pattern (subnormals, infinities, NaN payloads) converts as
    half::f16::to_f32 does, i.e. exactly (numpy's float16 -> float32)."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    path = str(tmp_path / "h.safetensors")
    st_write(path, {"h": ("F16", h.shape, h.tobytes())})
    with SafeTensorsFile(path) as st:
        got = st.tensor_to_f32("h")
    ref = h.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(bits(got[fin]), bits(ref[fin]))
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(np.isinf(got) & (got > 0), np.isinf(ref) & (ref > 0))


def test_safetensors_bf16_conversion_is_a_shift(tmp_path):
    b = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    path = str(tmp_path / "b.safetensors")
    st_write(path, {"b": ("BF16", b.shape, b.tobytes())})
    with SafeTensorsFile(path) as st:
        np.testing.assert_array_equal(bits(st.tensor_to_f32("b")), b.astype(np.uint32) << 16)


def test_safetensors_directory_sorted_and_shadowed(tmp_path):
    """load_model opens every *.safetensors file in sorted order; a later file's
    tensor replaces an earlier one of the same name."""
    one = np.ones(2, np.float32).tobytes()
    two = (2 * np.ones(2, np.float32)).tobytes()
    st_write(tmp_path / "model-00002-of-00002.safetensors",
             {"shared": ("F32", (2,), two), "model.language_model.layers.3.mlp.up_proj.weight": ("F32", (2,), two)})
    st_write(tmp_path / "model-00001-of-00002.safetensors", {"shared": ("F32", (2,), one), "a": ("F32", (2,), one)},
             metadata={"total_size": "16"})
    (tmp_path / "config.json").write_text("{}")
    with SafeTensorsFile(str(tmp_path)) as st:
        assert st.names() == ["a", "model.language_model.layers.3.mlp.up_proj.weight", "shared"]
        np.testing.assert_array_equal(st.tensor_to_f32("shared"), [2, 2])
        assert st.layer_name(3, "mlp.up_proj.weight") == "model.language_model.layers.3.mlp.up_proj.weight"
        with pytest.raises(KeyError):
            st.layer_name(4, "mlp.up_proj.weight")


def _raises(code, fn, *a):
    with pytest.raises(KlearuError) as e:
        fn(*a)
    assert e.value.code == code, str(e.value)


def test_safetensors_malformed_files(tmp_path):
    p = tmp_path / "x.safetensors"
    p.write_bytes(b"\x01\x00\x00")
    _raises(KH_ERR_ARG, SafeTensorsFile, str(p))                                    # file too small
    p.write_bytes(struct.pack("<Q", 100) + b"{}")
    _raises(KH_ERR_ARG, SafeTensorsFile, str(p))                                    # invalid header length
    st_write(p, {"i": ("I64", (1,), b"\0" * 8)})
    _raises(KH_ERR_UNSUPPORTED, SafeTensorsFile, str(p))                            # unsupported dtype
    p.write_bytes(struct.pack("<Q", 2) + b"[]")
    _raises(KH_ERR_ARG, SafeTensorsFile, str(p))                                    # header is not an object
    hdr = json.dumps({"t": {"dtype": "F32", "shape": [2], "data_offsets": [8, 4]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 8)
    _raises(KH_ERR_ARG, SafeTensorsFile, str(p))                                    # end < start
    _raises(KH_ERR_ARG, SafeTensorsFile, str(tmp_path / "missing.safetensors"))
    empty = tmp_path / "empty"
    empty.mkdir()
    _raises(KH_ERR_ARG, SafeTensorsFile, str(empty))                                # no .safetensors files


def test_safetensors_bounds_and_sizes_checked_on_read(tmp_path):
    p = tmp_path / "x.safetensors"
    hdr = json.dumps({"oob": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]},
                      "short": {"dtype": "F32", "shape": [3], "data_offsets": [0, 8]},
                      # 2^62 elements of 4 bytes: the byte count wraps to 0 in 64 bits
                      "wrap": {"dtype": "F32", "shape": [1 << 62], "data_offsets": [0, 0]}}).encode()
    p.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 8)
    with SafeTensorsFile(str(p)) as st:
        _raises(KH_ERR_ARG, st.tensor_to_f32, "oob")                                 # data out of bounds
        _raises(KH_ERR_ARG, st.tensor_to_f32, "short")                               # bytes != shape
        _raises(KH_ERR_ARG, _lib.call, "kh_safetensors_read_f32", st._h, b"wrap",    # shape overflows bytes
                hp(np.empty(1, np.float32)), 1 << 62)
        _raises(KH_ERR_ARG, _lib.call, "kh_safetensors_read_raw", st._h, b"wrap", hp(np.empty(1, np.float32)), 0)
        _raises(KH_ERR_ARG, st.info, "absent")                                       # MissingWeight
        out = np.empty(5, np.float32)
        _raises(KH_ERR_ARG, _lib.call, "kh_safetensors_read_f32", st._h, b"short", hp(out), 5)
        buf = C.create_string_buffer(3)
        _raises(KH_ERR_CAPACITY, _lib.call, "kh_safetensors_name", st._h, 0, buf, 3)
