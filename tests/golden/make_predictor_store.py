"""Writes the PredictorStore fixture: tests/golden/predictor_store/.

A directory as PredictorStore::save leaves it (crates/klearu-llm/src/sparse/
predictor_store.rs:59-74): layer_{i}_head.json / layer_{i}_neuron.json, each the
serde_json text of a SparsityPredictor (crates/klearu-dejavu/src/predictor/
mlp_predictor.rs:10-26): {"w1":[[..]..],"b1":[..],"w2":[[..]..],"b2":[..],
"input_dim":..,"hidden_dim":..,"output_dim":..}, every f32 in ryu's shortest
spelling.  Layers 0 (head 8->4->6, neuron 8->4->12) and 2 (neuron only) are
present; layer 1 is absent (the first-k fallback).  The weights mix N(0, std)
draws, as SparsityPredictor::new draws them, with edge values (subnormals,
-0.0, f32 max, 1e-7, integers).  expected.npz holds the same arrays, the
inputs the reference's tests use (0.5 and 0.1 constant rows) and nothing else.

    python tests/golden/make_predictor_store.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "predictor_store")

EDGE = np.array([1e-45, -1e-45, 1.1754944e-38, -0.0, 0.0, 3.4028235e38, -3.4028235e38, 1e-7, 1e-6, 0.1,
                 2.0, 16777216.0, 1.5e13, 9999999.0, 1e13, 123456.79, 0.000123], np.float32)


def ryu(v) -> str:
    """f32 -> serde_json's spelling (ryu): shortest digits; positional when
    -6 < kk <= 13 with 10^(kk-1) <= |v| < 10^kk, else d.ddde<exp>."""
    v = np.float32(v)
    sign = "-" if np.signbit(v) else ""
    if v == 0:
        return sign + "0.0"
    m, e = np.format_float_scientific(abs(v), unique=True, trim="-").split("e")
    digits = m.replace(".", "")
    kk = int(e) + 1
    n = len(digits)
    if 0 < kk <= 13:
        body = digits + "0" * (kk - n) + ".0" if n <= kk else digits[:kk] + "." + digits[kk:]
    elif -6 < kk <= 0:
        body = "0." + "0" * (-kk) + digits
    else:
        body = digits[0] + ("." + digits[1:] if n > 1 else "") + "e" + str(kk - 1)
    return sign + body


def dump(w1, b1, w2, b2):
    arr = lambda a: "[" + ",".join(ryu(x) for x in a) + "]"
    mat = lambda a: "[" + ",".join(arr(r) for r in a) + "]"
    return ('{"w1":' + mat(w1) + ',"b1":' + arr(b1) + ',"w2":' + mat(w2) + ',"b2":' + arr(b2) +
            f',"input_dim":{w1.shape[1]},"hidden_dim":{w1.shape[0]},"output_dim":{w2.shape[0]}}}')


def predictor(rng, din, dh, dout, edges):
    std1 = np.sqrt(2.0 / (din + dh))
    std2 = np.sqrt(2.0 / (dh + dout))
    w1 = (rng.standard_normal((dh, din)) * std1).astype(np.float32)
    w2 = (rng.standard_normal((dout, dh)) * std2).astype(np.float32)
    b1 = (rng.standard_normal(dh) * 0.01).astype(np.float32)
    b2 = (rng.standard_normal(dout) * 0.01).astype(np.float32)
    if edges:
        flat = w2.reshape(-1)
        flat[: EDGE.size] = EDGE
    return w1, b1, w2, b2


def main():
    os.makedirs(OUT, exist_ok=True)
    rng = np.random.default_rng(42)
    files = {"layer_0_head": predictor(rng, 8, 4, 6, False),
             "layer_0_neuron": predictor(rng, 8, 4, 12, True),
             "layer_2_neuron": predictor(rng, 8, 4, 12, False)}
    exp = {}
    for name, (w1, b1, w2, b2) in files.items():
        text = dump(w1, b1, w2, b2)
        # the text is valid JSON whose numbers read back (decimal -> f64 -> f32) to the arrays
        d = json.loads(text)
        assert np.array_equal(np.array(d["w2"], np.float64).astype(np.float32).view(np.uint32), w2.view(np.uint32))
        with open(os.path.join(OUT, name + ".json"), "w") as f:
            f.write(text)
        for k, a in zip(("w1", "b1", "w2", "b2"), (w1, b1, w2, b2)):
            exp[f"{name}.{k}"] = a
    exp["edge"] = EDGE
    exp["edge_text"] = np.array([ryu(x) for x in EDGE])
    np.savez(os.path.join(OUT, "expected.npz"), **exp)


if __name__ == "__main__":
    main()
