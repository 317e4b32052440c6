"""Hidden rows that stress the exact parallel sum of squares behind RmsNorm
(rms_norm.rs:48-51), at a given width: a running sum stuck at 2^24 while the
exact sum grows (every square 1.0 is a tie that rounds back down, so every
chunk's speculative window misses), squares just above half an ulp (each
rounds up, so the sum drifts from its guess), leading zeros, an all-zero row,
tiny and huge magnitudes and a wide exponent range."""
import numpy as np


def hard_hidden_rows(rng, n):
    rows = {}
    rows["normal"] = rng.standard_normal(n)
    stuck = np.ones(n)
    stuck[0] = 4096.0  # 4096^2 = 2^24, then + 1.0 ties back to 2^24 every step
    rows["ties stuck at 2^24"] = stuck
    up = np.full(n, np.sqrt(1.0000001))
    up[0] = 4096.0
    rows["round-up drift"] = up
    z = rng.standard_normal(n)
    z[: (n * 700) // 4096] = 0.0
    rows["leading zeros"] = z
    rows["all zero"] = np.zeros(n)
    rows["tiny"] = rng.standard_normal(n) * 1e-20
    rows["huge"] = rng.standard_normal(n) * 1e17
    rows["wide range"] = rng.standard_normal(n) * np.exp(rng.uniform(-20, 20, n))
    return {k: v.astype(np.float32) for k, v in rows.items()}
