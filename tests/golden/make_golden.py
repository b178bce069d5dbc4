"""Writes the golden fixtures under tests/golden/ from first principles.

Nothing here runs or imports the reference (it is Rust and cannot be built in
this image).  Each fixture is computed independently of the oracle:

* lcg_kat.json      -- the Lcg recurrence of phobos-base/src/rng.rs:9-20 and its
                       known-answer test (rng.rs:50-63), evaluated with Python
                       integers and numpy float32 rounding.
* f16_pairs.json    -- f32 -> f16 RNE pairs from numpy.float16 (IEEE RNE, the
                       rounding half 2.7.1 uses at main.rs:447-449), including
                       ties, subnormals, overflow and signed zero.
* int_gemm.npz      -- exact-integer GEMM (phobos-bench/examples/masking.rs:108-110
                       style inputs a = i%7-3, b = i%5-2): every partial sum is an
                       integer below 2^24, so any summation order is exact.
* flash_tiny.json   -- softmax(Q K^T * scale) V in float64 closed form.

Run:  python tests/golden/make_golden.py
"""
import json
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
MASK = (1 << 64) - 1


def lcg_unit(seed, n):
    s = seed
    out = []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & MASK
        v = np.float32(s >> 33)                       # `as f32`, RNE
        out.append(float(v / np.float32(2.0 ** 31) - np.float32(1.0)))
    return out


def lcg_states(seed, n):
    s, out = seed, []
    for _ in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & MASK
        out.append(s)
    return out


def main():
    kat = {
        "recurrence": "s = s*6364136223846793005 + 1442695040888963407 mod 2^64; "
                      "u = f32(s>>33) / 2^31 - 1",
        "seed1_states": [str(x) for x in lcg_states(1, 8)],
        "seed1_unit": lcg_unit(1, 8),
        "seed2_unit": lcg_unit(2, 8),
        "seed3_unit": lcg_unit(3, 8),
        "seed7_unit": lcg_unit(7, 8),
    }
    with open(os.path.join(HERE, "lcg_kat.json"), "w") as f:
        json.dump(kat, f, indent=1)

    specials = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, 1e9, -1e9,
                float("inf"), float("-inf"), 2.0 ** -14, 2.0 ** -24, 2.0 ** -25,
                2.0 ** -25 * 1.5, 2.0 ** -26, 3 * 2.0 ** -25, 5.960464477539063e-08,
                1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -11 + 2.0 ** -23,
                0.1, -0.3, 3.14159265, 1e-5, -6.1e-5, 6.097555e-05, 2049.0, 2051.0,
                4097.0, 1.0 / 3.0]
    rng = np.random.default_rng(1234)
    rand = np.concatenate([rng.standard_normal(200) * 10.0 ** rng.integers(-8, 5, 200)])
    vals = np.array(specials + list(rand), dtype=np.float32)
    bits_in = vals.view(np.uint32).tolist()
    with np.errstate(over="ignore"):
        bits_out = vals.astype(np.float16).view(np.uint16).tolist()
    with open(os.path.join(HERE, "f16_pairs.json"), "w") as f:
        json.dump({"f32_bits": bits_in, "f16_bits": bits_out}, f)

    M, K, N = 96, 64, 100
    a = (np.arange(M * K) % 7 - 3).astype(np.int64).reshape(M, K)
    b = (np.arange(K * N) % 5 - 2).astype(np.int64).reshape(K, N)
    c = a @ b
    np.savez(os.path.join(HERE, "int_gemm.npz"), a=a.astype(np.float32), b=b.astype(np.float32),
             c=c.astype(np.float32))

    q = np.array([[1.0, 0.0], [0.0, 1.0], [0.5, -0.5], [2.0, 2.0]])
    k = np.array([[1.0, 1.0], [-1.0, 0.5], [0.25, -2.0]])
    v = np.array([[1.0, 2.0], [3.0, -1.0], [-2.0, 0.5]])
    scale = 0.7
    s = q @ k.T * scale
    p = np.exp(s - s.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    with open(os.path.join(HERE, "flash_tiny.json"), "w") as f:
        json.dump({"q": q.tolist(), "k": k.tolist(), "v": v.tolist(), "scale": scale,
                   "o": (p @ v).tolist()}, f, indent=1)


if __name__ == "__main__":
    main()
