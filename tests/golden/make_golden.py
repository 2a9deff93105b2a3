"""Writes tests/golden/quant_golden.npz: small vectors from scalar loops.

The loops are an element-by-element reading of the reference's definitions
(examples/52_dequantize.py:36-53 and :67-74 for dequantize,
examples/38_quantized_matmul.py:178-212 for the matvec, accumulated in
float64 as the reference's Python-float loop does).  They share no code with
oracle/quant_ref.py, which tests/test_oracle.py checks against them.
Run: python tests/golden/make_golden.py
"""

import os

import numpy as np


def scalar_case(seed, M, N, K, G):
    rng = np.random.default_rng(seed)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W4 = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    S4 = rng.uniform(0.001, 0.01, (N, K // G)).astype(np.float32)
    W8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
    S8 = rng.uniform(0.002, 0.02, (N, K // G)).astype(np.float32)
    deq4 = np.zeros((N, K), np.float32)
    deq8 = np.zeros((N, K), np.float32)
    for n in range(N):
        for b in range(K // 2):
            p = int(W4[n, b])
            deq4[n, 2 * b] = np.float32(float(p & 15) - 8.0) * S4[n, (2 * b) // G]
            deq4[n, 2 * b + 1] = np.float32(float(p >> 4) - 8.0) * S4[n, (2 * b + 1) // G]
        for k in range(K):
            deq8[n, k] = np.float32(float(W8[n, k])) * S8[n, k // G]
    y4 = np.zeros((M, N)); y8 = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            a4 = a8 = 0.0
            for k in range(K):
                a4 += float(X[m, k]) * float(deq4[n, k])
                a8 += float(X[m, k]) * float(deq8[n, k])
            y4[m, n], y8[m, n] = a4, a8
    return dict(X=X, W4=W4, S4=S4, W8=W8, S8=S8, G=np.int64(G), deq4=deq4, deq8=deq8, y4=y4, y8=y8)


def main():
    out = {}
    for tag, args in (("a", (0, 3, 24, 128, 32)), ("b", (1, 2, 10, 96, 96))):
        for k, v in scalar_case(*args).items():
            out[f"{tag}_{k}"] = v
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quant_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
