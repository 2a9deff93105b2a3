"""Seeded synthetic inputs for the five workload configurations.

Draw order X -> W -> S from ``np.random.default_rng(seed)`` (seed 0 by
default): int4 weights are uniform packed bytes (both nibbles uniform in
0..15), int8 weights uniform in [-127, 127], activations N(0, 1), scales
uniform in the configuration's range.
"""

from __future__ import annotations

import numpy as np


def int4_weights(rng, N, K):
    return rng.integers(0, 256, size=(N, K // 2), dtype=np.uint8)


def int8_weights(rng, N, K):
    return rng.integers(-127, 128, size=(N, K), dtype=np.int8)


def scales(rng, N, num_scales, lo, hi, dtype=np.float16):
    return rng.uniform(lo, hi, size=(N, num_scales)).astype(dtype)


def activations(rng, M, K, dtype=np.float16):
    return rng.standard_normal((M, K), dtype=np.float32).astype(dtype)


def matvec_case(wbits, M, N, K, G, lo, hi, x_dtype=np.float16, s_dtype=np.float16, seed=0):
    """(X [M,K], W, S [N,K/G]) for a dequant-matmul configuration."""
    rng = np.random.default_rng(seed)
    X = activations(rng, M, K, x_dtype)
    W = int4_weights(rng, N, K) if wbits == 4 else int8_weights(rng, N, K)
    S = scales(rng, N, K // G, lo, hi, s_dtype)
    return X, W, S


def dequant_case(wbits, N, K, G, lo, hi, s_dtype=np.float16, seed=0):
    rng = np.random.default_rng(seed)
    W = int4_weights(rng, N, K) if wbits == 4 else int8_weights(rng, N, K)
    S = scales(rng, N, K // G, lo, hi, s_dtype)
    return W, S


# The BASELINE configurations.
CFG1 = dict(wbits=8, M=4, N=512, K=512, G=512, lo=0.005, hi=0.02,
            x_dtype=np.float32, s_dtype=np.float32)                    # W8A32, fp32
CFG2 = dict(wbits=4, N=4096, K=4096, G=32, lo=0.001, hi=0.01)          # dequant int4
CFG3 = dict(wbits=4, N=11008, K=4096, G=128, lo=0.001, hi=0.01)        # GEMV W4A16 (M = 1, 4, 16)
CFG4 = dict(wbits=8, M=64, N=14336, K=4096, G=4096, lo=0.002, hi=0.02)  # W8A16 M = 64
CFG5A = dict(wbits=4, M=2048, N=4096, K=4096, G=128, lo=0.001, hi=0.01)  # prefill GEMM

# SmolLM2-135M decode linear stack (hidden 576, intermediate 1536), int4 G=32, M=1:
# per layer (N, K) of q, k, v, o, gate, up, down.
SMOLLM2_LAYER = [(576, 576), (192, 576), (192, 576), (576, 576),
                 (1536, 576), (1536, 576), (576, 1536)]
SMOLLM2_LAYERS = 30
