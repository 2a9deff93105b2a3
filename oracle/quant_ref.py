"""CPU oracle for locomp's quantized-inference path (int4 / int8 weight-only).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker / the timed CPU baseline.  The product path (``locomp_amd``) never
imports it and has no CPU fallback.

Every function restates the reference's NumPy code (Zyora-Dev/locomp v1.0.0)
and cites the file:line it follows.  The reference computes in fp32 with fp32
scales and activations; the BASELINE configurations add fp16 (and bf16)
activations, scales and outputs.  The generalisation keeps the reference's
fp32 intermediate: the dequantised weight is formed as
``float32(q - 8) * float32(s)`` and only the final result is cast to the
output dtype (round-to-nearest-even), exactly as ``astype`` does.

Pinning (how each function is checked independently of its own formula; the
tests live in ``tests/test_oracle.py``):

* ``unpack_int4`` / ``dequant_int4_ref`` / ``dequant_int8_ref``: exhaustive
  256-byte x scale table against the scalar definition of the reference
  kernel loop (examples/52_dequantize.py:36-53), closed forms (q=8 -> +0.0,
  linearity in s, low nibble = even k), a swapped-nibble layout that must
  fail, and the brute-force loop restatement ``numpy_matvec_int4`` below.
* ``fast_numpy_matvec_int4/int8``: float64 brute force over the reference's
  own loop definition (examples/38_quantized_matmul.py:178-212) on small
  shapes; special cases (all q=8 -> Y=0, single non-zero group -> textbook
  dot product, G=K -> per-channel).
* ``quantize_*``: round trip dequant(quantize(w)) within s/2 per element and
  ties-to-even on constructed halfway inputs.
* ``rms_norm_ref`` / ``residual_rms_norm_ref`` (the decode step around the
  linears): closed form on constant rows (c w / sqrt(c^2 + eps)), a float64
  scalar loop over the reference kernel's own loops, invariance of the
  output under scaling the row when eps = 0, and the residual add as a
  separate sum.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "f32_to_bf16_bits", "bf16_bits_to_f32", "cast_out",
    "unpack_int4", "dequant_int4_ref", "dequant_int8_ref",
    "numpy_matvec_int4", "numpy_matvec_int8",
    "fast_numpy_matvec_int4", "fast_numpy_matvec_int8",
    "quantize_int4", "quantize_int8", "quantize_int4_ref",
    "rms_norm_ref", "residual_rms_norm_ref",
]


# ---------------------------------------------------------------------------
# bf16 helpers (NumPy has no bfloat16): bf16 is kept as its uint16 bit pattern.
# ---------------------------------------------------------------------------

def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 with round-to-nearest-even, returned as uint16 bits."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    r = np.where(nan, (u >> 16) | 0x40, r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def _as_f32(a: np.ndarray, dtype: str | None = None) -> np.ndarray:
    """Promote a scale / activation array to fp32 (bf16 given as uint16 bits)."""
    if dtype == "bf16" or (dtype is None and a.dtype == np.uint16):
        return bf16_bits_to_f32(a)
    return np.asarray(a).astype(np.float32)


def cast_out(y32: np.ndarray, out_dtype: str) -> np.ndarray:
    """Final cast of an fp32 result, as ``astype`` does (RNE)."""
    if out_dtype == "f32":
        return y32.astype(np.float32)
    if out_dtype == "f16":
        return y32.astype(np.float16)
    if out_dtype == "bf16":
        return f32_to_bf16_bits(y32)
    raise ValueError(out_dtype)


# ---------------------------------------------------------------------------
# Dequantize
# ---------------------------------------------------------------------------

def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """uint8 [N, K/2] -> float32 [N, K] of (q - 8), low nibble at even k.

    Follows examples/38_quantized_matmul.py:220-226 (and
    examples/52_dequantize.py:131-136): low nibble -> k = 2j, high -> 2j + 1.
    """
    p = np.asarray(packed, dtype=np.uint8)
    n, half_k = p.shape
    low = (p.astype(np.int32) & 0xF).astype(np.float32) - 8.0
    high = (p.astype(np.int32) >> 4).astype(np.float32) - 8.0
    w = np.empty((n, 2 * half_k), dtype=np.float32)
    w[:, 0::2] = low
    w[:, 1::2] = high
    return w


def dequant_int4_ref(packed, scales, N, K, group_size=32, scale_dtype=None):
    """fp32 [N, K] dequantised weights.

    Follows examples/52_dequantize.py:129-143: unpack, then multiply each
    group of ``group_size`` columns by ``scales[:, g]`` in fp32.
    """
    w = unpack_int4(np.asarray(packed).reshape(N, K // 2))
    s = _as_f32(np.asarray(scales).reshape(N, K // group_size), scale_dtype)
    for g in range(K // group_size):
        w[:, g * group_size:(g + 1) * group_size] *= s[:, g:g + 1]
    return w


def dequant_int8_ref(w_int8, scales, N, K, group_size=32, scale_dtype=None):
    """fp32 [N, K]: ``w_int8.astype(float32) * repeat(scales, G)``.

    Follows the int8 formula of examples/52_dequantize.py:166 (the kernel
    body examples/52_dequantize.py:67-74 computes the same per element).
    """
    w = np.asarray(w_int8, dtype=np.int8).reshape(N, K).astype(np.float32)
    s = _as_f32(np.asarray(scales).reshape(N, K // group_size), scale_dtype)
    return w * np.repeat(s, group_size, axis=1)[:, :K]


# ---------------------------------------------------------------------------
# Dequant-matvec / matmul
# ---------------------------------------------------------------------------

def numpy_matvec_int4(x, w_packed, scales, group_size=32):
    """Brute-force float64 loop of examples/38_quantized_matmul.py:178-199.

    The reference accumulates in a Python float (fp64); ``x`` may be [K] or
    [M, K].  Small shapes only.
    """
    x2 = np.atleast_2d(np.asarray(x, dtype=np.float64))
    N, half_k = w_packed.shape
    s = np.asarray(scales, dtype=np.float64)
    out = np.zeros((x2.shape[0], N), dtype=np.float64)
    for m in range(x2.shape[0]):
        for n_idx in range(N):
            acc = 0.0
            for byte_i in range(half_k):
                packed = int(w_packed[n_idx, byte_i])
                k_low, k_high = 2 * byte_i, 2 * byte_i + 1
                w_low = (float(packed & 0xF) - 8.0) * s[n_idx, k_low // group_size]
                w_high = (float(packed >> 4) - 8.0) * s[n_idx, k_high // group_size]
                acc += x2[m, k_low] * w_low + x2[m, k_high] * w_high
            out[m, n_idx] = acc
    return out if np.ndim(x) == 2 else out[0]


def numpy_matvec_int8(x, w_int8, scales, group_size=32):
    """Brute-force float64 loop of examples/38_quantized_matmul.py:202-212."""
    x2 = np.atleast_2d(np.asarray(x, dtype=np.float64))
    N, K = w_int8.shape
    s = np.asarray(scales, dtype=np.float64)
    out = np.zeros((x2.shape[0], N), dtype=np.float64)
    for m in range(x2.shape[0]):
        for n_idx in range(N):
            acc = 0.0
            for k in range(K):
                acc += x2[m, k] * (float(w_int8[n_idx, k]) * s[n_idx, k // group_size])
            out[m, n_idx] = acc
    return out if np.ndim(x) == 2 else out[0]


def fast_numpy_matvec_int4(x, w_packed, scales, group_size=32, x_dtype=None, scale_dtype=None):
    """fp32 ``W_deq @ x`` (x [K]) or ``X @ W_deq.T`` (X [M, K]).

    Follows examples/38_quantized_matmul.py:215-232: fp32 dequantised
    intermediate, then one BLAS product.  Activations are promoted to fp32.
    Returns fp32; the caller casts with ``cast_out``.
    """
    N, half_k = w_packed.shape
    K = 2 * half_k
    w_full = unpack_int4(w_packed)
    s = _as_f32(scales, scale_dtype)
    w_dequant = w_full * np.repeat(s, group_size, axis=1)[:, :K]
    xf = _as_f32(x, x_dtype)
    if xf.ndim == 1:
        return w_dequant @ xf
    return xf @ w_dequant.T


def fast_numpy_matvec_int8(x, w_int8, scales, group_size=32, x_dtype=None, scale_dtype=None):
    """Follows examples/38_quantized_matmul.py:235-241, generalised to [M, K]."""
    N, K = w_int8.shape
    w_float = np.asarray(w_int8, dtype=np.int8).astype(np.float32)
    s = _as_f32(scales, scale_dtype)
    w_dequant = w_float * np.repeat(s, group_size, axis=1)[:, :K]
    xf = _as_f32(x, x_dtype)
    if xf.ndim == 1:
        return w_dequant @ xf
    return xf @ w_dequant.T


# ---------------------------------------------------------------------------
# Weight producers (off the measured path; used by round-trip tests)
# ---------------------------------------------------------------------------

def quantize_int4(weights, group_size=32):
    """Follows examples/38_quantized_matmul.py:248-271 (per-group amax/7)."""
    N, K = weights.shape
    assert K % group_size == 0
    G = K // group_size
    wg = np.asarray(weights, dtype=np.float32).reshape(N, G, group_size)
    amax = np.abs(wg).max(axis=2)
    scales = np.where(amax > 0, amax / np.float32(7.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round(wg / scales[:, :, None]) + 8, 0, 15).astype(np.uint8).reshape(N, K)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, scales


def quantize_int8(weights, group_size=32):
    """Follows examples/38_quantized_matmul.py:274-291 (per-group amax/127)."""
    N, K = weights.shape
    assert K % group_size == 0
    G = K // group_size
    wg = np.asarray(weights, dtype=np.float32).reshape(N, G, group_size)
    amax = np.abs(wg).max(axis=2)
    scales = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.round(wg / scales[:, :, None]), -128, 127).astype(np.int8).reshape(N, K)
    return q, scales


def quantize_int4_ref(w, group_size=32):
    """Follows examples/52_dequantize.py:110-126 (1e-10 floor and 1e-10 bias)."""
    N, K = w.shape
    assert K % group_size == 0
    G = K // group_size
    wg = np.asarray(w, dtype=np.float32).reshape(N, G, group_size)
    absmax = np.maximum(np.abs(wg).max(axis=2, keepdims=True), 1e-10)
    scales = absmax.reshape(N, G) / 7.0
    q = np.round(wg / (scales.reshape(N, G, 1) + 1e-10)) + 8
    q = np.clip(q, 0, 15).astype(np.uint8).reshape(N, K)
    packed = (q[:, 1::2] << 4) | q[:, 0::2]
    return packed.astype(np.uint8), scales.astype(np.float32)


# ---------------------------------------------------------------------------
# The decode step around the quantized linears (SmolLM2, examples/54).
# ---------------------------------------------------------------------------

def rms_norm_ref(x, w, eps=1e-5):
    """Per row: out = x * rsqrt(sum(x^2) / N + eps) * w, in fp32
    (examples/54_smollm2_inference.py:40-73: sum of squares at :49-51,
    rsqrt(total / N + eps) at :65, val * rms * w at :73)."""
    x = np.asarray(x, np.float32)
    ss = np.sum(x * x, axis=-1, keepdims=True, dtype=np.float32)
    rms = (np.float32(1.0) / np.sqrt(ss / np.float32(x.shape[-1]) + np.float32(eps))).astype(np.float32)
    return (x * rms * np.asarray(w, np.float32)).astype(np.float32)


def residual_rms_norm_ref(h, r, w, eps=1e-5, dtype=np.float32):
    """The hidden-state update and norm between two linears of the decode
    step: h += r (examples/54:164-167, the residual adds at :538 and :554)
    stored in the activation dtype, then rms_norm_ref of the stored h.
    Returns (new h, normed output), both in `dtype`."""
    h32 = np.asarray(h, np.float32)
    if r is not None:
        h32 = h32 + np.asarray(r, np.float32)
    h_new = h32.astype(dtype)
    y = rms_norm_ref(h_new.astype(np.float32), np.asarray(w, dtype).astype(np.float32), eps)
    return h_new, y.astype(dtype)
