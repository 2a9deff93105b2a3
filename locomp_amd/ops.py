"""Host wrappers with the signatures of locomp's quantized-path helpers.

``gpu_matvec_int4/int8`` follow examples/38_quantized_matmul.py:141-171 and
``gpu_dequant_int4/int8`` follow examples/52_dequantize.py:81-107: they take
host arrays, upload, launch and return host arrays.  Differences from the
reference, all widening: ``x`` may be [K] or [M, K]; K only has to be a
multiple of GROUP_SIZE (and even for int4) instead of 256 / 128; the output
dtype defaults to the activation dtype (fp32 for the reference's fp32
inputs) and can be set with ``out_dtype``.
"""

from __future__ import annotations

import numpy as np

from . import kernels as _k
from .tensor import Tensor, bfloat16, empty, tensor


def _float_dtype_of(a):
    if isinstance(a, Tensor):
        return a.dtype
    d = np.asarray(a).dtype
    return d if d in (np.float16, np.float32) else np.dtype(np.float32)


def _as_dev(a, dtype=None):
    if isinstance(a, Tensor):
        return a
    arr = np.asarray(a)
    if dtype is not None:
        arr = arr.astype(dtype)
    return tensor(np.ascontiguousarray(arr))


def gpu_matvec_int4(x, w_packed, scales, group_size=32, out_dtype=None):
    """INT4 quantized matvec. x: [K] or [M, K]; w_packed: [N, K//2] uint8; scales: [N, K//G]."""
    K = x.shape[-1]
    N = w_packed.shape[0]
    if K % group_size or K % 2:
        raise ValueError(f"K={K} must be even and a multiple of group_size={group_size}")
    M = 1 if len(x.shape) == 1 else x.shape[0]
    xd = _float_dtype_of(x)
    X_g = _as_dev(x, None if isinstance(x, Tensor) else xd)
    W_g = _as_dev(w_packed, np.uint8)
    S_g = _as_dev(scales)
    O_g = empty((M, N) if len(x.shape) == 2 else (N,), out_dtype or xd)
    _k.dequant_matvec_int4[(N,), (128,)](X_g, W_g, S_g, O_g, K, K // 2, K // group_size, group_size)
    return O_g.numpy()


def gpu_matvec_int8(x, w_int8, scales, group_size=32, out_dtype=None):
    """INT8 quantized matvec. x: [K] or [M, K]; w_int8: [N, K] int8; scales: [N, K//G]."""
    K = x.shape[-1]
    N = w_int8.shape[0]
    if K % group_size:
        raise ValueError(f"K={K} must be a multiple of group_size={group_size}")
    M = 1 if len(x.shape) == 1 else x.shape[0]
    xd = _float_dtype_of(x)
    X_g = _as_dev(x, None if isinstance(x, Tensor) else xd)
    W_g = _as_dev(w_int8, np.int8)
    S_g = _as_dev(scales)
    O_g = empty((M, N) if len(x.shape) == 2 else (N,), out_dtype or xd)
    _k.dequant_matvec_int8[(N,), (128,)](X_g, W_g, S_g, O_g, K, K // group_size, group_size)
    return O_g.numpy()


def gpu_dequant_int4(w_packed, scales, N, K, group_size=32, out_dtype=np.float32):
    """Dequantize INT4 packed weights. w_packed: [N, K//2] uint8; scales: [N, K//G] -> [N, K]."""
    W_g = _as_dev(np.asarray(w_packed).reshape(-1), np.uint8)
    S_g = _as_dev(np.asarray(scales).reshape(-1))
    O_g = empty(N * K, out_dtype)
    _k.dequant_int4[(N,), (128,)](W_g, S_g, O_g, K, K // 2, K // group_size, group_size)
    result = O_g.numpy().reshape(N, K)
    W_g.free(); S_g.free(); O_g.free()
    return result


def gpu_dequant_int8(w_int8, scales, N, K, group_size=32, out_dtype=np.float32):
    """Dequantize INT8 weights. w_int8: [N, K] int8; scales: [N, K//G] -> [N, K]."""
    W_g = _as_dev(np.asarray(w_int8).reshape(-1), np.int8)
    S_g = _as_dev(np.asarray(scales).reshape(-1))
    O_g = empty(N * K, out_dtype)
    _k.dequant_int8[(N,), (128,)](W_g, S_g, O_g, K, K // group_size, group_size)
    result = O_g.numpy().reshape(N, K)
    W_g.free(); S_g.free(); O_g.free()
    return result


def interleave_gate_up(gate, up):
    """Rows of two [I, ...] arrays interleaved into [2I, ...] (gate_i, up_i, ...):
    the weight / scale layout of ``gpu_matvec_int4_silu_mul``."""
    gate, up = np.asarray(gate), np.asarray(up)
    if gate.shape != up.shape:
        raise ValueError(f"gate {gate.shape} and up {up.shape} differ")
    out = np.empty((2 * gate.shape[0],) + gate.shape[1:], gate.dtype)
    out[0::2] = gate
    out[1::2] = up
    return out


def gpu_matvec_int4_silu_mul(x, w_gate_up, scales, group_size=32, out_dtype=None):
    """silu(x @ deq(W_gate)^T) * (x @ deq(W_up)^T) in one launch.

    ``w_gate_up`` / ``scales``: gate and up rows interleaved ([2I, K//2] uint8,
    [2I, K//G]; see ``interleave_gate_up``); x: [K] or [M, K] -> [I] or [M, I].
    Replaces examples/54_smollm2_inference.py:545-548 (two matvecs and
    silu_mul_kernel, :113-120)."""
    from . import _lib
    from .kernels import _current_stream
    from .tensor import code_of
    K = x.shape[-1]
    N2 = w_gate_up.shape[0]
    if K % group_size or K % 2 or N2 % 2:
        raise ValueError(f"K={K} must be even and a multiple of group_size={group_size}; "
                         f"rows={N2} must be even")
    I = N2 // 2
    M = 1 if len(x.shape) == 1 else x.shape[0]
    xd = _float_dtype_of(x)
    X_g = _as_dev(x, None if isinstance(x, Tensor) else xd)
    W_g = _as_dev(w_gate_up, np.uint8)
    S_g = _as_dev(scales)
    O_g = empty((M, I) if len(x.shape) == 2 else (I,), out_dtype or xd)
    rc = _lib.load().locomp_amd_dequant_matvec_int4_silu_mul(
        X_g.data_ptr, W_g.data_ptr, S_g.data_ptr, O_g.data_ptr, K, K // 2, K // group_size,
        group_size, I, M, code_of(X_g.dtype), code_of(S_g.dtype), code_of(O_g.dtype),
        _current_stream())
    _lib.check(rc, "dequant_matvec_int4_silu_mul")
    return O_g.numpy()
