"""GPU weight producers with the reference's quantizer signatures.

``quantize_int4(weights, group_size=32)`` and ``quantize_int8`` follow
examples/38_quantized_matmul.py:248-291, ``quantize_int4_ref`` follows
examples/52_dequantize.py:110-126: float weights [N, K] in, ``(packed or
int8 weights, float32 scales)`` out, bit-identical to the reference's NumPy
results.  The work runs as one HIP launch (``locomp_amd_quantize_int4/8``).

Inputs may be host arrays (float32 / float16) or device ``Tensor``s
(float32 / float16 / bfloat16).  With ``as_tensors=True`` the results stay on
the device (as ``Tensor``s), ready for the dequant-matmul kernels.
"""

from __future__ import annotations

import numpy as np

from . import _lib
from .kernels import _current_stream
from .tensor import Tensor, code_of, empty, tensor


def _input(weights):
    if isinstance(weights, Tensor):
        if len(weights.shape) != 2:
            raise ValueError(f"weights must be [N, K], got {weights.shape}")
        return weights, weights.shape
    arr = np.asarray(weights)
    if arr.ndim != 2:
        raise ValueError(f"weights must be [N, K], got {arr.shape}")
    if arr.dtype not in (np.float32, np.float16):
        arr = arr.astype(np.float32)
    return tensor(np.ascontiguousarray(arr)), arr.shape


def _run(fn_name, mode_args, weights, group_size, qshape, qdtype, as_tensors):
    W, (N, K) = _input(weights)
    if group_size <= 0 or K % group_size:
        raise ValueError(f"K={K} must be a multiple of group_size={group_size}")
    Q = empty(qshape(N, K), qdtype)
    S = empty((N, K // group_size), np.float32)
    lib = _lib.load()
    rc = getattr(lib, fn_name)(W.data_ptr, Q.data_ptr, S.data_ptr, N, K, group_size, *mode_args,
                               code_of(W.dtype), _current_stream())
    _lib.check(rc, fn_name)
    if as_tensors:
        return Q, S
    return Q.numpy(), S.numpy()


def quantize_int4(weights, group_size=32, as_tensors=False):
    """INT4 symmetric per-group quantizer of examples/38_quantized_matmul.py:248-271.
    Returns (packed uint8 [N, K//2], scales float32 [N, K//G])."""
    return _run("locomp_amd_quantize_int4", (_lib.QUANT_EX38,), weights, group_size,
                lambda n, k: (n, k // 2), np.uint8, as_tensors)


def quantize_int4_ref(w, group_size=32, as_tensors=False):
    """INT4 quantizer of examples/52_dequantize.py:110-126 (1e-10 floor and bias)."""
    return _run("locomp_amd_quantize_int4", (_lib.QUANT_EX52,), w, group_size,
                lambda n, k: (n, k // 2), np.uint8, as_tensors)


def quantize_int8(weights, group_size=32, as_tensors=False):
    """INT8 symmetric per-group quantizer of examples/38_quantized_matmul.py:274-291.
    Returns (int8 [N, K], scales float32 [N, K//G])."""
    return _run("locomp_amd_quantize_int8", (), weights, group_size, lambda n, k: (n, k),
                np.int8, as_tensors)
