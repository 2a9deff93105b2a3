"""Kernel objects with locomp's launch syntax: ``kernel[(gx,), (bx,)](*args)``.

The four kernels of locomp's quantized path are exposed under their
reference names and positional signatures:

=====================  ==============================================  ======================================
kernel                 positional arguments                            reference
=====================  ==============================================  ======================================
dequant_int4           W, SCALES, OUT, K, HALF_K, NUM_SCALES, GROUP_SIZE       examples/52_dequantize.py:27-53
dequant_int8           W, SCALES, OUT, K, NUM_SCALES, GROUP_SIZE               examples/52_dequantize.py:60-74
dequant_matvec_int4    X, W, scales, O, K_dim, HALF_K, NUM_SCALES, GROUP_SIZE  examples/38_quantized_matmul.py:30-87
dequant_matvec_int8    X, W, scales, O, K_dim, NUM_SCALES, GROUP_SIZE          examples/38_quantized_matmul.py:94-134
=====================  ==============================================  ======================================

``dequant_matmul_int4`` / ``dequant_matmul_int8`` are the same launches
under GEMM names (X holds M rows).  The grid's first extent is the number of
weight rows N, as in the reference (grid ``(N,)``, locomp/api.py:480-487);
the block shape is validated and otherwise ignored, because each kernel picks
its own gfx950 launch geometry.  The activation row count M is X.size / K
(the reference only has M = 1).  Float parameters take fp32, fp16 or bf16
(locomp.Tensor / Float16 / BFloat16); the library computes
float32(q - 8) * float32(s) and rounds once to O's dtype.

Argument errors raise before anything is launched: ``TypeError`` for a wrong
dtype, ``ValueError`` for inconsistent sizes (the reference raises
``AssertionError`` in its wrappers, examples/38_quantized_matmul.py:145,162).
Launches are asynchronous on the current HIP stream; ``Tensor.numpy()``
waits.  Host ``numpy`` arguments are uploaded to temporaries and an output
given as a host array is copied back after the launch.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _lib
from .tensor import Tensor, bfloat16, code_of, tensor as _to_device

_FLOAT = "float"
_U8 = "u8"
_I8 = "i8"


@dataclass(frozen=True)
class ArgInfo:
    """Size and dtype of a pointer argument (what validation looks at)."""
    size: int
    dtype: object


def _info(a) -> ArgInfo:
    if isinstance(a, Tensor):
        return ArgInfo(a.size, a.dtype)
    if isinstance(a, np.ndarray):
        return ArgInfo(int(a.size), a.dtype)
    try:
        import torch
        if isinstance(a, torch.Tensor):
            d = bfloat16 if a.dtype == torch.bfloat16 else np.dtype(str(a.dtype).replace("torch.", ""))
            return ArgInfo(int(a.numel()), d)
    except ImportError:  # pragma: no cover
        pass
    raise TypeError(f"unsupported argument type {type(a).__name__}")


def _check_kind(name: str, info: ArgInfo, kind: str) -> None:
    d = info.dtype
    if kind == _U8:
        if d is bfloat16 or np.dtype(d) != np.uint8:
            raise TypeError(f"{name} must be uint8 (locomp.UInt8), got {d}")
    elif kind == _I8:
        if d is bfloat16 or np.dtype(d) != np.int8:
            raise TypeError(f"{name} must be int8 (locomp.Int8), got {d}")
    else:
        if d is not bfloat16 and np.dtype(d) not in (np.dtype(np.float32), np.dtype(np.float16)):
            raise TypeError(f"{name} must be float32, float16 or bfloat16, got {d}")


def _check_grid(grid, block) -> int:
    if not isinstance(grid, tuple) or len(grid) < 1:
        raise ValueError(f"grid must be a tuple (N,), got {grid!r}")
    for g in grid[1:]:
        if int(g) != 1:
            raise ValueError(f"grid must be (N,) (extra extents must be 1), got {grid!r}")
    n = int(grid[0])
    if n < 0:
        raise ValueError(f"grid extent must be >= 0, got {n}")
    if block is not None:
        bs = tuple(int(b) for b in block)
        total = 1
        for b in bs:
            if b <= 0:
                raise ValueError(f"block extents must be positive, got {block!r}")
            total *= b
        if total > 1024:
            raise ValueError(f"block of {total} threads exceeds 1024")
    return n


def _ints(vals, names):
    out = []
    for v, nm in zip(vals, names):
        if isinstance(v, bool) or int(v) != v:
            raise TypeError(f"{nm} must be an integer, got {v!r}")
        out.append(int(v))
    return out


# ----------------------------------------------------------- validation --
# Pure functions of sizes / dtypes: they return the integer arguments of the
# C entry point (everything but pointers and the stream).

def plan_dequant_int4(N, W, S, OUT, K, HALF_K, NUM_SCALES, GROUP_SIZE):
    K, HALF_K, NUM_SCALES, GROUP_SIZE = _ints((K, HALF_K, NUM_SCALES, GROUP_SIZE),
                                              ("K", "HALF_K", "NUM_SCALES", "GROUP_SIZE"))
    _check_kind("W", W, _U8); _check_kind("SCALES", S, _FLOAT); _check_kind("OUT", OUT, _FLOAT)
    if GROUP_SIZE <= 0 or K < 0 or HALF_K * 2 != K or NUM_SCALES * GROUP_SIZE != K:
        raise ValueError(f"need K == 2*HALF_K == NUM_SCALES*GROUP_SIZE, got K={K} HALF_K={HALF_K} "
                         f"NUM_SCALES={NUM_SCALES} GROUP_SIZE={GROUP_SIZE}")
    if W.size != N * HALF_K:
        raise ValueError(f"W has {W.size} bytes, expected N*HALF_K = {N * HALF_K}")
    if S.size != N * NUM_SCALES:
        raise ValueError(f"SCALES has {S.size} elements, expected {N * NUM_SCALES}")
    if OUT.size != N * K:
        raise ValueError(f"OUT has {OUT.size} elements, expected N*K = {N * K}")
    return [K, HALF_K, NUM_SCALES, GROUP_SIZE, N, code_of(S.dtype), code_of(OUT.dtype)]


def plan_dequant_int8(N, W, S, OUT, K, NUM_SCALES, GROUP_SIZE):
    K, NUM_SCALES, GROUP_SIZE = _ints((K, NUM_SCALES, GROUP_SIZE), ("K", "NUM_SCALES", "GROUP_SIZE"))
    _check_kind("W", W, _I8); _check_kind("SCALES", S, _FLOAT); _check_kind("OUT", OUT, _FLOAT)
    if GROUP_SIZE <= 0 or K < 0 or NUM_SCALES * GROUP_SIZE != K:
        raise ValueError(f"need K == NUM_SCALES*GROUP_SIZE, got K={K} NUM_SCALES={NUM_SCALES} "
                         f"GROUP_SIZE={GROUP_SIZE}")
    if W.size != N * K:
        raise ValueError(f"W has {W.size} elements, expected N*K = {N * K}")
    if S.size != N * NUM_SCALES:
        raise ValueError(f"SCALES has {S.size} elements, expected {N * NUM_SCALES}")
    if OUT.size != N * K:
        raise ValueError(f"OUT has {OUT.size} elements, expected N*K = {N * K}")
    return [K, NUM_SCALES, GROUP_SIZE, N, code_of(S.dtype), code_of(OUT.dtype)]


def _rows_of(X, O, K, N):
    if K == 0:
        if N == 0:
            return 0
        if O.size % N:
            raise ValueError(f"O has {O.size} elements, not a multiple of N={N}")
        return O.size // N
    if X.size % K:
        raise ValueError(f"X has {X.size} elements, not a multiple of K={K}")
    M = X.size // K
    if O.size != M * N:
        raise ValueError(f"O has {O.size} elements, expected M*N = {M}*{N}")
    return M


def plan_dequant_matvec_int4(N, X, W, S, O, K_dim, HALF_K, NUM_SCALES, GROUP_SIZE):
    K, HALF_K, NUM_SCALES, GROUP_SIZE = _ints((K_dim, HALF_K, NUM_SCALES, GROUP_SIZE),
                                              ("K_dim", "HALF_K", "NUM_SCALES", "GROUP_SIZE"))
    _check_kind("X", X, _FLOAT); _check_kind("W", W, _U8)
    _check_kind("scales", S, _FLOAT); _check_kind("O", O, _FLOAT)
    if GROUP_SIZE <= 0 or K < 0 or HALF_K * 2 != K or NUM_SCALES * GROUP_SIZE != K:
        raise ValueError(f"need K_dim == 2*HALF_K == NUM_SCALES*GROUP_SIZE, got K_dim={K} "
                         f"HALF_K={HALF_K} NUM_SCALES={NUM_SCALES} GROUP_SIZE={GROUP_SIZE}")
    if W.size != N * HALF_K:
        raise ValueError(f"W has {W.size} bytes, expected N*HALF_K = {N * HALF_K}")
    if S.size != N * NUM_SCALES:
        raise ValueError(f"scales has {S.size} elements, expected {N * NUM_SCALES}")
    M = _rows_of(X, O, K, N)
    return [K, HALF_K, NUM_SCALES, GROUP_SIZE, N, M, code_of(X.dtype), code_of(S.dtype),
            code_of(O.dtype)]


def plan_dequant_matvec_int8(N, X, W, S, O, K_dim, NUM_SCALES, GROUP_SIZE):
    K, NUM_SCALES, GROUP_SIZE = _ints((K_dim, NUM_SCALES, GROUP_SIZE),
                                      ("K_dim", "NUM_SCALES", "GROUP_SIZE"))
    _check_kind("X", X, _FLOAT); _check_kind("W", W, _I8)
    _check_kind("scales", S, _FLOAT); _check_kind("O", O, _FLOAT)
    if GROUP_SIZE <= 0 or K < 0 or NUM_SCALES * GROUP_SIZE != K:
        raise ValueError(f"need K_dim == NUM_SCALES*GROUP_SIZE, got K_dim={K} "
                         f"NUM_SCALES={NUM_SCALES} GROUP_SIZE={GROUP_SIZE}")
    if W.size != N * K:
        raise ValueError(f"W has {W.size} elements, expected N*K = {N * K}")
    if S.size != N * NUM_SCALES:
        raise ValueError(f"scales has {S.size} elements, expected {N * NUM_SCALES}")
    M = _rows_of(X, O, K, N)
    return [K, NUM_SCALES, GROUP_SIZE, N, M, code_of(X.dtype), code_of(S.dtype), code_of(O.dtype)]


# ------------------------------------------------------------- kernels --

class QuantKernel:
    """A fixed, hand-written kernel with locomp's ``[grid, block](...)`` call."""

    def __init__(self, name, c_name, ptr_names, n_ints, outputs, planner):
        self.__name__ = name
        self.func_name = name
        self._c_name = c_name
        self._ptr_names = ptr_names
        self._n_ints = n_ints
        self._outputs = outputs   # indices of output pointer args
        self._planner = planner

    @property
    def n_args(self) -> int:
        return len(self._ptr_names) + self._n_ints

    def __getitem__(self, grid):
        # Same forms as locomp/api.py:480-487.
        if isinstance(grid, tuple) and len(grid) == 2 and isinstance(grid[0], tuple):
            return _Launch(self, grid[0], grid[1])
        if not isinstance(grid, tuple):
            grid = (grid,)
        return _Launch(self, grid, None)

    def plan(self, grid, block, *args):
        """Validate and return the C entry's integer arguments (no launch)."""
        if len(args) != self.n_args:
            raise TypeError(f"{self.__name__} takes {self.n_args} positional arguments "
                            f"({', '.join(self._ptr_names)}, + {self._n_ints} ints), got {len(args)}")
        n = _check_grid(grid, block)
        np_ = len(self._ptr_names)
        infos = [_info(a) for a in args[:np_]]
        return self._planner(n, *infos, *args[np_:])

    def __repr__(self) -> str:
        return f"<locomp_amd kernel {self.__name__}>"


def _current_stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(a) -> int:
    if isinstance(a, Tensor):
        return a.data_ptr
    return a.data_ptr()  # torch tensor


class _Launch:
    def __init__(self, kernel: QuantKernel, grid, block):
        self.kernel = kernel
        self.grid = grid
        self.block = block

    def __call__(self, *args, **kwargs):
        k = self.kernel
        args = list(args) + list(kwargs.values())
        ints = k.plan(self.grid, self.block, *args)
        lib = _lib.load()
        np_ = len(k._ptr_names)
        dev_args = []
        copy_back = []
        for i, a in enumerate(args[:np_]):
            if isinstance(a, np.ndarray):
                t = _to_device(np.ascontiguousarray(a))
                dev_args.append(t)
                if i in k._outputs:
                    copy_back.append((a, t))
            else:
                if not isinstance(a, Tensor):
                    import torch
                    if not (isinstance(a, torch.Tensor) and a.is_cuda and a.is_contiguous()):
                        raise TypeError(f"{k._ptr_names[i]} must be a device tensor or ndarray")
                dev_args.append(a)
        ptrs = [ctypes.c_void_p(_ptr(a)) for a in dev_args]
        rc = getattr(lib, k._c_name)(*ptrs, *ints, _current_stream())
        _lib.check(rc, k.__name__)
        for host, dev in copy_back:
            host[...] = dev.numpy().reshape(host.shape)
        return None


dequant_int4 = QuantKernel("dequant_int4", "locomp_amd_dequant_int4",
                           ("W", "SCALES", "OUT"), 4, (2,), plan_dequant_int4)
dequant_int8 = QuantKernel("dequant_int8", "locomp_amd_dequant_int8",
                           ("W", "SCALES", "OUT"), 3, (2,), plan_dequant_int8)
dequant_matvec_int4 = QuantKernel("dequant_matvec_int4", "locomp_amd_dequant_matvec_int4",
                                  ("X", "W", "scales", "O"), 4, (3,), plan_dequant_matvec_int4)
dequant_matvec_int8 = QuantKernel("dequant_matvec_int8", "locomp_amd_dequant_matvec_int8",
                                  ("X", "W", "scales", "O"), 3, (3,), plan_dequant_matvec_int8)
# examples/58_benchmark_suite.py:241-264 defines the same int8 kernel under this name.
quant_matvec_int8 = dequant_matvec_int8
dequant_matmul_int4 = dequant_matvec_int4
dequant_matmul_int8 = dequant_matvec_int8
