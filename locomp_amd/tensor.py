"""Device-resident tensors with locomp's host-side surface.

Mirrors ``locomp.tensor / empty / zeros / ones`` (locomp/api.py:323-402) and
the tensor methods callers of the quantized path use: ``.numpy()``,
``.free()``, ``.shape``, ``.dtype``, ``.size`` (locomp/backends/
rocm_runtime.py:52-97, locomp/api.py:72-90, 267-320).  Memory comes from
PyTorch-ROCm's caching allocator on the current HIP device; ``.numpy()``
copies device -> host after the stream's queued work has finished.

Unlike the reference, creation always places data on the GPU (the
reference's ``backend="auto"`` never selects ROCm on Linux,
locomp/api.py:405-407, so its outputs were lost after the launch).

bfloat16 has no NumPy dtype: ``dtype=bfloat16`` tensors take float input
(rounded to nearest even) and ``.numpy()`` returns the raw uint16 bit
patterns.
"""

from __future__ import annotations

import numpy as np

from . import _lib


class _BF16Marker:
    """dtype marker for bfloat16 (locomp.BFloat16 parameters)."""

    name = "bfloat16"
    itemsize = 2

    def __repr__(self) -> str:
        return "locomp_amd.bfloat16"


bfloat16 = _BF16Marker()

_SUPPORTED = {np.dtype(np.float32), np.dtype(np.float16), np.dtype(np.int8),
              np.dtype(np.uint8), np.dtype(np.int32)}

_torch = None


def _t():
    global _torch
    if _torch is None:
        import torch
        _torch = torch
    return _torch


def _torch_dtype(dtype):
    torch = _t()
    if dtype is bfloat16:
        return torch.bfloat16
    return {
        np.dtype(np.float32): torch.float32, np.dtype(np.float16): torch.float16,
        np.dtype(np.int8): torch.int8, np.dtype(np.uint8): torch.uint8,
        np.dtype(np.int32): torch.int32,
    }[np.dtype(dtype)]


def _normalize_dtype(dtype):
    if dtype is bfloat16 or (isinstance(dtype, str) and dtype in ("bfloat16", "bf16")):
        return bfloat16
    d = np.dtype(dtype)
    if d == np.float64:            # locomp's LocompTensor keeps float64 host data;
        d = np.dtype(np.float32)   # no kernel on this path reads fp64
    if d not in _SUPPORTED:
        raise TypeError(f"unsupported dtype {d}")
    return d


def code_of(dtype) -> int:
    """Library dtype code of a float dtype (raises for non-float dtypes)."""
    if dtype is bfloat16:
        return _lib.BF16
    d = np.dtype(dtype)
    if d == np.float32:
        return _lib.F32
    if d == np.float16:
        return _lib.F16
    raise TypeError(f"{d} is not a float dtype accepted here")


def _device():
    torch = _t()
    if not torch.cuda.is_available():
        raise RuntimeError("locomp_amd needs a HIP device (MI355X); none is visible")
    return torch.device("cuda", torch.cuda.current_device())


class Tensor:
    """A GPU-resident tensor (row-major, contiguous)."""

    __slots__ = ("_t", "_dtype", "_shape", "_freed")

    def __init__(self, t, dtype, shape):
        self._t = t
        self._dtype = dtype
        self._shape = tuple(int(s) for s in shape)
        self._freed = False

    # -- locomp surface -----------------------------------------------------
    @property
    def shape(self):
        return self._shape

    @property
    def size(self) -> int:
        n = 1
        for s in self._shape:
            n *= s
        return n

    @property
    def dtype(self):
        return self._dtype

    @property
    def ndim(self) -> int:
        return len(self._shape)

    @property
    def itemsize(self) -> int:
        return self._dtype.itemsize

    @property
    def nbytes(self) -> int:
        return self.size * self.itemsize

    def numpy(self) -> np.ndarray:
        """Copy to host (waits for queued work on the current stream)."""
        self._check_live()
        host = self._t.detach().to("cpu")
        if self._dtype is bfloat16:
            return host.view(_t().int16).numpy().view(np.uint16).reshape(self._shape).copy()
        return host.numpy().reshape(self._shape).copy()

    def free(self) -> None:
        """Release the device memory (idempotent)."""
        if not self._freed:
            self._t = None
            self._freed = True

    def reshape(self, *shape) -> "Tensor":
        if len(shape) == 1 and isinstance(shape[0], (tuple, list)):
            shape = tuple(shape[0])
        shape = list(shape)
        if shape.count(-1) > 1:
            raise ValueError("Only one -1 allowed in reshape")
        if -1 in shape:
            rest = 1
            for s in shape:
                if s != -1:
                    rest *= s
            shape[shape.index(-1)] = self.size // max(rest, 1)
        n = 1
        for s in shape:
            n *= s
        if n != self.size:
            raise ValueError(f"cannot reshape {self._shape} to {tuple(shape)}")
        self._check_live()
        return Tensor(self._t, self._dtype, shape)

    # -- interop ------------------------------------------------------------
    @property
    def data_ptr(self) -> int:
        self._check_live()
        return self._t.data_ptr()

    @property
    def torch(self):
        """The underlying torch tensor (flat, on the device)."""
        self._check_live()
        return self._t

    @classmethod
    def from_torch(cls, t, dtype=None) -> "Tensor":
        torch = _t()
        if not t.is_cuda:
            raise ValueError("tensor must be on the HIP device")
        t = t.contiguous()
        if dtype is None:
            dtype = bfloat16 if t.dtype == torch.bfloat16 else np.dtype(
                str(t.dtype).replace("torch.", ""))
        return cls(t.reshape(-1), dtype, tuple(t.shape))

    def _check_live(self):
        if self._freed:
            raise RuntimeError("tensor has been freed")

    def __repr__(self) -> str:
        return f"locomp_amd.Tensor(shape={self._shape}, dtype={self._dtype})"


def _upload(arr: np.ndarray, dtype) -> Tensor:
    torch = _t()
    dev = _device()
    if dtype is bfloat16:
        src = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32))
        t = src.to(torch.bfloat16).reshape(-1).to(dev)
    else:
        t = torch.from_numpy(np.ascontiguousarray(arr)).reshape(-1).to(dev)
    return Tensor(t, dtype, arr.shape)


def tensor(data, dtype=np.float32, backend: str = "auto") -> Tensor:
    """Upload ``data`` (list, scalar or ndarray) to the device.

    As in locomp/api.py:323-339, an ndarray keeps its own dtype and other
    data is converted to ``dtype``; ``backend`` is accepted for signature
    compatibility (only the HIP device exists here).
    """
    if isinstance(data, Tensor):
        return data
    if dtype is bfloat16 or dtype in ("bfloat16", "bf16"):
        return _upload(np.asarray(data, dtype=np.float32), bfloat16)
    arr = data if isinstance(data, np.ndarray) else np.asarray(data, dtype=dtype)
    d = _normalize_dtype(arr.dtype)
    return _upload(arr.astype(d, copy=False), d)


def _alloc(shape, dtype, fill):
    if isinstance(shape, int):
        shape = (shape,)
    d = _normalize_dtype(dtype)
    torch = _t()
    n = 1
    for s in shape:
        n *= int(s)
    td = _torch_dtype(d)
    dev = _device()
    if fill is None:
        t = torch.empty(n, dtype=td, device=dev)
    else:
        t = torch.full((n,), fill, dtype=td, device=dev)
    return Tensor(t, d, shape)


def empty(shape, dtype=np.float32, backend: str = "auto") -> Tensor:
    """Uninitialised device tensor (locomp/api.py:342-364)."""
    return _alloc(shape, dtype, None)


def zeros(shape, dtype=np.float32, backend: str = "auto") -> Tensor:
    """Zero-filled device tensor (locomp/api.py:367-389)."""
    return _alloc(shape, dtype, 0)


def ones(shape, dtype=np.float32, backend: str = "auto") -> Tensor:
    """One-filled device tensor (locomp/api.py:392-402)."""
    return _alloc(shape, dtype, 1)
