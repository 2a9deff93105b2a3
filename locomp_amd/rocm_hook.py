"""The binding a locomp maintainer adds to the reference's ROCm launch path.

locomp runs every ``kernel[grid, block](...)`` on ROCm through
``_KernelCall._launch_rocm`` (locomp/api.py:858-994): it splits the call into
pointer arguments and constexpr values (api.py:872-885), generates and
compiles ``locomp_launch_<name>`` per constexpr specialization, uploads host
arguments (``np.ndarray`` / ``LocompTensor``) to temporaries (api.py:966-983)
and calls the launcher with their device pointers.  One call at the top of
that function routes the quantized kernels here instead::

    from locomp_amd.rocm_hook import try_launch
    if try_launch(self.launcher.func_name, self.grid, self.threadgroup_size,
                  tensor_args, constexpr_values):
        return

``try_launch`` returns False for any other kernel (codegen proceeds as
before).  For the quantized kernels it takes the same argument kinds as
``_launch_rocm`` -- ``ROCmTensor`` (``._hip_ptr``, ``.dtype``, ``.size``),
``np.ndarray``, ``LocompTensor`` (``.data``) -- validates them like the
reference's wrappers would (sizes against the grid and the constexprs), and
launches through the library's ``locomp_amd_launch`` entry, which follows the
generated launchers' convention (``args[i]`` = device pointer of the i-th
pointer parameter).  Unlike ``_launch_rocm``, which frees host-argument
uploads without copying them back (so a host output array is never written,
api.py:977-994), outputs given as host arrays are copied back.  The launch is
synchronous, like the reference's (api.py:991).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib, kernels
from .kernels import ArgInfo

# kernel name -> (validator kernel, integer parameter names in signature
# order, position of the activation row count M in the validator's result)
KERNELS = {
    "dequant_int4": (kernels.dequant_int4, ("K", "HALF_K", "NUM_SCALES", "GROUP_SIZE"), None),
    "dequant_int8": (kernels.dequant_int8, ("K", "NUM_SCALES", "GROUP_SIZE"), None),
    "dequant_matvec_int4": (kernels.dequant_matvec_int4,
                            ("K_dim", "HALF_K", "NUM_SCALES", "GROUP_SIZE"), 5),
    "dequant_matvec_int8": (kernels.dequant_matvec_int8, ("K_dim", "NUM_SCALES", "GROUP_SIZE"), 4),
    "quant_matvec_int8": (kernels.dequant_matvec_int8, ("K_dim", "NUM_SCALES", "GROUP_SIZE"), 4),
}


def _default_upload(a: np.ndarray):
    from .tensor import tensor
    return tensor(np.ascontiguousarray(a))


def _arg_info(a):
    """(ArgInfo, host ndarray or None) for one pointer argument."""
    if hasattr(a, "_hip_ptr"):                      # the reference's ROCmTensor
        return ArgInfo(int(a.size), np.dtype(a.dtype)), None
    if isinstance(a, np.ndarray):
        return ArgInfo(int(a.size), a.dtype), a
    data = getattr(a, "data", None)                 # the reference's LocompTensor
    if isinstance(data, np.ndarray):
        return ArgInfo(int(data.size), data.dtype), data
    raise TypeError(f"Unsupported argument type for ROCm backend: {type(a)}")


def try_launch(func_name, grid, threadgroup_size, tensor_args, constexpr_values, *,
               lib=None, upload=_default_upload, sync=None) -> bool:
    """Run one of the quantized kernels on the library; False if `func_name`
    is not one of them.  ``lib`` / ``upload`` / ``sync`` replace the loaded
    library, the host-to-device upload and the final synchronisation (tests
    drive the argument mapping with stand-ins, no GPU)."""
    entry = KERNELS.get(func_name)
    if entry is None:
        return False
    kern, int_names, m_at = entry
    grid = tuple(grid) if isinstance(grid, (tuple, list)) else (grid,)
    args = list(tensor_args)
    if len(args) != len(kern._ptr_names):
        raise TypeError(f"{func_name} takes {len(kern._ptr_names)} pointer arguments "
                        f"({', '.join(kern._ptr_names)}), got {len(args)}")
    missing = [n for n in int_names if n not in constexpr_values]
    if missing:
        raise TypeError(f"{func_name}: missing constexpr value(s) {', '.join(missing)}")
    ints = [constexpr_values[n] for n in int_names]
    infos, hosts = zip(*(_arg_info(a) for a in args))
    n = kernels._check_grid(grid, tuple(threadgroup_size) if threadgroup_size else None)
    # sizes / dtypes as the wrappers check them (M = X.size / K, exactly)
    planned = kern._planner(n, *infos, *ints)
    m = planned[m_at] if m_at is not None else 1
    lib = lib if lib is not None else _lib.load()
    # `keep` holds every upload until the launch has finished: a temporary
    # dropped earlier returns its memory to the allocator, and the next
    # upload could land in it
    dev, back, keep = [], [], []
    for i, (a, h) in enumerate(zip(args, hosts)):
        if h is None:
            dev.append(int(a._hip_ptr))
            continue
        t = upload(h)
        keep.append(t)
        dev.append(int(t.data_ptr))
        if i in kern._outputs:
            back.append((h, t))
    arr = (ctypes.c_void_p * len(dev))(*dev)
    cx = (ctypes.c_int64 * len(ints))(*[int(v) for v in ints])
    dts = (ctypes.c_int * len(infos))(*[
        _lib.F32 if inf.dtype in (np.dtype(np.int8), np.dtype(np.uint8)) else
        kernels.code_of(inf.dtype) for inf in infos])
    bx = tuple(threadgroup_size) if threadgroup_size else (128,)
    rc = lib.locomp_amd_launch(func_name.encode(), n, 1, int(bx[0]),
                               int(bx[1]) if len(bx) > 1 else 1,
                               ctypes.cast(arr, ctypes.POINTER(ctypes.c_void_p)), cx, len(ints),
                               dts, m, None)
    _lib.check(rc, func_name)
    for h, t in back:
        h[...] = t.numpy().reshape(h.shape)
    if sync is not None:
        sync()
    else:
        import torch
        torch.cuda.synchronize()
    del keep
    return True
