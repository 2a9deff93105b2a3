"""The reference-side binding (locomp_amd.rocm_hook.try_launch, the call a
maintainer adds to locomp/api.py _launch_rocm) and the name-dispatched C entry
locomp_amd_launch, on the CPU: argument mapping with stand-in tensors, the
reference's host-argument kinds, validation, and the C entry's error codes
(nothing reaches a device)."""

import ctypes

import numpy as np
import pytest

from locomp_amd import _lib
from locomp_amd.rocm_hook import try_launch


class FakeROCmTensor:
    """Stand-in for locomp.backends.rocm_runtime.ROCmTensor (_hip_ptr, size, dtype)."""

    def __init__(self, ptr, size, dtype):
        self._hip_ptr, self.size, self.dtype = ptr, size, np.dtype(dtype)


class FakeLocompTensor:
    """Stand-in for locomp.api.LocompTensor (host data in .data)."""

    def __init__(self, data):
        self.data = data


class FakeLib:
    def __init__(self, rc=0):
        self.calls, self.rc = [], rc

    def locomp_amd_launch(self, name, gx, gy, bx, by, args, cx, ncx, dts, m, stream):
        n_ptr = {b"dequant_int4": 3, b"dequant_int8": 3}.get(name, 4)
        self.calls.append(dict(name=name.decode(), grid=(gx, gy), block=(bx, by),
                               ptrs=[args[i] for i in range(n_ptr)],
                               constexprs=[cx[i] for i in range(ncx)],
                               dtypes=[dts[i] for i in range(n_ptr)], m=m, stream=stream))
        return self.rc


class FakeDev:
    """What the upload stand-in returns: a device pointer and its readback."""

    def __init__(self, host, ptr):
        self.data_ptr, self._host = ptr, host

    def numpy(self):
        return np.full(self._host.shape, 7, self._host.dtype)


def _uploader():
    made = []

    def up(a):
        made.append(FakeDev(a, 0x9000 + 0x100 * len(made)))
        return made[-1]
    return up, made


def test_other_kernels_fall_through():
    lib = FakeLib()
    assert try_launch("softmax", (4,), (128,), [], {}, lib=lib) is False
    assert lib.calls == []


def test_matvec_int4_device_args_map_to_the_launcher_convention():
    K, N, G, M = 256, 8, 32, 3
    X = FakeROCmTensor(0x1000, M * K, np.float16)
    W = FakeROCmTensor(0x2000, N * K // 2, np.uint8)
    S = FakeROCmTensor(0x3000, N * K // G, np.float32)
    O = FakeROCmTensor(0x4000, M * N, np.float32)
    lib = FakeLib()
    cx = {"K_dim": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    assert try_launch("dequant_matvec_int4", (N,), (128,), [X, W, S, O], cx, lib=lib, sync=lambda: None)
    (c,) = lib.calls
    assert c["name"] == "dequant_matvec_int4" and c["grid"] == (N, 1) and c["block"] == (128, 1)
    assert c["ptrs"] == [0x1000, 0x2000, 0x3000, 0x4000]
    assert c["constexprs"] == [K, K // 2, K // G, G]
    assert c["dtypes"][0] == _lib.F16 and c["dtypes"][2] == _lib.F32 and c["dtypes"][3] == _lib.F32
    assert c["m"] == M


def test_int8_names_and_constexpr_order():
    K, N = 128, 4
    args = [FakeROCmTensor(0x10, K, np.float32), FakeROCmTensor(0x20, N * K, np.int8),
            FakeROCmTensor(0x30, N, np.float32), FakeROCmTensor(0x40, N, np.float32)]
    for name in ("dequant_matvec_int8", "quant_matvec_int8"):
        lib = FakeLib()
        assert try_launch(name, (N,), (128,), args, {"GROUP_SIZE": K, "NUM_SCALES": 1, "K_dim": K},
                          lib=lib, sync=lambda: None)
        assert lib.calls[0]["constexprs"] == [K, 1, K] and lib.calls[0]["m"] == 1
    lib = FakeLib()
    deq = [FakeROCmTensor(0x20, N * K, np.int8), FakeROCmTensor(0x30, N * 4, np.float16),
           FakeROCmTensor(0x40, N * K, np.float16)]
    assert try_launch("dequant_int8", (N,), (128,), deq, {"K": K, "NUM_SCALES": 4, "GROUP_SIZE": 32},
                      lib=lib, sync=lambda: None)
    assert lib.calls[0]["constexprs"] == [K, 4, 32] and lib.calls[0]["dtypes"][1:] == [_lib.F16, _lib.F16]


def test_host_arguments_are_uploaded_and_outputs_written_back():
    """np.ndarray and LocompTensor arguments, as _launch_rocm accepts them
    (locomp/api.py:966-983); the output comes back into the host array."""
    K, N, G = 256, 4, 128
    X = np.ones(K, np.float32)
    W = FakeLocompTensor(np.zeros((N, K // 2), np.uint8))
    S = np.ones((N, K // G), np.float32)
    O = np.zeros(N, np.float32)
    up, made = _uploader()
    lib = FakeLib()
    cx = {"K_dim": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    assert try_launch("dequant_matvec_int4", (N,), (128,), [X, W, S, O], cx, lib=lib, upload=up,
                      sync=lambda: None)
    assert [d.data_ptr for d in made] == lib.calls[0]["ptrs"]
    assert (O == 7).all()            # written back from the device copy
    assert (X == 1).all()            # inputs untouched


def test_validation_before_any_launch():
    K, N, G = 256, 4, 128
    cx = {"K_dim": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    W = FakeROCmTensor(2, N * K // 2, np.uint8)
    S = FakeROCmTensor(3, N * K // G, np.float32)
    lib = FakeLib()
    # X not a whole number of K-rows
    with pytest.raises(ValueError, match="multiple of K"):
        try_launch("dequant_matvec_int4", (N,), (128,),
                   [FakeROCmTensor(1, K + 3, np.float32), W, S, FakeROCmTensor(4, N, np.float32)],
                   cx, lib=lib)
    X = FakeROCmTensor(1, K, np.float32)
    O = FakeROCmTensor(4, N, np.float32)
    with pytest.raises(ValueError):                       # wrong N for W
        try_launch("dequant_matvec_int4", (N + 1,), (128,), [X, W, S, O], cx, lib=lib)
    with pytest.raises(ValueError):                       # 2-D grid
        try_launch("dequant_matvec_int4", (N, 2), (128,), [X, W, S, O], cx, lib=lib)
    with pytest.raises(TypeError, match="missing constexpr"):
        try_launch("dequant_matvec_int4", (N,), (128,), [X, W, S, O], {"K_dim": K}, lib=lib)
    with pytest.raises(TypeError):                        # int8 weights for the int4 kernel
        try_launch("dequant_matvec_int4", (N,), (128,),
                   [X, FakeROCmTensor(2, N * K // 2, np.int8), S, O], cx, lib=lib)
    with pytest.raises(TypeError, match="Unsupported argument type"):
        try_launch("dequant_matvec_int4", (N,), (128,), [X, W, S, 5], cx, lib=lib)
    with pytest.raises(ValueError, match="dequant_matvec_int4"):   # a library error code
        try_launch("dequant_matvec_int4", (N,), (128,), [X, W, S, O], cx, lib=FakeLib(rc=-1),
                   sync=lambda: None)
    assert lib.calls == []


def test_c_launch_entry_rejects_before_launch():
    """The real library, no device: argument errors return before any HIP call."""
    lib = _lib.load()
    P = ctypes.c_void_p(0x1000)
    args = (ctypes.c_void_p * 4)(P, P, P, P)
    argp = ctypes.cast(args, ctypes.POINTER(ctypes.c_void_p))
    dts = (ctypes.c_int * 4)(0, 0, 0, 0)

    def cx(*v):
        return (ctypes.c_int64 * len(v))(*v), len(v)

    c, n = cx(256, 128, 8, 32)
    assert lib.locomp_amd_launch(b"softmax", 4, 1, 128, 1, argp, c, n, dts, 1, None) == _lib.ERR_NAME
    assert lib.locomp_amd_launch(None, 4, 1, 128, 1, argp, c, n, dts, 1, None) == _lib.ERR_NAME
    assert lib.locomp_amd_launch(b"dequant_matvec_int4", 4, 2, 128, 1, argp, c, n, dts, 1, None) == _lib.ERR_SHAPE
    assert lib.locomp_amd_launch(b"dequant_matvec_int4", 4, 1, 2048, 1, argp, c, n, dts, 1, None) == _lib.ERR_SHAPE
    c3, n3 = cx(256, 8, 32)                 # int4 needs four integers
    assert lib.locomp_amd_launch(b"dequant_matvec_int4", 4, 1, 128, 1, argp, c3, n3, dts, 1, None) == _lib.ERR_SHAPE
    bad, nb = cx(256, 128, 7, 32)           # NUM_SCALES * GROUP_SIZE != K
    assert lib.locomp_amd_launch(b"dequant_matvec_int4", 4, 1, 128, 1, argp, bad, nb, dts, 1, None) == _lib.ERR_SHAPE
    bad8, n8 = cx(256, 3, 64)
    assert lib.locomp_amd_launch(b"quant_matvec_int8", 4, 1, 128, 1, argp, bad8, n8, dts, 1, None) == _lib.ERR_SHAPE
    assert lib.locomp_amd_launch(b"dequant_int4", 4, 1, 128, 1, argp, bad, nb, dts, 1, None) == _lib.ERR_SHAPE
    baddt = (ctypes.c_int * 4)(0, 0, 9, 0)
    assert lib.locomp_amd_launch(b"dequant_matvec_int8", 4, 1, 128, 1, argp, *cx(256, 8, 32), baddt, 1, None) == _lib.ERR_DTYPE
    assert _lib.strerror(_lib.ERR_NAME) == "unknown kernel name"


def test_uploads_live_until_the_launch_is_done():
    """Every uploaded temporary is still referenced when the library is
    called (one dropped earlier could hand its memory to the next upload)."""
    import weakref
    K, N, G = 256, 4, 128
    alive = []

    class Dev(FakeDev):
        pass

    made = []

    def up(a):
        d = Dev(a, 0x100 + len(made))
        made.append(weakref.ref(d))
        return d

    class CheckLib(FakeLib):
        def locomp_amd_launch(self, *a):
            alive.append(all(r() is not None for r in made))
            return super().locomp_amd_launch(*a)

    cx = {"K_dim": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    args = [np.ones(K, np.float32), np.zeros((N, K // 2), np.uint8), np.ones((N, 2), np.float32),
            FakeROCmTensor(9, N, np.float32)]
    assert try_launch("dequant_matvec_int4", (N,), (128,), args, cx, lib=CheckLib(), upload=up,
                      sync=lambda: None)
    assert alive == [True] and len(made) == 3
