"""Host-side tests (no GPU): C-ABI exports and argument validation, the Python
launch surface's validation, and CPU emulations of the kernels' bit tricks."""

import ctypes
import os
import re

import numpy as np
import pytest

from locomp_amd import _lib, kernels
from locomp_amd.kernels import ArgInfo

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "locomp_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(locomp_amd_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = _declared_functions()
    assert len(names) >= 8
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_lib.SIGNATURES), "bindings and header disagree"
    assert lib.locomp_amd_abi_version() == _lib.ABI_VERSION


def test_error_strings_and_policy():
    assert _lib.strerror(0) == "success"
    assert "sizes" in _lib.strerror(_lib.ERR_SHAPE)
    assert "dtype" in _lib.strerror(_lib.ERR_DTYPE)
    lib = _lib.load()
    assert lib.locomp_amd_set_policy(7) == _lib.ERR_POLICY
    assert lib.locomp_amd_set_policy(_lib.POLICY_GENERIC) == 0
    assert lib.locomp_amd_get_policy() == _lib.POLICY_GENERIC
    assert lib.locomp_amd_set_policy(_lib.POLICY_AUTO) == 0


# The C entry points validate before touching the device, so invalid calls can
# be exercised without a GPU (pointers are never dereferenced).
P = ctypes.c_void_p(0x1000)
NULL = ctypes.c_void_p(0)


def test_c_abi_rejects_bad_shapes_without_launch():
    lib = _lib.load()
    # K != 2 * HALF_K
    assert lib.locomp_amd_dequant_int4(P, P, P, 64, 31, 2, 32, 4, 1, 1, NULL) == _lib.ERR_SHAPE
    # NUM_SCALES * GROUP_SIZE != K
    assert lib.locomp_amd_dequant_int4(P, P, P, 64, 32, 3, 32, 4, 1, 1, NULL) == _lib.ERR_SHAPE
    assert lib.locomp_amd_dequant_int8(P, P, P, 64, 2, 0, 4, 1, 1, NULL) == _lib.ERR_SHAPE
    # bad dtype code
    assert lib.locomp_amd_dequant_int4(P, P, P, 64, 32, 2, 32, 4, 9, 1, NULL) == _lib.ERR_DTYPE
    assert lib.locomp_amd_dequant_matvec_int4(P, P, P, P, 64, 32, 2, 32, 4, 1, 1, 5, 1, NULL) == _lib.ERR_DTYPE
    # negative M / N
    assert lib.locomp_amd_dequant_matvec_int8(P, P, P, P, 64, 2, 32, -1, 1, 1, 1, 1, NULL) == _lib.ERR_SHAPE
    assert lib.locomp_amd_dequant_matvec_int8(P, P, P, P, 64, 2, 32, 4, -1, 1, 1, 1, NULL) == _lib.ERR_SHAPE
    # null pointers for a non-empty problem
    assert lib.locomp_amd_dequant_int4(NULL, P, P, 64, 32, 2, 32, 4, 1, 1, NULL) == _lib.ERR_NULL
    assert lib.locomp_amd_dequant_matvec_int4(NULL, P, P, P, 64, 32, 2, 32, 4, 1, 1, 1, 1, NULL) == _lib.ERR_NULL
    # empty problems succeed without touching pointers
    assert lib.locomp_amd_dequant_int4(NULL, NULL, NULL, 64, 32, 2, 32, 0, 1, 1, NULL) == 0
    assert lib.locomp_amd_dequant_matvec_int4(NULL, NULL, NULL, NULL, 64, 32, 2, 32, 4, 0, 1, 1, 1, NULL) == 0


def test_quantize_abi_validates_without_a_gpu():
    lib = _lib.load()
    q4, q8 = lib.locomp_amd_quantize_int4, lib.locomp_amd_quantize_int8
    EX38, EX52 = _lib.QUANT_EX38, _lib.QUANT_EX52
    # (W, PACKED, SCALES, N, K, GROUP_SIZE, variant, in_dtype, stream)
    assert q4(P, P, P, 4, 64, 24, EX38, 0, NULL) == _lib.ERR_SHAPE     # G does not divide K
    assert q4(P, P, P, 4, 45, 9, EX38, 0, NULL) == _lib.ERR_SHAPE      # odd int4 group
    assert q4(P, P, P, 4, 64, 0, EX38, 0, NULL) == _lib.ERR_SHAPE
    assert q4(P, P, P, -1, 64, 32, EX38, 0, NULL) == _lib.ERR_SHAPE
    assert q4(P, P, P, 4, 64, 32, 7, 0, NULL) == _lib.ERR_SHAPE        # unknown variant
    assert q4(P, P, P, 4, 64, 32, EX52, 5, NULL) == _lib.ERR_DTYPE
    assert q4(NULL, P, P, 4, 64, 32, EX38, 0, NULL) == _lib.ERR_NULL
    assert q4(NULL, NULL, NULL, 0, 64, 32, EX38, 0, NULL) == 0          # empty: nothing touched
    assert q8(P, P, P, 4, 64, 24, 0, NULL) == _lib.ERR_SHAPE
    assert q8(P, NULL, P, 4, 64, 32, 0, NULL) == _lib.ERR_NULL
    assert q8(P, P, P, 4, 64, 32, 3, NULL) == _lib.ERR_DTYPE


def test_silu_mul_abi_validates_without_a_gpu():
    lib = _lib.load()
    f = lib.locomp_amd_dequant_matvec_int4_silu_mul
    # (X, W, scales, O, K_dim, HALF_K, NUM_SCALES, GROUP_SIZE, I, M, xd, sd, od, stream)
    assert f(P, P, P, P, 64, 31, 2, 32, 8, 1, 1, 1, 1, NULL) == _lib.ERR_SHAPE   # HALF_K
    assert f(P, P, P, P, 64, 32, 3, 32, 8, 1, 1, 1, 1, NULL) == _lib.ERR_SHAPE   # NUM_SCALES * G != K
    assert f(P, P, P, P, 64, 32, 2, 32, 8, -1, 1, 1, 1, NULL) == _lib.ERR_SHAPE  # M < 0
    assert f(P, P, P, P, 64, 32, 2, 32, 8, 1, 7, 1, 1, NULL) == _lib.ERR_DTYPE
    assert f(NULL, P, P, P, 64, 32, 2, 32, 8, 1, 1, 1, 1, NULL) == _lib.ERR_NULL
    assert f(P, P, P, NULL, 64, 32, 2, 32, 8, 1, 1, 1, 1, NULL) == _lib.ERR_NULL
    assert f(NULL, NULL, NULL, NULL, 64, 32, 2, 32, 0, 1, 1, 1, 1, NULL) == 0    # I = 0: nothing to do


def test_fused_abi_validates_without_a_gpu():
    lib = _lib.load()
    f = lib.locomp_amd_dequant_matvec_int4_fused
    # (X, W, scales, O, K_dim, HALF_K, NUM_SCALES, GROUP_SIZE, N, M, xd, sd, od,
    #  norm_weight, eps, residual, silu_mul, stream)
    ok = (64, 32, 2, 32, 8, 1, 1, 1, 1)
    assert f(P, P, P, P, 64, 31, 2, 32, 8, 1, 1, 1, 1, P, 1e-5, None, 0, NULL) == _lib.ERR_SHAPE  # HALF_K
    assert f(P, P, P, P, 64, 32, 3, 32, 8, 1, 1, 1, 1, P, 1e-5, None, 0, NULL) == _lib.ERR_SHAPE  # G
    assert f(P, P, P, P, *ok, P, 1e-5, P, 1, NULL) == _lib.ERR_SHAPE        # SiLU * mul with a residual
    assert f(P, P, P, P, 64, 32, 2, 32, 7, 1, 1, 1, 1, P, 1e-5, None, 1, NULL) == _lib.ERR_SHAPE  # odd rows
    assert f(P, P, P, P, 64, 32, 2, 32, 8, 1, 7, 1, 1, P, 1e-5, None, 0, NULL) == _lib.ERR_DTYPE
    assert f(NULL, P, P, P, *ok, P, 1e-5, None, 0, NULL) == _lib.ERR_NULL
    assert f(P, P, P, NULL, *ok, P, 1e-5, P, 0, NULL) == _lib.ERR_NULL
    assert f(NULL, NULL, NULL, NULL, 64, 32, 2, 32, 8, 0, 1, 1, 1, P, 1e-5, P, 0, NULL) == 0  # M = 0


def test_rms_norm_abi_validates_without_a_gpu():
    lib = _lib.load()
    f = lib.locomp_amd_rms_norm
    # (H, R, gamma, Y, M, K, eps, dtype, stream); fp16, bf16 and fp32 accepted
    assert f(P, NULL, P, P, 1, 576, 1e-5, 7, NULL) == _lib.ERR_DTYPE
    assert f(P, NULL, P, P, -1, 576, 1e-5, 2, NULL) == _lib.ERR_SHAPE
    assert f(NULL, NULL, P, P, 1, 576, 1e-5, 2, NULL) == _lib.ERR_NULL
    assert f(NULL, NULL, NULL, NULL, 0, 576, 1e-5, 2, NULL) == 0


def test_interleave_gate_up():
    import locomp_amd as lq
    g = np.arange(12, dtype=np.uint8).reshape(3, 4)
    u = 100 + np.arange(12, dtype=np.uint8).reshape(3, 4)
    w = lq.interleave_gate_up(g, u)
    assert w.shape == (6, 4) and np.array_equal(w[0::2], g) and np.array_equal(w[1::2], u)
    with pytest.raises(ValueError):
        lq.interleave_gate_up(g, u[:2])


def test_check_maps_codes_to_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.ERR_SHAPE, "x")
    with pytest.raises(_lib.LocompAMDError):
        _lib.check(1, "x")
    _lib.check(0, "x")


# ------------------------------------------------------------ planners --

U8, I8, F16, F32 = np.dtype(np.uint8), np.dtype(np.int8), np.dtype(np.float16), np.dtype(np.float32)


def test_plan_matvec_int4_ok_and_codes():
    N, K, G, M = 8, 64, 32, 3
    ints = kernels.plan_dequant_matvec_int4(
        N, ArgInfo(M * K, F16), ArgInfo(N * K // 2, U8), ArgInfo(N * K // G, F16),
        ArgInfo(M * N, F32), K, K // 2, K // G, G)
    assert ints == [K, K // 2, K // G, G, N, M, _lib.F16, _lib.F16, _lib.F32]


@pytest.mark.parametrize("bad", ["W", "S", "O", "X", "K", "G"])
def test_plan_matvec_int4_rejects(bad):
    N, K, G, M = 8, 64, 32, 2
    args = dict(X=ArgInfo(M * K, F16), W=ArgInfo(N * K // 2, U8), S=ArgInfo(N * K // G, F16),
                O=ArgInfo(M * N, F16))
    ints = [K, K // 2, K // G, G]
    if bad == "W":
        args["W"] = ArgInfo(N * K // 2 - 1, U8)
    elif bad == "S":
        args["S"] = ArgInfo(N * K // G + 1, F16)
    elif bad == "O":
        args["O"] = ArgInfo(M * N + 1, F16)
    elif bad == "X":
        args["X"] = ArgInfo(M * K + 3, F16)
    elif bad == "K":
        ints = [K, K // 2 + 1, K // G, G]
    elif bad == "G":
        ints = [K, K // 2, K // G, G + 1]
    with pytest.raises(ValueError):
        kernels.plan_dequant_matvec_int4(N, args["X"], args["W"], args["S"], args["O"], *ints)


def test_plan_dtype_errors():
    N, K, G = 4, 32, 32
    with pytest.raises(TypeError):   # int8 weights passed to the int4 kernel
        kernels.plan_dequant_int4(N, ArgInfo(N * K // 2, I8), ArgInfo(N, F16), ArgInfo(N * K, F16),
                                  K, K // 2, 1, G)
    with pytest.raises(TypeError):   # uint8 scales
        kernels.plan_dequant_int8(N, ArgInfo(N * K, I8), ArgInfo(N, U8), ArgInfo(N * K, F16), K, 1, G)
    with pytest.raises(TypeError):   # non-integer constexpr
        kernels.plan_dequant_int8(N, ArgInfo(N * K, I8), ArgInfo(N, F16), ArgInfo(N * K, F16), 32.5, 1, G)


def test_launch_syntax_and_grid_validation():
    k = kernels.dequant_matvec_int4
    call = k[(8,), (128,)]
    assert call.grid == (8,) and call.block == (128,)
    assert k[8].grid == (8,)
    N, K, G = 8, 64, 32
    args = [np.zeros(K, np.float16), np.zeros((N, K // 2), np.uint8), np.zeros((N, 2), np.float16),
            np.zeros(N, np.float16), K, K // 2, 2, G]
    assert k.plan((N,), (128,), *args)[4] == N
    with pytest.raises(ValueError):
        k.plan((N, 2), (128,), *args)            # 2-D grid
    with pytest.raises(ValueError):
        k.plan((N,), (2048,), *args)             # block too large
    with pytest.raises(TypeError):
        k.plan((N,), (128,), *args[:-1])         # missing argument
    with pytest.raises(ValueError):
        k.plan((N + 1,), (128,), *args)          # grid does not match W


def test_reference_call_shapes_plan():
    """The exact launches of examples/38 (K % 256 == 0, G = 32) and 52 plan."""
    N, K, G = 256, 512, 32
    kernels.dequant_matvec_int4.plan((N,), (128,), np.zeros(K, np.float32), np.zeros((N, K // 2), np.uint8),
                                     np.zeros((N, K // G), np.float32), np.zeros(N, np.float32),
                                     K, K // 2, K // G, G)
    kernels.dequant_matvec_int8.plan((N,), (128,), np.zeros(K, np.float32), np.zeros((N, K), np.int8),
                                     np.zeros((N, K // G), np.float32), np.zeros(N, np.float32),
                                     K, K // G, G)
    kernels.dequant_int4.plan((N,), (128,), np.zeros(N * K // 2, np.uint8), np.zeros(N * K // G, np.float32),
                              np.zeros(N * K, np.float32), K, K // 2, K // G, G)
    kernels.dequant_int8.plan((N,), (128,), np.zeros(N * K, np.int8), np.zeros(N * K // G, np.float32),
                              np.zeros(N * K, np.float32), K, K // G, G)


# ------------------------------------------- CPU emulation of bit tricks --
# The decode helpers in locomp_amd/csrc/lq_common.h, replayed with NumPy on
# every byte value so a wrong mask, shift or selector fails here.

def _h(u16):
    return np.array(u16, np.uint16).view(np.float16).astype(np.float64)


def _perm(s0, s1, sel):
    """v_perm_b32: byte i of the result = byte sel_i of {s0:s1} (s1 = bytes 0..3)."""
    src = [(s1 >> (8 * i)) & 0xFF for i in range(4)] + [(s0 >> (8 * i)) & 0xFF for i in range(4)]
    out = 0
    for i in range(4):
        b = (sel >> (8 * i)) & 0xFF
        v = src[b] if b < 8 else (0 if b == 0x0C else 0xFF)
        out |= v << (8 * i)
    return out


def _words():
    rng = np.random.default_rng(0)
    ws = list(rng.integers(0, 2 ** 32, 300, dtype=np.uint64).astype(np.uint32))
    ws += [int(b) * 0x01010101 for b in range(256)]
    return [int(w) for w in ws]


def _nibbles(w):
    return [(w >> (4 * i)) & 0xF for i in range(8)]   # k0..k7


def test_int4_pair_decode_exact():
    """int4_pair_to_h2: perm + mask + OR 0x6400, fma (1, 1/16) + (-1032, -72)."""
    for w in _words():
        q = _nibbles(w)
        for p in range(4):
            u = _perm(w, w, p | (p << 16))
            t = (u & 0x00F0000F) | 0x64006400
            lo, hi = _h(t & 0xFFFF), _h(t >> 16)
            assert lo * 1.0 - 1032 == q[2 * p] - 8
            assert hi * 0.0625 - 72 == q[2 * p + 1] - 8


def test_int4_biased_kperm_and_xperm_agree():
    """int4x8_biased_kperm pairs (k0,k4),(k1,k5),(k2,k6),(k3,k7); xperm8 orders x alike."""
    x = np.arange(8, dtype=np.float16) + 1
    xd = x.view(np.uint32)
    xp = [_perm(xd[2], xd[0], 0x05040100), _perm(xd[2], xd[0], 0x07060302),
          _perm(xd[3], xd[1], 0x05040100), _perm(xd[3], xd[1], 0x07060302)]
    xs = np.array(xp, np.uint32).view(np.float16).astype(np.float64)
    assert list(xs) == [1, 5, 2, 6, 3, 7, 4, 8]
    for w in _words():
        q = _nibbles(w)
        r = [(w >> (4 * i)) & 0x000F000F | 0x64006400 for i in range(4)]
        vals = np.array(r, np.uint32).view(np.float16).astype(np.float64)
        want = [q[0], q[4], q[1], q[5], q[2], q[6], q[3], q[7]]
        assert list(vals - 1024) == want
        # x . (v - 1032) == sum x_k (q_k - 8) with the matching x order
        assert float(np.dot(xs, vals - 1032)) == float(np.dot(np.arange(1, 9), np.array(q) - 8))


def test_int4_segment_decode_with_sixteenth():
    """gemv_seg_kernel decode: masks 0x000F000F / 0x00F000F0 on w and w >> 8; the 16q
    halves meet activations pre-divided by 16 and the bias is 1032 / 1152."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal(8).astype(np.float16)
    xs = np.array([x[0], x[4], x[1], x[5], x[2], x[6], x[3], x[7]], np.float64)
    scale16 = np.array([1, 1, 1 / 16, 1 / 16, 1, 1, 1 / 16, 1 / 16])
    bias = np.array([1032, 1032, 1152, 1152, 1032, 1032, 1152, 1152], np.float64)
    for w in _words():
        q = np.array(_nibbles(w))
        w8 = w >> 8
        r = [(w & 0x000F000F) | 0x64006400, (w & 0x00F000F0) | 0x64006400,
             (w8 & 0x000F000F) | 0x64006400, (w8 & 0x00F000F0) | 0x64006400]
        v = np.array(r, np.uint32).view(np.float16).astype(np.float64)
        xp = xs * scale16
        got = float(np.dot(xp, v) - np.dot(xp, bias))
        want = float(np.dot(x.astype(np.float64), q - 8))
        assert abs(got - want) < 1e-9


def test_row_kernel_half_group_sums():
    """gemv_rows_kernel with G16 (scale groups of 16-k multiples): a lane's 32 k
    are 4 dwords of 8 k; dwords 0, 1 form the first 16 k and 2, 3 the second,
    each half with its own scale and its own bias correction (1032 x the sum
    of that half's activations).  Replayed on every dword pattern against the
    plain dot product with a scale per 16 k, and the group of each half is
    one group for every G % 16 == 0 (a lane's range starts at a multiple of 32)."""
    rng = np.random.default_rng(2)
    ws = _words()
    for t in range(200):
        x = rng.standard_normal(32).astype(np.float16)
        s = rng.uniform(0.001, 0.01, 2)
        wd = [ws[(4 * t + e) % len(ws)] for e in range(4)]
        acc = 0.0
        for h in range(2):
            pe, xsum = 0.0, 0.0
            for e in (2 * h, 2 * h + 1):
                xe = x[8 * e: 8 * e + 8]
                xd = xe.view(np.uint32)
                xp = [_perm(xd[2], xd[0], 0x05040100), _perm(xd[2], xd[0], 0x07060302),
                      _perm(xd[3], xd[1], 0x05040100), _perm(xd[3], xd[1], 0x07060302)]
                xs = np.array(xp, np.uint32).view(np.float16).astype(np.float64)
                r = [(wd[e] >> (4 * i)) & 0x000F000F | 0x64006400 for i in range(4)]
                v = np.array(r, np.uint32).view(np.float16).astype(np.float64)
                pe += float(np.dot(xs, v))
                xsum += float(np.sum(xs))
            acc += (pe - 1032.0 * xsum) * s[h]
        q = np.array([n for w in wd for n in _nibbles(w)], np.float64) - 8
        want = float(np.dot(x.astype(np.float64), q * np.repeat(s, 16)))
        assert abs(acc - want) <= 1e-9 * max(1.0, abs(want))
    for G in range(16, 1025, 16):
        for k0 in range(0, 8 * G, 32):
            for h in range(2):
                assert (k0 + 16 * h) // G == (k0 + 16 * h + 15) // G


def _rows16_plan(M, N, K, xd, epi):
    """Segments and rows per wave launch_rows16_m picks (None: not launched)."""
    nseg = (K + 2047) // 2048
    if nseg <= 2 and N <= 3072:
        return nseg, (2 if epi else 1)
    if nseg <= 2:
        return nseg, 4
    if M == 1 and xd != "f32":
        if nseg <= 4:
            return 4, 2
        if nseg <= 6:
            return 6, (2 if epi else 1)
        if not epi:
            return 8, 1
    return None


@pytest.mark.parametrize("M,N,K,G,xd,sd,epi", [
    (1, 11008, 4096, 16, "f16", "f16", False), (2, 1000, 4096, 16, "bf16", "f32", False),
    (1, 700, 10240, 16, "f16", "bf16", False), (1, 513, 14400, 48, "bf16", "f32", False),
    (2, 3000, 1440, 48, "f16", "f16", False), (1, 4100, 2080, 80, "f32", "f32", False),
    (1, 3072, 576, 16, "f32", "f32", True), (2, 2000, 4096, 16, "f16", "f32", True),
    (1, 1536, 12288, 48, "bf16", "bf16", True), (1, 1, 32, 16, "f16", "f32", False),
    (1, 7, 16352, 16, "f16", "f32", False), (2, 4098, 4096, 16, "bf16", "f16", True),
])
def test_row_kernel_g16_addresses_in_bounds(M, N, K, G, xd, sd, epi):
    """Every global load of gemv_rows_kernel in its G16 form, replayed for the
    grid launch_rows16_m picks: activations (clamped row and k-range), weights
    (clamped row), and each half's scale lie inside their arrays, and each
    half's 16 k lie in the group whose scale it loads."""
    plan = _rows16_plan(M, N, K, xd, epi)
    assert plan is not None
    nseg, rw = plan
    m_ = 1 if M == 1 else 2
    blocks = (N + 4 * rw - 1) // (4 * rw)
    ns = K // G
    xs, ss = (4 if xd == "f32" else 2), (4 if sd == "f32" else 2)
    n0 = (np.arange(blocks * 4, dtype=np.int64) * rw)[:, None, None]
    c = np.arange(nseg, dtype=np.int64)[None, :, None]
    lane = np.arange(64, dtype=np.int64)[None, None, :]
    k0 = np.minimum(c * 2048 + lane * 32, K - 32)
    assert k0.min() >= 0
    for m in range(m_):
        me = m if m < M else 0
        at = me * K + k0 + 8 * np.arange(4)[:, None, None, None]
        assert at.min() >= 0 and (at.max() + 8) * xs <= M * K * xs
    for r in range(rw):
        n = np.minimum(n0 + r, N - 1)
        assert ((n * (K // 2) + k0 // 2).max() + 16) <= N * K // 2
        for h in range(2):
            kh = k0 + 16 * h
            si = n * ns + kh // G
            assert si.min() >= 0 and (si.max() + 1) * ss <= N * ns * ss
            assert np.array_equal(kh // G, (kh + 15) // G)


def test_int8_decodes_exact():
    for w in _words():
        b = [((w >> (8 * i)) & 0xFF) for i in range(4)]
        sb = [v - 256 if v >= 128 else v for v in b]
        x = w ^ 0x80808080
        lo = _perm(0x64646464, x, 0x04010400)
        hi = _perm(0x64646464, x, 0x04030402)
        vals = np.array([lo, hi], np.uint32).view(np.float16).astype(np.float64) - 1152
        assert list(vals) == sb
    # int8x8_biased_kperm: byte i of w0 and of w1, xor 0x64806480
    for w0, w1 in zip(_words()[:100], _words()[100:200]):
        b0 = [((w0 >> (8 * i)) & 0xFF) for i in range(4)]
        b1 = [((w1 >> (8 * i)) & 0xFF) for i in range(4)]
        for i in range(4):
            r = _perm(w1, w0, 0x0C040C00 + i * 0x00010001) ^ 0x64806480
            v = np.array([r], np.uint32).view(np.float16).astype(np.float64) - 1152
            s0 = b0[i] - 256 if b0[i] >= 128 else b0[i]
            s1 = b1[i] - 256 if b1[i] >= 128 else b1[i]
            assert list(v) == [s0, s1]
