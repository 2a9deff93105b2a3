"""GPU parity for scale groups the MFMA kernels do not take (G % 32 != 0;
the reference accepts any G dividing K, examples/38_quantized_matmul.py:
141-155) and for activations too unaligned for them: the fp32-FMA VALU
kernel (`gemv_group.hip`), every activation dtype, int4 and int8, with and
without the k split over workgroups, and the gate|up SiLU * mul epilogue;
at M <= 2 with G % 16 == 0 the row kernel with a scale per 16 k
(`gemv_rows16.hip`).

Oracle: the restated reference NumPy path on the values the kernel sees.
Bars: fp32 activations and outputs rtol 1e-4 (+ atol 1e-5 max|Y|); fp16 /
bf16 ones 1e-2, as elsewhere.
"""

import ctypes

import numpy as np
import pytest

from locomp_amd import synth
from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

lq = pytest.importorskip("locomp_amd")

NP = {"f32": np.float32, "f16": np.float16}


def _used(a, name):
    if name == "bf16":
        return ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(np.asarray(a, np.float32))).reshape(np.shape(a))
    if name == "f16":
        return np.asarray(a).astype(np.float16).astype(np.float32)
    return np.asarray(a, np.float32)


def _dev(a, name):
    if name == "bf16":
        return lq.tensor(np.asarray(a, np.float32), dtype=lq.bfloat16)
    return lq.tensor(np.ascontiguousarray(np.asarray(a).astype(NP[name])))


def _out(Og, od, shape):
    got = Og.numpy()
    if od == "bf16":
        return ref.bf16_bits_to_f32(got).reshape(shape).astype(np.float64)
    return got.astype(np.float64)


def _check(got, want, xd, od):
    if xd == "f32" and od == "f32":
        atol = 1e-5 * max(1.0, float(np.abs(want).max()))
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2 * max(1.0, float(np.abs(want).max())))


@pytest.mark.parametrize("wbits,M,N,K,G", [
    (4, 1, 4096, 4096, 16),     # k split over workgroups
    (4, 3, 1000, 2048, 8),      # ragged row block, G = 8 (one dword per group)
    (4, 16, 640, 1536, 48),     # 3 groups of 16 k
    (4, 20, 130, 96, 24),       # two passes of 16 rows, groups of 3 dwords, few groups
    (4, 64, 2048, 4096, 16),
    (4, 200, 700, 512, 16),     # prefill-sized M
    (8, 1, 3000, 4096, 4),      # int8: one dword per group
    (8, 5, 2000, 1032, 12),
    (8, 33, 520, 2048, 16),
])
@pytest.mark.parametrize("xd,sd,od", [("f32", "f32", "f32"), ("f16", "f16", "f16"),
                                      ("bf16", "bf16", "bf16"), ("f32", "f16", "f32"),
                                      ("bf16", "f32", "f16")])
def test_small_groups(wbits, M, N, K, G, xd, sd, od):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, x_dtype=np.float32,
                                s_dtype=np.float32, seed=M + N + K + G + wbits)
    X = X * np.float32(3.0)
    Og = lq.empty((M, N), lq.bfloat16 if od == "bf16" else NP[od])
    if wbits == 4:
        lq.dequant_matvec_int4[(N,), (128,)](_dev(X, xd), lq.tensor(W), _dev(S, sd), Og, K, K // 2,
                                             K // G, G)
        want = ref.fast_numpy_matvec_int4(_used(X, xd), W, _used(S, sd), G)
    else:
        lq.dequant_matvec_int8[(N,), (128,)](_dev(X, xd), lq.tensor(W), _dev(S, sd), Og, K, K // G, G)
        want = ref.fast_numpy_matvec_int8(_used(X, xd), W, _used(S, sd), G)
    _check(_out(Og, od, (M, N)), np.asarray(want, np.float64), xd, od)


@pytest.mark.parametrize("M,N,K,G", [
    (1, 11008, 4096, 16),       # 2 segments, 4 rows per wave
    (2, 1000, 4096, 16),        # two activation rows
    (1, 700, 10240, 16),        # 5 segments on the 6-segment kernel, one row per wave
    (1, 513, 14400, 48),        # 8 segments, the last partial; groups of 3 halves
    (2, 3000, 1440, 48),        # one partial segment, one row per wave
    (1, 4100, 2080, 80),        # ragged last workgroup
])
@pytest.mark.parametrize("xd,sd,od", [("f16", "f16", "f16"), ("bf16", "bf16", "bf16"),
                                      ("f32", "f32", "f32"), ("f16", "f32", "bf16")])
def test_row_kernel_half_groups(M, N, K, G, xd, sd, od):
    """int4, M <= 2, G a multiple of 16 but not of 32: the row kernel with a
    scale per 16 k (fp32 activations: M = 1, K <= 4096; other shapes take
    the VALU kernel), against the oracle."""
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, x_dtype=np.float32,
                                s_dtype=np.float32, seed=M + N + K + G)
    Og = lq.empty((M, N), lq.bfloat16 if od == "bf16" else NP[od])
    lq.dequant_matvec_int4[(N,), (128,)](_dev(X, xd), lq.tensor(W), _dev(S, sd), Og, K, K // 2, K // G, G)
    want = ref.fast_numpy_matvec_int4(_used(X, xd), W, _used(S, sd), G)
    _check(_out(Og, od, (M, N)), np.asarray(want, np.float64), xd, od)


@pytest.mark.parametrize("M,I,K,G,xd", [
    (1, 1536, 576, 16, "f32"),
    (2, 1000, 4096, 16, "f16"),     # row kernel with the epilogue
    (1, 768, 12288, 48, "bf16"),    # 6 segments, 2 rows per wave
    (1, 500, 14336, 16, "f16"),     # 7 segments: the VALU kernel
    (2, 600, 2048, 16, "bf16"),
    (4, 700, 2048, 16, "bf16"),
    (24, 300, 1024, 8, "f16"),
    (130, 256, 480, 48, "f32"),
])
def test_small_groups_silu_mul(M, I, K, G, xd):
    """The gate|up SiLU * mul epilogue on the same kernel (gate and up rows
    in neighbouring lanes), with and without the k split."""
    Xa, Wg, Sg = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                   s_dtype=np.float32, seed=I + K + 3)
    _, Wu, Su = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                  s_dtype=np.float32, seed=I + K + 4)
    W = lq.interleave_gate_up(Wg, Wu)
    S = lq.interleave_gate_up(Sg, Su)
    Xu = _used(Xa, xd)
    got = lq.gpu_matvec_int4_silu_mul(_dev(Xa, xd), W, lq.tensor(S), G, out_dtype=np.float32)
    g = np.asarray(ref.fast_numpy_matvec_int4(Xu, Wg, Sg, G), np.float64)
    u = np.asarray(ref.fast_numpy_matvec_int4(Xu, Wu, Su, G), np.float64)
    silu = g / (1.0 + np.exp(-g))
    want = silu * u

    def mag(Wp, Sp):   # sum_k |x_k w_nk| per output
        q = np.empty((Wp.shape[0], K), np.float64)
        q[:, 0::2] = (Wp & 15).astype(np.float64) - 8
        q[:, 1::2] = (Wp >> 4).astype(np.float64) - 8
        return np.abs(Xu.astype(np.float64)) @ np.abs(q * np.repeat(Sp.astype(np.float64), G, axis=1)).T

    # the propagated bar of the two dot products (fp32: rtol 1e-4 of
    # sum|x w|; fp16 / bf16 activations: 1e-2)
    tol = 1e-4 if xd == "f32" else 1e-2
    bound = tol * (1.1 * np.abs(u) * mag(Wg, Sg) + np.abs(silu) * mag(Wu, Su)) + 1e-12
    err = np.abs(np.asarray(got, np.float64).reshape(M, I) - want)
    assert (err <= bound).all(), (err.max(), np.argmax(err - bound))


@pytest.mark.parametrize("offset", [2, 1])
def test_unaligned_activations(offset):
    """fp16 activations starting 4 bytes (offset 2) or 2 bytes (offset 1)
    past a 16-byte boundary: the MFMA kernels need 16-byte alignment; the
    VALU kernel takes 4-byte-aligned rows, the generic kernel the rest.
    Both against the oracle."""
    import torch

    from locomp_amd import _lib

    lib = _lib.load()
    vp = ctypes.c_void_p
    M, N, K, G = 4, 1024, 2048, 32
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=offset)
    want = ref.fast_numpy_matvec_int4(X, W, S, G)
    flat = torch.zeros(M * K + 8, dtype=torch.float16, device="cuda")
    flat[offset:offset + M * K] = torch.from_numpy(np.ascontiguousarray(X)).reshape(-1).cuda()
    Wd, Sd = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (W, S))
    Od = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    rc = lib.locomp_amd_dequant_matvec_int4(
        vp(flat.data_ptr() + 2 * offset), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(Od.data_ptr()),
        K, K // 2, K // G, G, N, M, _lib.F16, _lib.F16, _lib.F32, vp(torch.cuda.current_stream().cuda_stream))
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_allclose(Od.cpu().numpy(), want, rtol=1e-2, atol=1e-2 * float(np.abs(want).max()))
