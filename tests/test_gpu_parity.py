"""GPU parity: the HIP kernels (through the C ABI) against the CPU oracle.

Bars: dequantised weights bit-exact; dequant-matmul within rtol 1e-2 /
atol 1e-2 for fp16 activations, rtol 1e-4 (+ atol 1e-5 * max|Y|) for fp32.
"""

import numpy as np
import pytest

from locomp_amd import synth
from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

lq = pytest.importorskip("locomp_amd")

NP_OF = {"f32": np.float32, "f16": np.float16}


def _dtype(name):
    return lq.bfloat16 if name == "bf16" else NP_OF[name]


def _up(a, dtype_name=None):
    if dtype_name == "bf16":
        return lq.tensor(a.astype(np.float32), dtype=lq.bfloat16)
    return lq.tensor(np.ascontiguousarray(a))


def _scales_f32(S, s_name):
    return S.astype(np.float32)


@pytest.fixture(params=["auto", "generic"])
def policy(request):
    lq.set_policy(0 if request.param == "auto" else 1)
    yield request.param
    lq.set_policy(0)


# ---------------------------------------------------------------- dequant --

def _run_dequant4(W, S, N, K, G, od):
    Wg, Sg = _up(W), _up(S)
    Og = lq.empty(N * K, _dtype(od))
    lq.dequant_int4[(N,), (128,)](Wg, Sg, Og, K, K // 2, K // G, G)
    return Og.numpy().reshape(N, K)


def _run_dequant8(W, S, N, K, G, od):
    Wg, Sg = _up(W), _up(S)
    Og = lq.empty(N * K, _dtype(od))
    lq.dequant_int8[(N,), (128,)](Wg, Sg, Og, K, K // G, G)
    return Og.numpy().reshape(N, K)


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view({2: np.uint16, 4: np.uint32}[a.dtype.itemsize])


@pytest.mark.parametrize("sd", ["f16", "f32"])
@pytest.mark.parametrize("od", ["f16", "f32", "bf16"])
@pytest.mark.parametrize("N,K,G", [(64, 256, 32), (37, 96, 8), (5, 64, 64), (3, 30, 6), (16, 4, 2)])
def test_dequant_int4_bitexact(policy, sd, od, N, K, G):
    W, S = synth.dequant_case(4, N, K, G, 0.001, 0.01, s_dtype=NP_OF[sd], seed=N + K)
    got = _run_dequant4(W, S, N, K, G, od)
    want = ref.cast_out(ref.dequant_int4_ref(W, S, N, K, G), od)
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("sd", ["f16", "f32"])
@pytest.mark.parametrize("od", ["f16", "f32", "bf16"])
@pytest.mark.parametrize("N,K,G", [(64, 256, 32), (37, 96, 8), (5, 64, 64), (3, 30, 6)])
def test_dequant_int8_bitexact(policy, sd, od, N, K, G):
    W, S = synth.dequant_case(8, N, K, G, 0.002, 0.02, s_dtype=NP_OF[sd], seed=N * K)
    got = _run_dequant8(W, S, N, K, G, od)
    want = ref.cast_out(ref.dequant_int8_ref(W, S, N, K, G), od)
    assert np.array_equal(_bits(got), _bits(want))


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("sd", ["f16", "f32"])
@pytest.mark.parametrize("od", ["f16", "f32", "bf16"])
def test_dequant_bitexact_subnormal_and_negative_scales(wbits, sd, od):
    """Scales whose products are fp16 subnormals (|s| down to 2^-24, so
    (q - 8) s lands below 2^-14), zero, negative (q = 8 then gives -0.0),
    and large ones near the fp16 limit; every output bit must match the
    reference definition, through the fast kernels and the generic ones."""
    N, K, G = 48, 256, 32
    rng = np.random.default_rng(wbits * 10 + len(sd) + len(od))
    W, _ = synth.dequant_case(wbits, N, K, G, 0.001, 0.01, seed=3)
    mags = np.concatenate([np.exp2(rng.uniform(-24, -14, 180)),      # subnormal products
                           np.exp2(rng.uniform(-14, 4, 180)),
                           [0.0] * 8, [2.0 ** -24] * 8, [6.0e4 / 2048] * 8])   # N * K / G = 384
    sign = np.where(rng.random(mags.size) < 0.5, -1.0, 1.0)
    S = (mags * sign).reshape(N, K // G).astype(NP_OF[sd])
    for pol in (0, 1):
        lq.set_policy(pol)
        try:
            if wbits == 4:
                got = _run_dequant4(W, S, N, K, G, od)
                want = ref.cast_out(ref.dequant_int4_ref(W, S, N, K, G), od)
            else:
                got = _run_dequant8(W, S, N, K, G, od)
                want = ref.cast_out(ref.dequant_int8_ref(W, S, N, K, G), od)
        finally:
            lq.set_policy(0)
        assert np.array_equal(_bits(got), _bits(want)), f"policy {pol}"
        if od == "f16" and sd == "f16":
            w16 = np.ascontiguousarray(want).view(np.uint16)
            assert ((w16 & 0x7C00) == 0).any() and ((w16 & 0x7FFF) != 0).any()   # subnormals present
            assert (w16 == 0x8000).any() or wbits == 8                          # -0.0 from q = 8


def test_dequant_int4_cfg2_full_bitexact():
    c = synth.CFG2
    W, S = synth.dequant_case(4, c["N"], c["K"], c["G"], c["lo"], c["hi"])
    got = _run_dequant4(W, S, c["N"], c["K"], c["G"], "f16")
    want = ref.dequant_int4_ref(W, S, c["N"], c["K"], c["G"]).astype(np.float16)
    assert np.array_equal(_bits(got), _bits(want))


def test_dequant_reference_selfcheck_shapes():
    """examples/52_dequantize.py:146-170: seed 42, G=32, three shapes, fp32."""
    rng = np.random.default_rng(42)
    for N, K in [(64, 256), (128, 512), (256, 1024)]:
        w = rng.standard_normal((N, K)).astype(np.float32) * 0.5
        packed, scales = ref.quantize_int4_ref(w, 32)
        got = lq.gpu_dequant_int4(packed, scales, N, K, 32)
        want = ref.dequant_int4_ref(packed, scales, N, K, 32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
        absmax = np.abs(w.reshape(N, K // 32, 32)).max(axis=2)
        s8 = (absmax / 127.0).astype(np.float32)
        q8 = np.clip(np.round(w / (np.repeat(s8, 32, axis=1) + 1e-10)), -128, 127).astype(np.int8)
        got8 = lq.gpu_dequant_int8(q8, s8, N, K, 32)
        want8 = q8.astype(np.float32) * np.repeat(s8, 32, axis=1)
        assert np.array_equal(got8.view(np.uint32), want8.view(np.uint32))


# --------------------------------------------------------------- matvec --

def _matvec(wbits, X, W, S, N, K, G, od):
    M = X.shape[0]
    Xg, Wg, Sg = _up(X), _up(W), _up(S)
    Og = lq.empty((M, N), _dtype(od))
    if wbits == 4:
        lq.dequant_matvec_int4[(N,), (128,)](Xg, Wg, Sg, Og, K, K // 2, K // G, G)
    else:
        lq.dequant_matvec_int8[(N,), (128,)](Xg, Wg, Sg, Og, K, K // G, G)
    return Og.numpy()


def _oracle(wbits, X, W, S, G):
    if wbits == 4:
        return ref.fast_numpy_matvec_int4(X, W, S, G)
    return ref.fast_numpy_matvec_int8(X, W, S, G)


def _close(got, want, fp32=False):
    got = got.astype(np.float32)
    if fp32:
        atol = 1e-5 * max(1.0, float(np.abs(want).max()))
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M,N,K,G", [
    (1, 64, 256, 32), (4, 100, 512, 128), (16, 48, 1024, 1024), (3, 17, 96, 32),
    (1, 192, 576, 32), (1, 576, 1536, 32), (33, 40, 256, 64), (64, 80, 512, 512),
    (2, 7, 40, 8), (5, 9, 16, 16),
    (2, 3072, 576, 32),    # row kernel, one row per wave, two activation rows
    (1, 3100, 1024, 32)])  # row kernel, four rows per wave (N > 3072), ragged
def test_matvec_fp16_small(policy, wbits, M, N, K, G):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=M * 1000 + N)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M,N,K,G", [
    (2, 37, 1024, 32), (3, 1000, 2048, 128), (8, 64, 6144, 64), (16, 33, 3072, 1024),
    (5, 250, 4096, 16), (16, 11008, 1024, 128), (12, 96, 2560, 512), (9, 13000, 1024, 64)])
def test_matvec_lds_ring_shapes(wbits, M, N, K, G):
    """Decode sizes 2 <= M <= 16 with whole 512-byte row chunks (the LDS-ring
    kernel): ragged N, odd chunk counts, post-scaled and pre-scaled groups
    (int4 G = 16 takes the LDS kernel instead)."""
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=7 * M + N + K)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M,N,K,G", [
    (17, 64, 1024, 64), (33, 300, 2048, 16), (64, 1000, 4096, 4096), (48, 4100, 1536, 512),
    (16, 1000, 4096, 4096), (3, 77, 1024, 1024), (32, 11008, 4096, 128), (64, 9000, 768, 32),
    (40, 500, 1536, 384), (24, 333, 3072, 768), (64, 14336, 4096, 4096), (12, 777, 2048, 512),
    (9, 4100, 1024, 1024),
    # 16 < M <= 64 (int8: 32 < M) at N <= 4096 with long rows: the split-K
    # GEMM (8 uneven splits of 172 / 160 / 224 steps)
    (64, 4096, 11008, 128), (33, 4000, 10240, 64), (48, 4096, 14336, 14336), (20, 3100, 11008, 32)])
def test_matvec_many_rows_and_per_channel(wbits, M, N, K, G):
    """Decode/verify sizes up to M = 64 and per-channel / large groups
    (one or few scales per row, whose scale rows are not 16-byte multiples).
    At 16 < M <= 64 the int8 kernel sums whole-chunk groups (G % 256 == 0:
    768 = 3 chunks, per-channel) before scaling and scales other groups
    (384, 128, ...) every chunk; each workgroup starts at a different chunk,
    so the group walks wrap.  int4 G = 16 takes the skinny kernel."""
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=3 * M + N + K)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M,N,K,G", [(96, 160, 256, 128), (130, 64, 512, 32), (256, 256, 1024, 64),
                                     (300, 200, 576, 64)])
def test_matmul_prefill_small(policy, wbits, M, N, K, G):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=M + N + K)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


def test_int8_prefill_large():
    """W8A16 prefill (M = 512, 4096 x 4096, G = 128) on the MFMA GEMM."""
    M, N, K, G = 512, 4096, 4096, 128
    X, W, S = synth.matvec_case(8, M, N, K, G, 0.002, 0.02, seed=8)
    got = _matvec(8, X, W, S, N, K, G, "f16")
    _close(got, _oracle(8, X, W, S, G))


# Decode (M <= 4) with K not a multiple of 2048: the 2048-k segment kernel
# with a partial last segment (k >= K read as zeros through out-of-range
# buffer offsets).
@pytest.mark.parametrize("M,N,K,G", [
    (1, 4096, 11008, 128),    # LLaMA-7B down projection, 5.375 segments
    (1, 333, 2176, 128),      # 1 full + 128-k segment, ragged N
    (2, 640, 11008, 128),
    (3, 96, 6144, 256),
    (4, 257, 14336, 128),     # 7 segments -> 8
    (1, 100, 3200, 640),
    (2, 4096, 4096, 128),     # M = 2 on the segment kernel (whole segments)
    (2, 11008, 4096, 128),    # M = 2 on the segment kernel at cfg 3's N
    (1, 4096, 11008, 32),     # G % 128 != 0: the row kernel at 8 segments
    (1, 300, 14336, 64),
    (2, 11008, 4096, 32),     # M = 2, G % 128 != 0: the row kernel, 2 segments
    (2, 333, 3200, 64),       # ragged, partial second segment
    (2, 1000, 5120, 128),     # M = 2, 2.5 segments -> 4
])
def test_matvec_int4_partial_segment(M, N, K, G):
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=M + N + K)
    got = _matvec(4, X, W, S, N, K, G, "f16")
    _close(got, _oracle(4, X, W, S, G))


# Both sides of every int4 M <= 2 routing limit (the kernel choice changes at
# each): M = 1 K = 8192 / 8448 (row kernel at 4 / 8 segments), K = 16384 /
# 16512 (row kernel's last K, then the ring tile kernel), N = 8192 / 8193 at
# K > 12288 with G % 128 == 0 (segment kernel, then the ring), M = 2 K = 4096 /
# 4160 with G % 128 != 0 (row kernel, then the ring), M = 2 K = 2048 / 4096
# with G = 128 (ring, then the segment kernel).
@pytest.mark.parametrize("M,N,K,G", [
    (1, 300, 8192, 32), (1, 300, 8448, 32), (1, 200, 16384, 32), (1, 200, 16512, 32),
    (1, 8192, 12416, 128), (1, 8193, 12416, 128), (1, 8193, 8448, 128),
    (2, 500, 4096, 64), (2, 500, 4160, 64), (2, 700, 2048, 128), (2, 700, 4096, 128),
    # M = 1 segment counts 3 and 6 (1, 2, 4 rows per wave), 8 at 1 or 2 rows
    # per wave, and N > 8192 on 6 segments / on the ring at 7
    (1, 4096, 6144, 128), (1, 8192, 5120, 128), (1, 2000, 11008, 128), (1, 4100, 10240, 256),
    (1, 11008, 11008, 128), (1, 4096, 14336, 128), (1, 300, 16384, 128), (1, 8200, 12416, 128),
    # M = 3, 4 at N <= 2048, 2048 < K <= 4096: the segment kernel (M = 4
    # instantiation), the ring at N = 2049 and at K = 2048
    (3, 1024, 4096, 128), (4, 2048, 3072, 256), (4, 2049, 4096, 128), (4, 1000, 2048, 128),
    # the row kernel (G % 128 != 0) at 3 (2 / 4 rows per wave) and 6 segments
    (1, 4096, 6144, 32), (1, 8192, 5120, 64), (1, 2000, 11008, 32), (1, 5000, 12288, 96),
])
def test_matvec_int4_route_limits(M, N, K, G):
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=M + N + K + G)
    got = _matvec(4, X, W, S, N, K, G, "f16")
    _close(got, _oracle(4, X, W, S, G))


# LDS-ring tile kernel with a partial last 512-byte row chunk (zeros past the
# row end through out-of-range buffer offsets, activations zeroed past K).
@pytest.mark.parametrize("wbits,M,N,K,G", [
    (4, 4, 640, 11008, 128),     # 5504-byte rows: 10 chunks + 384 bytes
    (4, 16, 300, 4128, 32),      # 2064-byte rows: 16 bytes in the last chunk
    (4, 3, 257, 5120 + 96, 32),  # 2608-byte rows
    (8, 1, 1000, 11008, 128),    # int8 M = 1 takes this kernel too
    (8, 8, 333, 2064, 16),
    (8, 2, 130, 11008, 11008),   # per-channel
])
def test_matvec_tile_partial_chunk(wbits, M, N, K, G):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=M + N + K + wbits)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


@pytest.mark.parametrize("wbits,G", [(4, 32), (4, 64), (8, 16), (8, 64), (8, 128)])
@pytest.mark.parametrize("sd,od", [("bf16", "f16"), ("f16", "bf16"), ("bf16", "bf16"), ("bf16", "f32")])
@pytest.mark.parametrize("M,N", [(1, 1001), (4, 333), (16, 130), (40, 257)])
def test_matvec_bf16_scales_or_output_groups(wbits, G, sd, od, M, N):
    """bf16 scales / outputs with int4 and int8 weights, the tile kernels'
    multi-group scale reads (2 or 4 groups per wave eighth), the (bf16
    scales, fp32 output) pair, and ragged N whose scale array is not a whole
    number of dwords for odd N (those shapes take the kernels that read
    scales per element)."""
    K = 2048
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=M + N + G + wbits)
    S = S.astype(np.float32)
    if sd == "bf16":
        S_used = ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(S)).reshape(S.shape)
        Sg = _up(S, "bf16")
    else:
        S_used = S.astype(np.float16).astype(np.float32)
        Sg = _up(S.astype(np.float16))
    Og = lq.empty((M, N), _dtype(od))
    if wbits == 4:
        lq.dequant_matvec_int4[(N,), (128,)](_up(X), _up(W), Sg, Og, K, K // 2, K // G, G)
    else:
        lq.dequant_matvec_int8[(N,), (128,)](_up(X), _up(W), Sg, Og, K, K // G, G)
    got = Og.numpy()
    got = ref.bf16_bits_to_f32(got).reshape(M, N) if od == "bf16" else got.astype(np.float32)
    want = _oracle(wbits, X, W, S_used, G)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("sd,od", [("bf16", "f16"), ("f16", "bf16"), ("bf16", "bf16"), ("f32", "bf16")])
@pytest.mark.parametrize("M,N,K", [(1, 1000, 4096), (1, 300, 6144), (3, 200, 2048), (4, 1000, 4096),
                                   (16, 300, 2048), (1, 200, 11008), (40, 300, 2048)])
def test_matvec_int4_bf16_scales_or_output(sd, od, M, N, K):
    """bf16 scales and/or bf16 outputs (M = 1: the segment kernel, partial
    segments included, or the LDS-ring tile kernel for K > 8192; M >= 2: the
    tile kernel, or the LDS / skinny kernels for fp32-with-bf16 mixes).  The oracle uses
    the bf16-rounded scales; bf16 outputs are compared after widening."""
    G = 128
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=M + N + K)
    S = S.astype(np.float32)
    if sd == "bf16":
        S_used = ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(S)).reshape(S.shape)
        Sg = _up(S, "bf16")
    elif sd == "f16":
        S_used = S.astype(np.float16).astype(np.float32)
        Sg = _up(S.astype(np.float16))
    else:
        S_used = S
        Sg = _up(S)
    Og = lq.empty((M, N), _dtype(od))
    lq.dequant_matvec_int4[(N,), (128,)](_up(X), _up(W), Sg, Og, K, K // 2, K // G, G)
    got = Og.numpy()
    got = ref.bf16_bits_to_f32(got).reshape(M, N) if od == "bf16" else got.astype(np.float32)
    want = ref.fast_numpy_matvec_int4(X, W, S_used, G)
    # the 1e-2 bar holds for bf16 outputs too (their rounding adds 2^-9 relative)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


# Split-K prefill (fewer 128 x 128 output tiles than CUs): k split 8, 6, 4
# ways, fp32 partial slices reduced in order; odd M x N takes the scalar tail
# of the reduction.  Cases run back to back, so the cached workspace grows.
@pytest.mark.parametrize("wbits,M,N,K,G,od", [
    (4, 67, 301, 1024, 64, "f16"),       # 3 tiles, 4 splits, odd M x N
    (4, 100, 640, 1536, 32, "f32"),      # 5 tiles, 6 splits
    (8, 100, 640, 1536, 128, "f16"),     # int8: 6 splits of 256 k (whole groups)
    (4, 128, 4096, 4096, 128, "f16"),    # 32 tiles, 8 splits
    (8, 128, 4096, 4096, 128, "f32"),
    (4, 300, 2048, 2048, 128, "f16"),    # 48 tiles, 4 splits
    (8, 96, 4096, 11008, 128, "f16"),    # 86 scale groups > LDS: uneven splits, groups straddle splits
    (8, 256, 640, 4096, 4096, "f32"),    # per-channel: splits shorter than the group
    (8, 130, 384, 4096, 64, "f16"),      # 64 groups: fit without a forced split
    # int8 with G % 64 == 32 (scales after a 32-k half), split and unsplit
    (8, 100, 640, 1536, 32, "f16"),
    (8, 2048, 1024, 1920, 96, "f16"),
    # uneven runs (the last split shorter): 172 steps in 8, 65 in 6, 79 in 8
    (4, 96, 4096, 11008, 32, "f16"),
    (4, 100, 640, 4160, 32, "f32"),
    (8, 200, 1000, 5056, 64, "f16"),     # int8 post-scales: groups straddle uneven splits
    (8, 70, 4096, 14336 - 64, 14336 - 64, "f16"),   # per channel, 223 steps in 8
])
def test_matmul_prefill_split_k(wbits, M, N, K, G, od):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=M * 7 + N + K)
    got = _matvec(wbits, X, W, S, N, K, G, od)
    _close(got, _oracle(wbits, X, W, S, G), fp32=False)


def test_int8_prefill_forced_split_big_tiles():
    """256-row tiles with more int8 scale groups (65) than LDS stages: K is
    split in two although the tiles fill the CUs (every output checked)."""
    M, N, K, G = 2048, 4096, 8320, 128
    X, W, S = synth.matvec_case(8, M, N, K, G, 0.002, 0.02, seed=12)
    got = _matvec(8, X, W, S, N, K, G, "f16")
    _close(got, _oracle(8, X, W, S, G))


@pytest.mark.parametrize("wbits", [4, 8])
def test_prefill_big_tiles_split_two(wbits):
    """128 <= 256-row tiles < 256 CUs: 256 x 128 tiles with k split in two
    (every output checked)."""
    M, N, K, G = 1024, 4096, 2048, 128
    X, W, S = synth.matvec_case(wbits, M, N, K, G, 0.001, 0.01, seed=21 + wbits)
    got = _matvec(wbits, X, W, S, N, K, G, "f16")
    _close(got, _oracle(wbits, X, W, S, G))


def test_release_workspaces_then_split_k_again():
    """Freeing the cached split-K workspace (and the SiLU staging one) leaves
    later calls correct: they allocate again."""
    M, N, K, G = 128, 2048, 4096, 128
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=31)
    first = _matvec(4, X, W, S, N, K, G, "f16")
    lq.release_workspaces()
    again = _matvec(4, X, W, S, N, K, G, "f16")
    assert np.array_equal(first.view(np.uint16), again.view(np.uint16))
    _close(again, _oracle(4, X, W, S, G))
    lq.release_workspaces()


def test_matmul_prefill_split_k_graph():
    """Split-K GEMM + reduction captured in a graph: every replay (with eager
    work and synchronisations between them) matches the eager result."""
    import torch
    M, N, K, G = 96, 1024, 2048, 128
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=3)
    Xg, Wg, Sg = _up(X), _up(W), _up(S)
    Og = lq.empty((M, N), np.float16)
    run = lambda: lq.dequant_matvec_int4[(N,), (128,)](Xg, Wg, Sg, Og, K, K // 2, K // G, G)
    st = torch.cuda.Stream()
    st.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(st):
        run()                                     # eager: sizes the workspace
    torch.cuda.synchronize()
    eager = Og.numpy().copy()
    _close(eager, _oracle(4, X, W, S, G))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        run()
    for _ in range(3):
        Og.torch.fill_(0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(Og.numpy(), eager)


def test_cfg1_w8a32_fp32():
    c = synth.CFG1
    X, W, S = synth.matvec_case(8, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"],
                                x_dtype=np.float32, s_dtype=np.float32)
    got = _matvec(8, X, W, S, c["N"], c["K"], c["G"], "f32")
    _close(got, _oracle(8, X, W, S, c["G"]), fp32=True)


@pytest.mark.parametrize("M", [1, 4, 16])
def test_cfg3_gemv_w4a16_full(M):
    c = synth.CFG3
    X, W, S = synth.matvec_case(4, M, c["N"], c["K"], c["G"], c["lo"], c["hi"])
    got = _matvec(4, X, W, S, c["N"], c["K"], c["G"], "f16")
    _close(got, _oracle(4, X, W, S, c["G"]))


def test_cfg4_w8a16_m64_full():
    c = synth.CFG4
    X, W, S = synth.matvec_case(8, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"])
    got = _matvec(8, X, W, S, c["N"], c["K"], c["G"], "f16")
    _close(got, _oracle(8, X, W, S, c["G"]))


def test_cfg5a_prefill_full():
    c = synth.CFG5A
    X, W, S = synth.matvec_case(4, c["M"], c["N"], c["K"], c["G"], c["lo"], c["hi"])
    got = _matvec(4, X, W, S, c["N"], c["K"], c["G"], "f16")
    _close(got, _oracle(4, X, W, S, c["G"]))     # every output (BLAS on the host)


# Prefill on the 128 x 256 pair-split kernel (int4 weights, fp16 activations,
# at least 256 tiles, K % 128 == 0, power-of-two G >= 16): ragged tiles in
# both dimensions, output rows that are not 16-byte multiples (element
# stores), both LDS splits (scale rows within 32 KB: four activation units;
# within 64 KB: three), odd unit counts, fp32 / bf16 scales and outputs, more
# workgroups than CUs with a tile count that is not a multiple of 8.
@pytest.mark.parametrize("M,N,K,G,sd,od", [
    (2000, 4100, 1024, 64, "f16", "f16"),
    (1100, 8192, 640, 32, "f32", "f32"),
    (2048, 4096, 4096, 32, "bf16", "bf16"),
    (1024, 8192, 2048, 16, "f16", "f16"),
    (1030, 8200, 384, 128, "f16", "f32"),
    (2560, 4352, 512, 128, "f16", "bf16"),
])
def test_prefill_pair_kernel(M, N, K, G, sd, od):
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, s_dtype=np.float32, seed=M + N + G)
    if sd == "bf16":
        S_used = ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(S)).reshape(S.shape)
        Sg = _up(S, "bf16")
    else:
        S_used = S.astype(NP_OF[sd]).astype(np.float32)
        Sg = _up(S.astype(NP_OF[sd]))
    Og = lq.empty((M, N), _dtype(od))
    lq.dequant_matvec_int4[(N,), (128,)](_up(X), _up(W), Sg, Og, K, K // 2, K // G, G)
    got = Og.numpy()
    if od == "bf16":
        got = ref.bf16_bits_to_f32(got).reshape(M, N)
    _close(got, _oracle(4, X, W, S_used, G))


def test_reference_fp32_matvec_api():
    """examples/38_quantized_matmul.py:312-321 flow: quantize_int4, then gpu_matvec_int4."""
    rng = np.random.default_rng(42)
    for N, K in [(256, 256), (512, 512)]:
        w = rng.standard_normal((N, K)).astype(np.float32) * 0.1
        x = rng.standard_normal(K).astype(np.float32) * 0.1
        wp, s = ref.quantize_int4(w, 32)
        got = lq.gpu_matvec_int4(x, wp, s, 32)
        _close(got, ref.fast_numpy_matvec_int4(x, wp, s, 32), fp32=True)
        w8, s8 = ref.quantize_int8(w, 32)
        got8 = lq.gpu_matvec_int8(x, w8, s8, 32)
        _close(got8, ref.fast_numpy_matvec_int8(x, w8, s8, 32), fp32=True)


def test_empty_and_zero_k():
    Og = lq.zeros((2, 3), np.float16)
    Og.torch.fill_(7)
    lq.dequant_matvec_int4[(3,), (128,)](lq.empty(0, np.float16), lq.empty(0, np.uint8),
                                         lq.empty(0, np.float16), Og, 0, 0, 0, 32)
    assert (Og.numpy() == 0).all()
    # N = 0: nothing launched, no error
    lq.dequant_int4[(0,), (128,)](lq.empty(0, np.uint8), lq.empty(0, np.float16),
                                  lq.empty(0, np.float16), 64, 32, 2, 32)


@pytest.mark.parametrize("M,K", [(1, 512), (4, 512), (1, 4096), (16, 2048), (128, 512)])
def test_all_q8_gives_zero(M, K):
    """All weights q = 8 -> zero output.  The decode kernels carry a +1032
    (or +1152) bias through the MFMA and subtract BIAS * sum(x) afterwards,
    so the result is zero up to fp32 cancellation (|Y| < 1e-4 here)."""
    N, G = 48, 128
    W = np.full((N, K // 2), 0x88, np.uint8)
    S = np.full((N, K // G), 0.01, np.float16)
    X = np.random.default_rng(1).standard_normal((M, K)).astype(np.float16)
    got = _matvec(4, X, W, S, N, K, G, "f16").astype(np.float32)
    assert np.abs(got).max() < 1e-4


def test_smollm2_layer_shapes_int4_g32():
    """One SmolLM2-135M layer's seven linears (int4 g32, M = 1) and the LM head
    over the tied embeddings (49152 x 576, examples/54_smollm2_inference.py:31,
    573-574)."""
    from locomp_amd import synth as sy
    for i, (N, K) in enumerate(sy.SMOLLM2_LAYER + [(49152, 576)]):
        X, W, S = sy.matvec_case(4, 1, N, K, 32, 0.001, 0.01, seed=100 + i)
        got = _matvec(4, X, W, S, N, K, 32, "f16")
        _close(got, _oracle(4, X, W, S, 32))


# ------------------------------------------------- fused SiLU * mul (MLP) --

def _silu_mul_oracle(X, Wg, Sg, Wu, Su, G):
    """silu(g) * u of examples/54_smollm2_inference.py:113-120 in float64 on
    the oracle's matvecs, and the error bound that the matmul bar (1e-2 on g
    and on u) allows after the product: 1e-2 * (|silu(g)| + |u| * max|silu'|
    + 1) plus 1e-2 relative (silu' is at most 1.1)."""
    g = np.asarray(ref.fast_numpy_matvec_int4(X, Wg, Sg, G), np.float64)
    u = np.asarray(ref.fast_numpy_matvec_int4(X, Wu, Su, G), np.float64)
    silu = g / (1.0 + np.exp(-g))
    want = silu * u
    bound = 1e-2 * (np.abs(silu) + 1.1 * np.abs(u) + 1.0) + 1e-2 * np.abs(want)
    return want, bound


@pytest.mark.parametrize("M,I,K,G,xd", [
    (1, 1536, 576, 32, "f16"),      # SmolLM2 gate|up, row-contiguous kernel
    (2, 100, 576, 32, "f16"),
    (3, 64, 512, 64, "f16"),        # M > 2: generic kernel
    (1, 48, 256, 16, "f16"),        # G % 32 != 0: generic kernel
    (2, 40, 128, 32, "f32"),        # fp32 activations: generic kernel
    (4, 1536, 2048, 32, "f16"),     # 2 <= M <= 16: LDS-ring tile kernel epilogue
    (16, 520, 1024, 128, "f16"),    # ragged last tile (1040 rows)
    (3, 300, 4128, 32, "f16"),      # tile kernel, partial last chunk
    (32, 1000, 1024, 128, "f16"),   # 16 < M <= 64: activation-in-LDS kernel epilogue
    (64, 520, 768, 32, "f16"),
    (96, 600, 1024, 32, "f16"),     # prefill GEMM epilogue, k split
    (300, 1100, 512, 64, "f16"),    # prefill GEMM epilogue, ragged tiles
    (2048, 2048, 1024, 64, "f16"),  # 128 x 256 pair-split kernel epilogue (staged stores)
    (2000, 2050, 512, 32, "f16"),   # pair-split kernel, ragged tiles (element stores)
    (1100, 2048, 1024, 128, "f16"), # 256-row tiles
    (40, 300, 576, 32, "f16"),      # no fused kernel: staged fp32 matvec + pairwise epilogue
    (1, 700, 11008, 32, "f16"),     # row kernel at 6 segments with the epilogue
    (1, 4100, 6144, 32, "f16"),     # row kernel at 3 segments, 4 rows per wave
    (1, 300, 14336, 64, "f16"),     # row kernel at 8 segments
    (8, 100, 576, 64, "f16"),
])
def test_matvec_int4_silu_mul(policy, M, I, K, G, xd):
    dt = np.float16 if xd == "f16" else np.float32
    Xa, Wg, Sg = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=dt, seed=I + K)
    _, Wu, Su = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=dt, seed=I + K + 1)
    W = lq.interleave_gate_up(Wg, Wu)
    S = lq.interleave_gate_up(Sg, Su)
    got = lq.gpu_matvec_int4_silu_mul(Xa, W, S, G).astype(np.float64)
    want, bound = _silu_mul_oracle(Xa, Wg, Sg, Wu, Su, G)
    err = np.abs(got - want)
    assert (err <= bound).all(), (err.max(), np.argmax(err - bound))


@pytest.mark.parametrize("M,I,K,G", [(1, 1536, 576, 32), (4, 700, 2048, 128), (40, 300, 2048, 64),
                                     (130, 256, 1024, 128),
                                     (2, 700, 1024, 32), (1, 3000, 4096, 64)])   # row kernel epilogue
@pytest.mark.parametrize("xd,sd,od", [("f16", "bf16", "bf16"), ("bf16", "f16", "bf16"),
                                      ("bf16", "bf16", "f32"), ("f32", "f32", "f32")])
def test_matvec_int4_silu_mul_other_dtypes(M, I, K, G, xd, sd, od):
    """bf16 scales / outputs and bf16 / fp32 activations: fp16 activations
    with bf16 dtypes take the fast matvec into the staged fp32 buffer, then
    the pairwise epilogue; bf16 / fp32 activations the fused epilogues (row
    kernel, decode kernels, GEMM; fp32 as two bf16 part rows per row)."""
    Xa, Wg, Sg = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                   s_dtype=np.float32, seed=I + K + 7)
    _, Wu, Su = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                  s_dtype=np.float32, seed=I + K + 8)
    used = {"bf16": lambda a: ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(a)).reshape(a.shape),
            "f16": lambda a: a.astype(np.float16).astype(np.float32), "f32": lambda a: a}
    Xu, Sgu, Suu = used[xd](Xa), used[sd](Sg), used[sd](Su)
    W = lq.interleave_gate_up(Wg, Wu)
    S = lq.interleave_gate_up(Sg, Su)
    Xg = _up(Xa, "bf16") if xd == "bf16" else _up(Xa.astype(_dtype(xd)))
    Sdev = _up(S, "bf16") if sd == "bf16" else _up(S.astype(_dtype(sd)))
    got = lq.gpu_matvec_int4_silu_mul(Xg, W, Sdev, G, out_dtype=_dtype(od))
    got = (ref.bf16_bits_to_f32(got).reshape(M, I) if od == "bf16" else got).astype(np.float64)
    want, bound = _silu_mul_oracle(Xu, Wg, Sgu, Wu, Suu, G)
    if od == "bf16":
        bound = bound + 2.0 ** -8 * np.abs(want)
    err = np.abs(got - want)
    assert (err <= bound).all(), (err.max(), np.argmax(err - bound))


@pytest.mark.parametrize("M,I,K,G,xd,sd,od", [
    (4, 1536, 2048, 32, "bf16", "f32", "f32"),     # tile kernel
    (3, 1500, 4128, 32, "bf16", "bf16", "f16"),    # tile kernel, partial last chunk
    (40, 1000, 1024, 128, "bf16", "f16", "bf16"),  # activation-in-LDS kernel
    (96, 600, 1024, 32, "bf16", "f32", "f32"),     # GEMM, k split
    (300, 1100, 512, 64, "bf16", "f16", "f16"),    # GEMM, ragged tiles
    (1, 1536, 6144, 32, "f32", "f32", "f32"),      # 2 part rows, tile kernel (row kernel: K <= 4096)
    (3, 1536, 2048, 32, "f32", "f32", "f32"),      # 6 part rows, tile kernel
    (8, 1000, 2048, 64, "f32", "bf16", "f32"),     # 16 part rows
    (20, 1000, 1024, 128, "f32", "f32", "f16"),    # 40 part rows, activation-in-LDS kernel
    (40, 600, 2048, 64, "f32", "f32", "f32"),      # 80 part rows, GEMM with k split
    (300, 1100, 1024, 32, "f32", "f16", "f32"),    # GEMM, ragged tiles
])
def test_silu_mul_fused_bf16_fp32_activations(M, I, K, G, xd, sd, od):
    """The SiLU * mul epilogue on the bf16 MFMA kernels for bf16 activations
    and for fp32 ones (two round-to-nearest bf16 part rows per row, added at
    the store before the epilogue).  fp32 outputs of fp32 activations are
    held to the fp32 bar: |err| <= 1e-4 (1.1 |u| sum|x w_gate| + |silu(g)|
    sum|x w_up|), the propagated rtol 1e-4 of the gate and up dot products;
    others to the fp16 / bf16 bar of the fp16 epilogue tests."""
    Xa, Wg, Sg = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                   s_dtype=np.float32, seed=I + K + 17)
    _, Wu, Su = synth.matvec_case(4, M, I, K, G, 0.01, 0.05, x_dtype=np.float32,
                                  s_dtype=np.float32, seed=I + K + 18)
    used = {"bf16": lambda a: ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(a)).reshape(a.shape),
            "f16": lambda a: a.astype(np.float16).astype(np.float32), "f32": lambda a: a}
    Xu, Sgu, Suu = used[xd](Xa), used[sd](Sg), used[sd](Su)
    W = lq.interleave_gate_up(Wg, Wu)
    S = lq.interleave_gate_up(Sg, Su)
    Xg = _up(Xa, "bf16") if xd == "bf16" else _up(Xa)
    Sdev = _up(S, "bf16") if sd == "bf16" else _up(S.astype(_dtype(sd)))
    got = lq.gpu_matvec_int4_silu_mul(Xg, W, Sdev, G, out_dtype=_dtype(od))
    got = (ref.bf16_bits_to_f32(got).reshape(M, I) if od == "bf16" else got).astype(np.float64)
    want, bound = _silu_mul_oracle(Xu, Wg, Sgu, Wu, Suu, G)
    if od == "bf16":
        bound = bound + 2.0 ** -8 * np.abs(want)
    if xd == "f32" and od == "f32":
        def deq(Wp, Sp):
            q = np.empty((Wp.shape[0], K), np.float64)
            q[:, 0::2] = (Wp & 15).astype(np.float64) - 8
            q[:, 1::2] = (Wp >> 4).astype(np.float64) - 8
            return q * np.repeat(Sp.astype(np.float64), G, axis=1)
        X64 = Xu.astype(np.float64)
        Dg, Du = deq(Wg, Sgu), deq(Wu, Suu)
        g, u = X64 @ Dg.T, X64 @ Du.T
        silu = g / (1.0 + np.exp(-g))
        want = silu * u
        bound = 1e-4 * (1.1 * np.abs(u) * (np.abs(X64) @ np.abs(Dg).T) +
                        np.abs(silu) * (np.abs(X64) @ np.abs(Du).T)) + 1e-12
    err = np.abs(got - want)
    assert (err <= bound).all(), (err.max(), np.argmax(err - bound))


def test_decode_gemm_route_in_graph_on_a_fresh_stream():
    """16 < M <= 64 at N = 4096 with long rows takes the split-K GEMM only
    when its workspace exists: a capture on a fresh stream (no workspace, no
    allocation under capture) runs the decode kernel instead.  The graph is
    replayed three times with eager calls (which take the GEMM) on the
    default stream in between; every result must match the oracle."""
    import ctypes

    import torch

    from locomp_amd import _lib

    lib = _lib.load()
    vp = ctypes.c_void_p
    M, N, K, G = 48, 4096, 11008, 128
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=91)
    want = _oracle(4, X, W, S, G)
    Xd, Wd, Sd = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (X, W, S))
    Od = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    Oe = torch.zeros((M, N), dtype=torch.float16, device="cuda")

    def call(out, stream):
        return lib.locomp_amd_dequant_matvec_int4(
            vp(Xd.data_ptr()), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(out.data_ptr()), K, K // 2,
            K // G, G, N, M, _lib.F16, _lib.F16, _lib.F16, vp(stream.cuda_stream))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        assert call(Od, s) == 0
    torch.cuda.synchronize()
    for _ in range(3):
        Od.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert call(Oe, torch.cuda.current_stream()) == 0   # eager work between replays
        torch.cuda.synchronize()
        _close(Od.cpu().numpy(), want)
        _close(Oe.cpu().numpy(), want)
