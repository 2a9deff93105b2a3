"""GPU parity for bf16 and fp32 activations (the reference's own kernels take
fp32 `locomp.Tensor` activations, examples/38_quantized_matmul.py:30-40, and
its frontend types bf16 parameters as locomp.BFloat16, locomp/frontend.py:53).

Both run on bf16 MFMAs with exact integer weights and fp32 group scales:
bf16 activations as given, fp32 ones split into bf16 parts: three exact
parts on the row and tile kernels (M <= 4), two round-to-nearest parts
(residual <= 2^-16 |x|) on the M = 1 segment kernel and beyond four rows.
The oracle is the restated reference NumPy path on the same values (bf16
activations widened exactly to fp32).  Bars: rtol / atol 1e-2 for bf16
activations; rtol 1e-4 (+ atol 1e-5 max|Y|) for fp32.
"""

import numpy as np
import pytest

from locomp_amd import synth
from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

lq = pytest.importorskip("locomp_amd")


def _bf16_round(a):
    return ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(np.asarray(a, np.float32))).reshape(np.shape(a))


def _dev(a, name):
    if name == "bf16":
        return lq.tensor(np.asarray(a, np.float32), dtype=lq.bfloat16)
    return lq.tensor(np.ascontiguousarray(a.astype({"f32": np.float32, "f16": np.float16}[name])))


def _run(wbits, X, W, S, N, K, G, xd, sd, od):
    M = X.shape[0]
    Og = lq.empty((M, N), lq.bfloat16 if od == "bf16" else {"f32": np.float32, "f16": np.float16}[od])
    Xg, Sg = _dev(X, xd), _dev(S, sd)
    if wbits == 4:
        lq.dequant_matvec_int4[(N,), (128,)](Xg, lq.tensor(W), Sg, Og, K, K // 2, K // G, G)
    else:
        lq.dequant_matvec_int8[(N,), (128,)](Xg, lq.tensor(W), Sg, Og, K, K // G, G)
    got = Og.numpy()
    if od == "bf16":
        return ref.bf16_bits_to_f32(got).reshape(M, N)
    return got.astype(np.float32)


def _used(a, name):
    """The values the kernel sees for an array uploaded as `name`."""
    if name == "bf16":
        return _bf16_round(a)
    if name == "f16":
        return np.asarray(a).astype(np.float16).astype(np.float32)
    return np.asarray(a, np.float32)


def _oracle(wbits, X, W, S, G):
    f = ref.fast_numpy_matvec_int4 if wbits == 4 else ref.fast_numpy_matvec_int8
    return f(X, W, S, G)


def _case(wbits, M, N, K, G, seed, lo=0.001, hi=0.01):
    X, W, S = synth.matvec_case(wbits, M, N, K, G, lo, hi, x_dtype=np.float32,
                                s_dtype=np.float32, seed=seed)
    return X, W, S


# ------------------------------------------------------------- bf16 X --

@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M", [1, 4, 16])
def test_bf16_activations_cfg3(wbits, M):
    """BASELINE cfg 3 shape (11008 x 4096, G = 128) with bf16 activations and
    bf16 outputs, full output against the oracle."""
    N, K, G = 11008, 4096, 128
    X, W, S = _case(wbits, M, N, K, G, seed=M + wbits)
    got = _run(wbits, X, W, S, N, K, G, "bf16", "f16", "bf16")
    want = _oracle(wbits, _used(X, "bf16"), W, _used(S, "f16"), G)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("wbits,M,N,K,G", [
    (4, 2, 300, 2048, 32),       # two / four scale groups per wave eighth
    (4, 5, 257, 4096, 64),
    (4, 3, 640, 11008, 128),     # partial last 512-byte chunk
    (4, 16, 96, 1024, 1024),
    (8, 1, 1000, 4096, 4096),    # per-channel
    (8, 7, 333, 2064, 16),       # partial chunk, 16-k groups
    (8, 16, 130, 11008, 128),
    (8, 2, 64, 1536, 64),
    (4, 33, 640, 2048, 64),      # 16 < M <= 64: the activation-in-LDS kernel, bf16 MFMAs
    (4, 64, 1000, 4096, 128),
    (4, 20, 11008, 1024, 32),
    (8, 40, 300, 2048, 128),
    (8, 24, 4100, 1536, 512),
    (8, 64, 257, 1024, 1024),    # per channel: raw sums over the whole row
    (4, 1, 300, 6144, 128),      # segment kernel at 3 / 6 / 8 segments, 2 rows per wave
    (4, 1, 257, 11008, 128),
    (4, 1, 130, 14336, 256),
])
@pytest.mark.parametrize("sd,od", [("f16", "f16"), ("bf16", "bf16"), ("f32", "f32"), ("f16", "bf16")])
def test_bf16_activations_shapes(wbits, M, N, K, G, sd, od):
    X, W, S = _case(wbits, M, N, K, G, seed=M * 7 + N + K)
    got = _run(wbits, X, W, S, N, K, G, "bf16", sd, od)
    want = _oracle(wbits, _used(X, "bf16"), W, _used(S, sd), G)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("wbits,M,N,K,G", [
    (4, 2048, 4096, 4096, 128),   # BASELINE cfg 5a with bf16 activations
    (4, 128, 4096, 4096, 128),    # split-K (8 ways)
    (8, 512, 4096, 4096, 128),
    (4, 96, 200, 1024, 64),
    (8, 300, 257, 2048, 2048),
    (4, 100, 640, 4160, 64),      # split-K with a shorter last split
    (8, 96, 1024, 11008, 128),
    (4, 2048, 1536, 576, 32),     # G = 32 (SmolLM2): scales after each 32-k half
    (8, 200, 500, 2048, 32),
    (4, 300, 700, 1536, 96),      # G = 96: groups end mid-step
    (8, 130, 4096, 4096, 32),     # 128 groups: split K so each split's groups fit LDS
])
def test_bf16_activations_prefill(wbits, M, N, K, G):
    """bf16 prefill on the MFMA GEMM (bf16 MFMAs on exact integer weights,
    fp32 group scales), every output row against the oracle."""
    X, W, S = _case(wbits, M, N, K, G, seed=M + N + wbits)
    got = _run(wbits, X, W, S, N, K, G, "bf16", "f16", "bf16")
    want = _oracle(wbits, _used(X, "bf16"), W, _used(S, "f16"), G)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


# ------------------------------------------------------------- fp32 X --

def _close32(got, want):
    atol = 1e-5 * max(1.0, float(np.abs(want).max()))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol)


def test_fp32_activations_cfg1():
    """BASELINE cfg 1 (the reference's CPU config): W8A32, X fp32 [4, 512],
    int8 [512, 512], per-output-channel fp32 scales, fp32 output."""
    rng = np.random.default_rng(0)
    X = rng.standard_normal((4, 512)).astype(np.float32)
    W = rng.integers(-127, 128, (512, 512)).astype(np.int8)
    S = rng.uniform(0.005, 0.02, (512, 1)).astype(np.float32)
    got = _run(8, X, W, S, 512, 512, 512, "f32", "f32", "f32")
    _close32(got, ref.fast_numpy_matvec_int8(X, W, S, 512))


@pytest.mark.parametrize("wbits", [4, 8])
@pytest.mark.parametrize("M", [1, 2, 3, 4])
def test_fp32_activations_cfg3(wbits, M):
    """cfg 3 shape with fp32 activations / scales / outputs (the reference's
    dtypes), full output, rtol 1e-4."""
    N, K, G = 11008, 4096, 128
    X, W, S = _case(wbits, M, N, K, G, seed=10 + M + wbits)
    got = _run(wbits, X, W, S, N, K, G, "f32", "f32", "f32")
    _close32(got, _oracle(wbits, X, W, S, G))


@pytest.mark.parametrize("wbits,M,N,K,G,sd", [
    (4, 1, 333, 2048, 32, "f16"), (4, 4, 100, 11008, 128, "f32"), (4, 3, 640, 4096, 64, "bf16"),
    (8, 2, 257, 2064, 16, "f32"), (8, 4, 96, 4096, 4096, "f16"), (8, 1, 1000, 1024, 128, "f32"),
    (4, 1, 4096, 6144, 128, "f16"), (4, 1, 300, 5120, 256, "f32"), (4, 1, 4097, 6144, 128, "f32")])
def test_fp32_activations_shapes(wbits, M, N, K, G, sd):
    X, W, S = _case(wbits, M, N, K, G, seed=M + N + K)
    X = X * np.float32(3.0)   # values across several binades
    got = _run(wbits, X, W, S, N, K, G, "f32", sd, "f32")
    _close32(got, _oracle(wbits, X, W, _used(S, sd), G))


@pytest.mark.parametrize("wbits,M,N,K,G,sd", [
    (4, 5, 2000, 2048, 64, "f16"),      # 15 part rows: the tile kernel
    (4, 6, 1000, 4096, 128, "f32"),     # 18 part rows: the bf16 GEMM (split K)
    (8, 16, 1100, 1024, 128, "bf16"),
    (4, 64, 1000, 4096, 128, "f16"),
    (8, 300, 640, 2048, 256, "f32"),
    (4, 2048, 4096, 4096, 128, "f16"),  # BASELINE cfg 5a shape with fp32 activations
    (4, 8, 2048, 1024, 32, "f16"),      # G = 32: the GEMM scales after each 32-k half
    (8, 40, 600, 1152, 96, "f32"),      # G = 96: groups end mid-step and at step ends
    (4, 16, 576, 576, 32, "f16"),       # < 2^24 multiply-adds: the generic kernel
    (8, 7, 3000, 4096, 128, "f16"),     # int8, 14 part rows: the tile kernel
    (8, 20, 1000, 2048, 64, "f32"),     # int8, 40 part rows: the activation-in-LDS kernel
    (4, 24, 4096, 11008, 128, "f16"),   # 48 part rows, long rows at N = 4096: the split-K GEMM
])
def test_fp32_activations_beyond_four_rows(wbits, M, N, K, G, sd):
    """fp32 activations at M > 4: two round-to-nearest bf16 parts per row as
    2 M rows on the bf16 route: the tile kernels with fp32 products and a
    second launch adding the part rows (2 M <= 64), else the MFMA GEMM adding
    them in its epilogue (M = 40: k split, partial sums of the pair sums);
    full output against the oracle at rtol 1e-4."""
    X, W, S = _case(wbits, M, N, K, G, seed=M + N + K + wbits)
    X = X * np.float32(3.0)
    got = _run(wbits, X, W, S, N, K, G, "f32", sd, "f32")
    _close32(got, _oracle(wbits, X, W, _used(S, sd), G))


@pytest.mark.parametrize("od", ["f16", "bf16"])
def test_fp32_activations_beyond_four_rows_low_precision_out(od):
    M, N, K, G = 40, 700, 2048, 128
    X, W, S = _case(4, M, N, K, G, seed=5)
    got = _run(4, X, W, S, N, K, G, "f32", "f16", od)
    want = _oracle(4, X, W, _used(S, "f16"), G)
    np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("xd", ["bf16", "f32"])
@pytest.mark.parametrize("M,N,K,G,sd,od", [
    (1, 576, 576, 32, "f16", "f16"),      # SmolLM2 shapes (the tile kernel's rows are too short)
    (1, 576, 1536, 32, "bf16", "f32"),
    (1, 3072, 576, 32, "f32", "bf16"),
    (2, 960, 576, 32, "f16", "f32"),      # bf16 M = 2 (fp32 M = 2 takes the tile kernel)
    (1, 2048, 2048, 64, "f16", "f16"),
    (1, 300, 4032, 96, "f32", "f32"),     # 2 segments
    (1, 1000, 6144, 32, "f16", "f16"),    # bf16: 3 segments (fp32 K > 4096: tile kernel)
    (1, 257, 11008, 32, "f16", "f16"),    # bf16: 6 segments, partial
    (2, 333, 3200, 64, "bf16", "bf16"),
    (4, 576, 576, 32, "f16", "f32"),      # M = 3, 4 on short rows: four activation rows per lane
    (3, 1536, 1536, 64, "bf16", "f16"),
])
def test_row_kernel_bf16_fp32_activations(xd, M, N, K, G, sd, od):
    """The row kernel (M <= 2, G % 32) with bf16 / fp32 activations: bf16
    weights 128 + q and v_dot2_f32_bf16, fp32 as three exact bf16 parts; fp32
    outputs at rtol 1e-4, others at 1e-2."""
    X, W, S = _case(4, M, N, K, G, seed=M + N + K + G)
    got = _run(4, X, W, S, N, K, G, xd, sd, od)
    want = _oracle(4, _used(X, xd), W, _used(S, sd), G)
    if xd == "f32" and od == "f32":
        _close32(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2)


def test_fp32_split_is_exact_on_hard_values():
    """Activations with 24 significant bits, tiny and huge magnitudes: the
    three-part split must reproduce fp32 products (one weight row of ones,
    so Y = scale * sum(x) is known in float64)."""
    rng = np.random.default_rng(5)
    K, N, G = 2048, 32, 2048
    X = (rng.standard_normal((1, K)) * np.exp2(rng.integers(-20, 20, (1, K)))).astype(np.float32)
    W = np.full((N, K), 1, np.int8)
    S = np.ones((N, 1), np.float32)
    got = _run(8, X, W, S, N, K, G, "f32", "f32", "f32")
    want = np.full((1, N), X.astype(np.float64).sum(), np.float64)
    scale = np.abs(X.astype(np.float64)).sum()
    # one bf16 part would err by ~2^-9 of the largest terms (~1e-3 of scale)
    assert np.abs(got - want).max() <= 2e-5 * scale


@pytest.mark.parametrize("K", [576, 2048, 4096])
def test_fp32_row_kernel_on_hard_values(K):
    """The row kernel's fp32 path (int4, G = 32: fp32 FMAs on the nibbles as
    floats) on activations spread over 2^40: every weight is q - 8 = 1, so
    Y = sum(x), known in float64; the error must stay at fp32-accumulation
    size, far below one bf16 rounding of the largest terms."""
    rng = np.random.default_rng(6)
    N, G = 48, 32
    X = (rng.standard_normal((1, K)) * np.exp2(rng.integers(-20, 20, (1, K)))).astype(np.float32)
    W = np.full((N, K // 2), 0x99, np.uint8)
    S = np.ones((N, K // G), np.float32)
    got = _run(4, X, W, S, N, K, G, "f32", "f32", "f32")
    want = np.full((1, N), X.astype(np.float64).sum(), np.float64)
    scale = np.abs(X.astype(np.float64)).sum()
    assert np.abs(got - want).max() <= 2e-5 * scale


def test_fp32_split_is_exact_on_hard_values_m3():
    """The same at M = 3 (the rows are split into bf16 part rows by a separate
    kernel first): row m of X scaled by 2^m, one weight row of ones."""
    rng = np.random.default_rng(6)
    K, N, G, M = 2048, 32, 2048, 3
    X = (rng.standard_normal((M, K)) * np.exp2(rng.integers(-20, 20, (M, K)))).astype(np.float32)
    W = np.full((N, K), 1, np.int8)
    S = np.ones((N, 1), np.float32)
    got = _run(8, X, W, S, N, K, G, "f32", "f32", "f32")
    for m in range(M):
        want = X[m].astype(np.float64).sum()
        assert np.abs(got[m] - want).max() <= 2e-5 * np.abs(X[m].astype(np.float64)).sum()


@pytest.mark.parametrize("M", [8, 64])
def test_fp32_stacked_route_tiny_and_mixed_magnitudes(M):
    """fp32 activations beyond four rows run as two bf16 part rows each
    (hi = RN(x), lo = RN(x - hi)) on the bf16 MFMA route (M = 8: tile kernel,
    products added by a second launch; M = 64: the GEMM, added in its
    epilogue).  Even rows hold activations of magnitude ~1e-36, whose lo
    parts lie below bf16's normal range (2^-126); odd rows spread over
    2^-30 .. 2^30 within the row.  Against the generic fp32 kernel (one fp32
    FMA chain per output) and a float64 oracle, each output stays within
    2e-5 of sum_k |x_k w_nk| of its row: a flushed lo part would err by up
    to 2^-9 of the tiny rows' terms."""
    rng = np.random.default_rng(40 + M)
    N, K, G = 2048, 2048, 32
    X = rng.standard_normal((M, K)).astype(np.float32)
    X[0::2] *= np.float32(1e-36)
    X[1::2] *= np.exp2(rng.integers(-30, 30, (M // 2, K))).astype(np.float32)
    W = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    S = rng.uniform(0.001, 0.01, (N, K // G)).astype(np.float32)
    got = _run(4, X, W, S, N, K, G, "f32", "f32", "f32").astype(np.float64)
    lq.set_policy(1)
    try:
        gen = _run(4, X, W, S, N, K, G, "f32", "f32", "f32").astype(np.float64)
    finally:
        lq.set_policy(0)
    q = np.empty((N, K), np.float64)
    q[:, 0::2] = (W & 15).astype(np.float64) - 8
    q[:, 1::2] = (W >> 4).astype(np.float64) - 8
    Wd = q * np.repeat(S.astype(np.float64), G, axis=1)
    X64 = X.astype(np.float64)
    want = X64 @ Wd.T
    mag = np.abs(X64) @ np.abs(Wd).T
    assert (np.abs(got - want) <= 2e-5 * mag).all(), np.max(np.abs(got - want) / mag)
    assert (np.abs(got - gen) <= 2e-5 * mag).all(), np.max(np.abs(got - gen) / mag)
    assert (np.abs(gen - want) <= 2e-5 * mag).all()


def test_fp32_activations_in_graph_on_a_fresh_stream():
    """A capture on a stream with no workspace yet cannot allocate the part
    rows: the tile kernel then splits the activations itself (a new torch
    stream normally has none; a pooled one reused from an earlier fp32 call
    would run the pre-split path inside the graph instead).  The graph is
    replayed three times with eager calls on the default stream in between;
    every replay must match the oracle (rtol 1e-4)."""
    import ctypes

    import torch

    from locomp_amd import _lib

    lib = _lib.load()
    vp = ctypes.c_void_p
    M, N, K, G = 3, 2000, 4096, 128
    X, W, S = _case(4, M, N, K, G, seed=77)
    want = _oracle(4, X, W, S, G)
    Xd, Wd, Sd = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (X, W, S))
    Od = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    Oe = torch.zeros((M, N), dtype=torch.float32, device="cuda")

    def call(out, stream):
        return lib.locomp_amd_dequant_matvec_int4(
            vp(Xd.data_ptr()), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(out.data_ptr()), K, K // 2,
            K // G, G, N, M, _lib.F32, _lib.F32, _lib.F32, vp(stream.cuda_stream))

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
        _close32(Od.cpu().numpy(), want)
        _close32(Oe.cpu().numpy(), want)


@pytest.mark.parametrize("M", [8, 40])
def test_fp32_activations_beyond_four_rows_in_graph(M):
    """fp32 at M > 4 needs workspaces (part rows; at M = 8 the fp32 products,
    at M = 40 the GEMM's split-K partial sums): a capture on a stream that
    has none takes the generic kernel; after an eager call on the same stream
    the capture takes the split route.  Both graphs are replayed three times
    with eager work in between, every result against the oracle."""
    import ctypes

    import torch

    from locomp_amd import _lib

    lib = _lib.load()
    vp = ctypes.c_void_p
    N, K, G = 2048, 1024, 128
    X, W, S = _case(4, M, N, K, G, seed=78 + M)
    want = _oracle(4, X, W, S, G)
    Xd, Wd, Sd = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (X, W, S))
    Oe = torch.zeros((M, N), dtype=torch.float32, device="cuda")

    def call(out, stream):
        return lib.locomp_amd_dequant_matvec_int4(
            vp(Xd.data_ptr()), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(out.data_ptr()), K, K // 2,
            K // G, G, N, M, _lib.F32, _lib.F32, _lib.F32, vp(stream.cuda_stream))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    for warm in (False, True):
        Od = torch.zeros((M, N), dtype=torch.float32, device="cuda")
        if warm:
            with torch.cuda.stream(s):
                assert call(Od, s) == 0   # sizes the stream's workspaces
            torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            assert call(Od, s) == 0
        torch.cuda.synchronize()
        for _ in range(3):
            Od.zero_()
            g.replay()
            torch.cuda.synchronize()
            assert call(Oe, torch.cuda.current_stream()) == 0
            torch.cuda.synchronize()
            _close32(Od.cpu().numpy(), want)
            _close32(Oe.cpu().numpy(), want)
        del g
