"""Pins the CPU oracle (oracle/quant_ref.py) independently of its own formulas.

The reference ships no golden vectors for this path (its only assertion is the
self-check in examples/52_dequantize.py:146-170), so the oracle is pinned by:
the scalar definition of the reference kernels evaluated element by element,
exhaustive tables, closed forms / special cases, a layout that must fail,
torch's independent bf16 conversion, and the committed fixtures under
tests/golden/ (written by tests/golden/make_golden.py from the brute-force loop
definitions, examples/38_quantized_matmul.py:178-212).
"""

import os

import numpy as np
import pytest

from oracle import quant_ref as ref

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _scalar_dequant_int4(packed, scales, N, K, G):
    """Element-wise scalar reading of the kernel body examples/52_dequantize.py:36-53."""
    out = np.zeros((N, K), np.float32)
    for r in range(N):
        for b in range(K // 2):
            p = int(packed[r, b])
            lo, hi = p & 15, p >> 4
            out[r, 2 * b] = np.float32(float(lo) - 8.0) * np.float32(scales[r, (2 * b) // G])
            out[r, 2 * b + 1] = np.float32(float(hi) - 8.0) * np.float32(scales[r, (2 * b + 1) // G])
    return out


def test_unpack_exhaustive_all_bytes():
    packed = np.arange(256, dtype=np.uint8).reshape(1, 256)
    w = ref.unpack_int4(packed)
    for b in range(256):
        assert w[0, 2 * b] == (b & 15) - 8
        assert w[0, 2 * b + 1] == (b >> 4) - 8


def test_dequant_int4_exhaustive_table_vs_scalar_definition():
    rng = np.random.default_rng(3)
    packed = np.tile(np.arange(256, dtype=np.uint8), (6, 1))            # N=6, K=512
    for sdt in (np.float32, np.float16):
        scales = rng.uniform(1e-4, 3.0, size=(6, 512 // 32)).astype(sdt)
        got = ref.dequant_int4_ref(packed, scales, 6, 512, 32)
        want = _scalar_dequant_int4(packed, scales, 6, 512, 32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_dequant_int4_closed_forms():
    N, K, G = 4, 64, 16
    s = np.full((N, K // G), 0.5, np.float32)
    # q = 8 everywhere -> +0.0 exactly (not -0.0)
    w = ref.dequant_int4_ref(np.full((N, K // 2), 0x88, np.uint8), s, N, K, G)
    assert np.array_equal(w.view(np.uint32), np.zeros((N, K), np.uint32))
    # low nibble is the even k, high nibble the odd k
    p = np.full((N, K // 2), 0xF0, np.uint8)  # lo = 0 -> -8, hi = 15 -> 7
    w = ref.dequant_int4_ref(p, s, N, K, G)
    assert (w[:, 0::2] == -4.0).all() and (w[:, 1::2] == 3.5).all()
    # linearity in the scale (power-of-two factor is exact)
    rng = np.random.default_rng(0)
    pk = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    s1 = rng.uniform(0.01, 1, (N, K // G)).astype(np.float32)
    assert np.array_equal(ref.dequant_int4_ref(pk, 2 * s1, N, K, G),
                          2 * ref.dequant_int4_ref(pk, s1, N, K, G))
    # group g only scales columns [g*G, (g+1)*G)
    s2 = s1.copy(); s2[:, 1] = 0
    w2 = ref.dequant_int4_ref(pk, s2, N, K, G)
    assert (w2[:, G:2 * G] == 0).all()
    assert np.array_equal(w2[:, :G], ref.dequant_int4_ref(pk, s1, N, K, G)[:, :G])


def test_swapped_nibbles_are_detected():
    rng = np.random.default_rng(1)
    pk = rng.integers(0, 256, (3, 16), dtype=np.uint8)
    s = np.ones((3, 1), np.float32)
    swapped = ((pk & 15) << 4) | (pk >> 4)
    assert not np.array_equal(ref.dequant_int4_ref(pk, s, 3, 32, 32),
                              ref.dequant_int4_ref(swapped.astype(np.uint8), s, 3, 32, 32))


def test_dequant_int8_vs_scalar():
    rng = np.random.default_rng(5)
    N, K, G = 5, 48, 16
    q = rng.integers(-128, 128, (N, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.1, (N, K // G)).astype(np.float32)
    got = ref.dequant_int8_ref(q, s, N, K, G)
    for r in range(N):
        for k in range(K):
            assert got[r, k] == np.float32(float(q[r, k])) * s[r, k // G]


@pytest.mark.parametrize("wbits", [4, 8])
def test_fast_matvec_matches_bruteforce_loop(wbits):
    rng = np.random.default_rng(7)
    N, K, G = 12, 64, 16
    x = rng.standard_normal(K).astype(np.float32)
    X = rng.standard_normal((3, K)).astype(np.float32)
    s = rng.uniform(0.001, 0.05, (N, K // G)).astype(np.float32)
    if wbits == 4:
        w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
        fast, slow = ref.fast_numpy_matvec_int4, ref.numpy_matvec_int4
    else:
        w = rng.integers(-127, 128, (N, K), dtype=np.int8)
        fast, slow = ref.fast_numpy_matvec_int8, ref.numpy_matvec_int8
    np.testing.assert_allclose(fast(x, w, s, G), slow(x, w, s, G), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(fast(X, w, s, G), slow(X, w, s, G), rtol=1e-5, atol=1e-6)


def test_matvec_special_cases():
    rng = np.random.default_rng(11)
    N, K, G = 8, 128, 32
    X = rng.standard_normal((2, K)).astype(np.float32)
    s = rng.uniform(0.01, 0.1, (N, K // G)).astype(np.float32)
    # all q = 8 -> zero
    assert (ref.fast_numpy_matvec_int4(X, np.full((N, K // 2), 0x88, np.uint8), s, G) == 0).all()
    # single non-zero group -> textbook dot product of that slice
    pk = np.full((N, K // 2), 0x88, np.uint8)
    pk[:, 16:32] = rng.integers(0, 256, (N, 16), dtype=np.uint8)    # k in [32, 64): group 1
    lo = (pk[:, 16:32] & 15).astype(np.float64) - 8
    hi = (pk[:, 16:32] >> 4).astype(np.float64) - 8
    wq = np.empty((N, 32)); wq[:, 0::2] = lo; wq[:, 1::2] = hi
    want = X[:, 32:64].astype(np.float64) @ (wq * s[:, 1:2].astype(np.float64)).T
    np.testing.assert_allclose(ref.fast_numpy_matvec_int4(X, pk, s, G), want, rtol=1e-5, atol=1e-6)
    # G = K: per-output-channel scale
    w8 = rng.integers(-127, 128, (N, K), dtype=np.int8)
    sc = rng.uniform(0.01, 0.1, (N, 1)).astype(np.float32)
    want = (X.astype(np.float64) @ w8.T.astype(np.float64)) * sc[:, 0].astype(np.float64)
    np.testing.assert_allclose(ref.fast_numpy_matvec_int8(X, w8, sc, K), want, rtol=1e-5, atol=1e-5)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(2)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1e-40, 3.0e38, np.inf, -np.inf], np.float32),
                        # exact halfway cases
                        (np.arange(1, 200, dtype=np.uint32) << 16 | 0x8000).view(np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ref.f32_to_bf16_bits(x), want)
    assert np.array_equal(ref.bf16_bits_to_f32(want), torch.from_numpy(want.view(np.int16)).view(
        torch.bfloat16).float().numpy())


def test_fp16_cast_is_rne_of_fp32_product():
    # fp16 scale * (q - 8) is exact in fp32 (<= 15 significant bits); the oracle's
    # fp16 output is then a single RNE rounding, checked against float64.
    rng = np.random.default_rng(9)
    pk = rng.integers(0, 256, (64, 128), dtype=np.uint8)
    s = rng.uniform(1e-3, 1e-2, (64, 8)).astype(np.float16)
    w32 = ref.dequant_int4_ref(pk, s, 64, 256, 32)
    w64 = ref.unpack_int4(pk).astype(np.float64) * np.repeat(s.astype(np.float64), 32, axis=1)
    assert np.array_equal(w32.astype(np.float64), w64)
    assert np.array_equal(ref.cast_out(w32, "f16"), w64.astype(np.float16))


def test_quantize_round_trip_and_ties():
    rng = np.random.default_rng(4)
    w = rng.standard_normal((16, 128)).astype(np.float32)
    for quant, deq, half_step in (
            (ref.quantize_int4, lambda p, s: ref.dequant_int4_ref(p, s, 16, 128, 32), 0.5),
            (ref.quantize_int4_ref, lambda p, s: ref.dequant_int4_ref(p, s, 16, 128, 32), 0.5),
            (ref.quantize_int8, lambda q, s: ref.dequant_int8_ref(q, s, 16, 128, 32), 0.5)):
        p, s = quant(w, 32)
        err = np.abs(deq(p, s) - w)
        bound = np.repeat(s, 32, axis=1) * half_step * (1 + 1e-5)
        assert (err <= bound).all()
    # ties go to even (np.round): values exactly k + 0.5 scale steps
    g = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5, 0.0] * 4], np.float32)
    p, s = ref.quantize_int4(g, 32)
    assert s[0, 0] == np.float32(1.0)
    q = ref.unpack_int4(p)[0] + 8
    assert list(q[:8]) == [15, 8, 10, 10, 8, 6, 12, 8]
    # all-zero group -> scale 1.0 (examples/38_quantized_matmul.py:263)
    p, s = ref.quantize_int4(np.zeros((1, 32), np.float32), 32)
    assert s[0, 0] == 1.0 and (p == 0x88).all()


def test_quantize_int8_ties_to_even():
    """quantize_int8 (examples/38_quantized_matmul.py:274-291): amax = 127
    makes the scale exactly 1.0, so x.5 values are exact ties; np.round sends
    them to the even integer (half-away-from-zero would give 1, 3, 3, -1, -2,
    127)."""
    g = np.array([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 0.0] * 4], np.float32)
    q, s = ref.quantize_int8(g, 32)
    assert s[0, 0] == np.float32(1.0)
    assert list(q[0, :8]) == [127, 0, 2, 2, 0, -2, 126, 0]
    q, s = ref.quantize_int8(np.zeros((1, 32), np.float32), 32)     # amax 0 -> scale 1
    assert s[0, 0] == 1.0 and (q == 0).all()


def test_quantize_int4_ref_ties_floor_and_bias():
    """quantize_int4_ref (examples/52_dequantize.py:110-126): scale =
    max(amax, 1e-10) / 7 and q = round(w / (scale + 1e-10)) + 8."""
    # ties: amax 7 -> scale 1.0; 1.0 + 1e-10 rounds to 1.0 in float32
    g = np.array([[7.0, 0.5, 1.5, 2.5, -0.5, -1.5, 3.5, 0.0] * 4], np.float32)
    p, s = ref.quantize_int4_ref(g, 32)
    assert s[0, 0] == np.float32(1.0)
    assert list(ref.unpack_int4(p)[0][:8] + 8) == [15, 8, 10, 10, 8, 6, 12, 8]
    # the +1e-10 in the divisor: with amax = 7 u (u = 2^-34, scale u exactly)
    # w / (u + 1e-10) = 7 / (1 + 1e-10 / u) = 7 / 2.718 = 2.575 for w = amax:
    # q = 8 + 3; -amax -> 8 - 3; amax / 2 -> 8 + round(1.288) = 9 (without the
    # term: 15, 1, 12)
    u = np.float32(2.0 ** -34)
    g = np.array([[7 * u, -7 * u, 3.5 * u, 0.0] * 8], np.float32)
    p, s = ref.quantize_int4_ref(g, 32)
    assert s[0, 0] == u
    assert list(ref.unpack_int4(p)[0][:4] + 8) == [11, 5, 9, 8]
    # the 1e-10 floor: an all-zero group keeps a positive scale 1e-10 / 7
    p, s = ref.quantize_int4_ref(np.zeros((1, 32), np.float32), 32)
    assert 1.42e-11 < s[0, 0] < 1.43e-11 and (p == 0x88).all()


def test_golden_fixtures():
    path = os.path.join(GOLDEN, "quant_golden.npz")
    g = np.load(path)  # allow_pickle=False by default
    for tag in ("a", "b"):
        X, W4, S4, W8, S8 = (g[f"{tag}_{k}"] for k in ("X", "W4", "S4", "W8", "S8"))
        G = int(g[f"{tag}_G"])
        N = W4.shape[0]; K = X.shape[1]
        assert np.array_equal(ref.dequant_int4_ref(W4, S4, N, K, G), g[f"{tag}_deq4"])
        assert np.array_equal(ref.dequant_int8_ref(W8, S8, N, K, G), g[f"{tag}_deq8"])
        np.testing.assert_allclose(ref.fast_numpy_matvec_int4(X, W4, S4, G), g[f"{tag}_y4"],
                                   rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(ref.fast_numpy_matvec_int8(X, W8, S8, G), g[f"{tag}_y8"],
                                   rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------- rms norm --

def test_rms_norm_closed_form_constant_rows():
    """A constant row c: rms = 1 / sqrt(c^2 + eps), out = c w / sqrt(c^2 + eps)."""
    K, eps = 576, 1e-5
    w = np.linspace(-2, 2, K).astype(np.float32)
    for c in (0.0, 1.0, -3.5, 1e-3):
        got = ref.rms_norm_ref(np.full((1, K), c, np.float32), w, eps)
        want = c * w.astype(np.float64) / np.sqrt(c * c + eps)
        np.testing.assert_allclose(got[0], want, rtol=1e-6, atol=1e-7)


def test_rms_norm_matches_the_kernel_loops_in_float64():
    """Scalar float64 restatement of examples/54:44-73: strided partial sums of
    squares, total, rsqrt(total / N + eps), val * rms * w."""
    rng = np.random.default_rng(11)
    M, K, eps = 3, 200, 1e-5
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = rng.standard_normal(K).astype(np.float32)
    got = ref.rms_norm_ref(x, w, eps)
    for m in range(M):
        parts = [0.0] * 128
        for tid in range(128):
            for i in range(tid, K, 128):
                parts[tid] += float(x[m, i]) ** 2
        rms = 1.0 / np.sqrt(sum(parts) / K + eps)
        want = [float(x[m, i]) * rms * float(w[i]) for i in range(K)]
        np.testing.assert_allclose(got[m], want, rtol=2e-6, atol=1e-7)


def test_rms_norm_scale_invariant_without_eps():
    rng = np.random.default_rng(12)
    x = rng.standard_normal((2, 576)).astype(np.float32)
    w = rng.standard_normal(576).astype(np.float32)
    a = ref.rms_norm_ref(x, w, 0.0)
    b = ref.rms_norm_ref(x * np.float32(64.0), w, 0.0)
    np.testing.assert_allclose(a, b, rtol=1e-6, atol=1e-7)
    # and a dropped square root or a missing mean would fail this
    assert abs(float(np.sqrt(np.mean((a / w) ** 2))) - 1.0) < 1e-4


def test_residual_rms_norm_adds_then_normalises():
    rng = np.random.default_rng(13)
    h = rng.standard_normal((1, 576)).astype(np.float16)
    r = rng.standard_normal((1, 576)).astype(np.float16)
    w = rng.standard_normal(576).astype(np.float16)
    h_new, y = ref.residual_rms_norm_ref(h, r, w, 1e-5, np.float16)
    assert np.array_equal(h_new, (h.astype(np.float32) + r.astype(np.float32)).astype(np.float16))
    want = ref.rms_norm_ref(h_new.astype(np.float32), w.astype(np.float32), 1e-5).astype(np.float16)
    assert np.array_equal(y, want)
    h2, y2 = ref.residual_rms_norm_ref(h, None, w, 1e-5, np.float16)
    assert np.array_equal(h2, h)
