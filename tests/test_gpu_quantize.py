"""GPU weight producers against the oracle's restatement of the reference
quantizers (examples/38_quantized_matmul.py:248-291,
examples/52_dequantize.py:110-126).  Bar: packed bytes, int8 values and
float32 scales bit-identical."""

import numpy as np
import pytest

from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

lq = pytest.importorskip("locomp_amd")


@pytest.fixture(params=["auto", "generic"])
def policy(request):
    lq.set_policy(0 if request.param == "auto" else 1)
    yield request.param
    lq.set_policy(0)


def _weights(N, K, seed, scale=1.0):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((N, K)) * scale).astype(np.float32)
    return w


def _eq(a, b):
    assert a.shape == b.shape and a.dtype == b.dtype, (a.shape, b.shape, a.dtype, b.dtype)
    assert np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


# (N, K, G): lane kernel for G = 8 .. 512 (power of two, K % 8 == 0), group
# kernel otherwise (G = 1024, 24, 10 with K % 8 != 0, per-channel G = K)
SHAPES = [(64, 256, 32), (100, 512, 64), (7, 96, 32), (33, 1024, 8), (5, 2048, 512),
          (3, 4096, 1024), (17, 96, 24), (9, 20, 10), (11, 384, 384), (256, 4096, 128)]


@pytest.mark.parametrize("N,K,G", SHAPES)
def test_quantize_int4_ex38(policy, N, K, G):
    w = _weights(N, K, seed=N + K + G)
    p, s = lq.quantize_int4(w, G)
    pr, sr = ref.quantize_int4(w, G)
    _eq(s, sr)
    _eq(p, pr)


@pytest.mark.parametrize("N,K,G", SHAPES)
def test_quantize_int4_ex52(policy, N, K, G):
    w = _weights(N, K, seed=2 * N + K + G, scale=0.02)
    p, s = lq.quantize_int4_ref(w, G)
    pr, sr = ref.quantize_int4_ref(w, G)
    _eq(s, sr)
    _eq(p, pr)


@pytest.mark.parametrize("N,K,G", SHAPES + [(4, 40, 5)])
def test_quantize_int8_ex38(policy, N, K, G):
    w = _weights(N, K, seed=3 * N + K + G, scale=3.0)
    q, s = lq.quantize_int8(w, G)
    qr, sr = ref.quantize_int8(w, G)
    _eq(s, sr)
    _eq(q, qr)


def test_quantize_special_values():
    """All-zero groups (scale 1.0 / 1e-10 floor), -0.0, exact halfway values
    (round half to even), the clip limits, tiny and huge magnitudes."""
    N, K, G = 6, 64, 32
    w = np.zeros((N, K), np.float32)
    w[1, :32] = -0.0
    w[2, :32] = np.arange(32, dtype=np.float32) * 0.5 - 7.5        # amax 8 -> s 8/7
    w[2, 32:] = np.array([7.0, -7.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5] * 4, np.float32)  # s = 1: ties
    w[3, :] = np.float32(1e-30) * np.arange(1, K + 1, dtype=np.float32)
    w[4, :] = np.float32(3e38) * np.sign(np.arange(K, dtype=np.float32) - 31.5)
    w[5, :32] = 127.0 * np.linspace(-1, 1, 32, dtype=np.float32)
    w[5, 32:] = np.array([127.0, -127.0, 63.5, -63.5, 0.5, 1.5, -0.5, -1.5] * 4, np.float32)
    for fn, rf in ((lq.quantize_int4, ref.quantize_int4), (lq.quantize_int4_ref, ref.quantize_int4_ref),
                   (lq.quantize_int8, ref.quantize_int8)):
        q, s = fn(w, G)
        qr, sr = rf(w, G)
        _eq(s, sr)
        _eq(q, qr)


@pytest.mark.parametrize("src", ["f16", "bf16"])
def test_quantize_16bit_inputs(src):
    """fp16 / bf16 device weights: the same result as quantizing their exact
    float32 values."""
    N, K, G = 48, 512, 32
    w = _weights(N, K, seed=11, scale=0.5)
    if src == "f16":
        w16 = w.astype(np.float16)
        dev = lq.tensor(w16)
        exact = w16.astype(np.float32)
    else:
        dev = lq.tensor(w, dtype=lq.bfloat16)
        exact = ref.bf16_bits_to_f32(ref.f32_to_bf16_bits(w)).reshape(N, K)
    for fn, rf in ((lq.quantize_int4, ref.quantize_int4), (lq.quantize_int8, ref.quantize_int8)):
        q, s = fn(dev, G)
        qr, sr = rf(exact, G)
        _eq(s, sr)
        _eq(q, qr)


def test_quantize_then_dequantize_round_trip():
    """Producer -> device dequant: |w - deq(q)| <= s / 2 per element (the
    reference's own round-trip bound), with the packed weights never leaving
    the device."""
    N, K, G = 128, 1024, 64
    w = _weights(N, K, seed=5)
    P, S = lq.quantize_int4(w, G, as_tensors=True)
    O = lq.empty(N * K, np.float32)
    lq.dequant_int4[(N,), (128,)](P, S, O, K, K // 2, K // G, G)
    d = O.numpy().reshape(N, K)
    s = np.repeat(S.numpy(), G, axis=1)
    assert np.all(np.abs(w - d) <= s * 0.5 + 1e-7 * np.abs(w))


@pytest.mark.parametrize("fn,rf,top", [("quantize_int4", "quantize_int4", 7.0),
                                      ("quantize_int4_ref", "quantize_int4_ref", 7.0),
                                      ("quantize_int8", "quantize_int8", 127.0)])
def test_quantize_rounding_ties(fn, rf, top):
    """Quotients w / s within a few ulps of half-integers, over scales from
    1e-20 to 1e20: the quantizer's division (one shared reciprocal per lane
    plus an fma correction) must round exactly as NumPy's float32 division
    before np.round, on every tie-adjacent value."""
    rng = np.random.default_rng(99)
    N, G = 8192, 8
    K = 8 * G
    amax = (10.0 ** rng.uniform(-20, 20, size=(N, K // G))).astype(np.float32)
    s = (amax / np.float32(top)).astype(np.float32)
    half = rng.integers(-int(top), int(top), size=(N, K)).astype(np.float32) + np.float32(0.5)
    ulps = rng.integers(-3, 4, size=(N, K)).astype(np.float32)
    sr = np.repeat(s, G, axis=1)
    w = (half * sr).astype(np.float32)
    w = (w + ulps * np.spacing(w)).astype(np.float32)
    w = np.clip(w, -np.repeat(amax, G, axis=1), np.repeat(amax, G, axis=1)).astype(np.float32)
    w[:, ::G] = np.repeat(amax, 1, axis=1) * np.where(rng.random((N, K // G)) < 0.5, 1, -1).astype(np.float32)
    q, sc = getattr(lq, fn)(w, G)
    qr, scr = getattr(ref, rf)(w, G)
    _eq(sc, scr)
    _eq(q, qr)
