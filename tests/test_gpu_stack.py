"""GPU: the SmolLM2-shaped decode step exactly as bench.py times it
(locomp_amd.stack.DecodeStack, chained: per layer residual add + RMSNorm ->
q|k|v -> o -> residual add + RMSNorm -> gate|up with SiLU * mul -> down, then
the final norm and the 49152 x 576 LM head), run link by link.  Every link is
checked against the oracle applied to the device's own input for that link
(the previous link's output as read back), so an error anywhere in the chain
shows at the link that makes it:

* residual add: bit-exact (one rounding of the fp32 sum to the dtype);
* RMSNorm output: within one rounding of the dtype (rsqrt differs from the
  oracle's 1 / sqrt by a few fp32 ulps);
* linears: the matmul bar (rtol / atol 1e-2 for fp16, rtol 1e-4 + atol
  1e-5 max|Y| for fp32); SiLU * mul: the bound that bar implies
  (examples/54_smollm2_inference.py:113-120, 545-549).
"""

import ctypes

import numpy as np
import pytest

from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _silu_mul_oracle(x, W, S, G):
    g = np.asarray(ref.fast_numpy_matvec_int4(x, W[0::2], S[0::2], G), np.float64)
    u = np.asarray(ref.fast_numpy_matvec_int4(x, W[1::2], S[1::2], G), np.float64)
    silu = g / (1.0 + np.exp(-g))
    want = silu * u
    bound = 1e-2 * (np.abs(silu) + 1.1 * np.abs(u) + 1.0) + 1e-2 * np.abs(want)
    return want, bound


@pytest.mark.parametrize("f32", [False, True])
def test_chained_decode_step_every_link(f32):
    from locomp_amd.stack import DecodeStack, RMS_EPS
    st = DecodeStack(chain=True, f32=f32, keep_host=True, seed=5)
    dt = np.float32 if f32 else np.float16
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    worst = 0.0
    for j, L in enumerate(st.links):
        if L.kind == "norm":
            h_in = L.H.cpu().numpy().copy()
            r = L.R.cpu().numpy()[: h_in.size] if L.R is not None else None
            st.run_link(j, sp)
            torch.cuda.synchronize()
            want_h, want_y = ref.residual_rms_norm_ref(h_in[None], None if r is None else r[None],
                                                       st.host[j], RMS_EPS, dt)
            assert np.array_equal(L.H.cpu().numpy()[None], want_h), L.name
            y = L.Y.cpu().numpy()[None].astype(np.float64)
            tol = 2e-6 if f32 else 2.0 ** -10
            assert np.all(np.abs(y - want_y) <= tol * np.abs(want_y) + 1e-6), L.name
            continue
        x = L.X.cpu().numpy()[: L.K][None].astype(dt)
        st.run_link(j, sp)
        torch.cuda.synchronize()
        got = L.O.cpu().numpy()[None].astype(np.float64)
        W, S = st.host[j]
        if L.epi:
            want, bound = _silu_mul_oracle(x, W, S, st.G)
            assert (np.abs(got - want) <= bound).all(), L.name
        else:
            want = ref.fast_numpy_matvec_int4(x, W, S, st.G).astype(np.float64)
            if f32:
                atol = 1e-5 * max(1.0, float(np.abs(want).max()))
                np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol, err_msg=L.name)
            else:
                np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2, err_msg=L.name)
        worst = max(worst, float(np.abs(want).max()))
    assert st.links[-1].name == "lm_head" and st.links[-1].N == 49152
    # the chain stays numerically alive: the norms keep every linear's output O(1)
    assert 0.1 < worst < 1e3, worst


def test_unchained_step_ends_with_the_lm_head():
    from locomp_amd.stack import DecodeStack
    st = DecodeStack(fused=True, silu=True, keep_host=True, seed=6)
    assert [L.name for L in st.links[-2:]] == ["29.down", "lm_head"]
    j = len(st.links) - 1
    L = st.links[j]
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st.run_link(j, sp)
    torch.cuda.synchronize()
    W, S = st.host[j]
    x = L.X.cpu().numpy().reshape(1, -1)[:, : L.K]
    np.testing.assert_allclose(L.O.cpu().numpy()[None].astype(np.float32),
                               ref.fast_numpy_matvec_int4(x, W, S, 32), rtol=1e-2, atol=1e-2)
