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


@pytest.mark.parametrize("f32", [False, True])
def test_fused_chain_every_link(f32):
    """The same step with the norms and residual adds fused into the linears
    (4 launches per layer): every link against the oracle on the device's
    own inputs: rmsnorm -> matmul (the norm output rounded to the dtype, as
    the separate norm stores it), matmul + residual (rounded once to the
    dtype), at the bars above."""
    from locomp_amd.stack import DecodeStack, RMS_EPS
    st = DecodeStack(fuse_norm=True, f32=f32, keep_host=True, seed=7)
    dt = np.float32 if f32 else np.float16
    sp = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert len(st.links) == 4 * 30 + 1
    worst = 0.0
    for j, L in enumerate(st.links):
        x = L.X.cpu().numpy()[: L.K][None].astype(dt)
        r = L.res.cpu().numpy()[None].astype(np.float64) if L.res is not None else None
        st.run_link(j, sp)
        torch.cuda.synchronize()
        got = L.O.cpu().numpy()[None].astype(np.float64)
        W, S = st.host[j][:2]
        if L.gamma is not None:
            x = ref.rms_norm_ref(x.astype(np.float32), st.host[j][2].astype(np.float32), RMS_EPS).astype(dt)
        if L.epi:
            want, bound = _silu_mul_oracle(x, W, S, st.G)
            assert (np.abs(got - want) <= bound).all(), L.name
            continue
        want = ref.fast_numpy_matvec_int4(x, W, S, st.G).astype(np.float64)
        if r is not None:
            want = (want + r).astype(dt).astype(np.float64)
        if f32:
            atol = 1e-5 * max(1.0, float(np.abs(want).max()))
            np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol, err_msg=L.name)
        else:
            np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2, err_msg=L.name)
        worst = max(worst, float(np.abs(want).max()))
    assert st.links[-1].name == "final_norm+lm_head" and st.links[-1].N == 49152
    assert 0.1 < worst < 1e4, worst


@pytest.mark.parametrize("M,N,K,G,xd,norm,res,silu,alias", [
    (1, 960, 576, 32, "f16", True, False, False, False),     # one launch: norm prologue
    (1, 576, 1536, 32, "bf16", False, True, False, True),    # residual store, in place
    (1, 3072, 576, 32, "f32", True, False, True, False),     # norm + SiLU * mul
    (1, 576, 576, 32, "f16", True, True, False, False),      # norm and residual
    (1, 4100, 4096, 128, "f32", True, True, False, True),    # two segments, 4 rows per wave
    (4, 1024, 2048, 32, "f16", True, True, False, True),     # staged: M > 1
    (1, 1024, 6144, 64, "f32", True, False, False, False),   # staged: K > 4096
    (3, 2048, 1024, 128, "bf16", True, False, True, False),  # staged SiLU * mul
    (2, 700, 512, 16, "f16", False, True, False, True),      # staged: G = 16 (VALU kernel)
])
def test_fused_entry(M, N, K, G, xd, norm, res, silu, alias):
    """locomp_amd_dequant_matvec_int4_fused on its one-launch shapes and on
    the staged ones, every option, the residual in place or separate."""
    from locomp_amd import _lib, synth
    lib = _lib.load()
    vp = ctypes.c_void_p
    codes = {"f16": _lib.F16, "bf16": _lib.BF16, "f32": _lib.F32}
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[xd]
    rng = np.random.default_rng(M + N + K)
    X = rng.standard_normal((M, K)).astype(np.float32)
    W = synth.int4_weights(rng, N, K)
    S = synth.scales(rng, N, K // G, 0.001, 0.01).astype(np.float32)
    g = rng.uniform(0.5, 1.5, K).astype(np.float32)
    on = N // 2 if silu else N
    Rh = rng.standard_normal((M, on)).astype(np.float32)
    Xd = torch.from_numpy(X).cuda().to(tdt)
    gd = torch.from_numpy(g).cuda().to(tdt)
    Rd = torch.from_numpy(Rh).cuda().to(tdt)
    Od = Rd.clone() if alias else torch.zeros((M, on), dtype=tdt, device="cuda")
    Rp = Od if alias else Rd
    Wd, Sd = torch.from_numpy(W).cuda(), torch.from_numpy(S).cuda()
    rc = lib.locomp_amd_dequant_matvec_int4_fused(
        vp(Xd.data_ptr()), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(Od.data_ptr()), K, K // 2, K // G, G,
        N, M, codes[xd], _lib.F32, codes[xd], vp(gd.data_ptr()) if norm else None, 1e-5,
        vp(Rp.data_ptr()) if res else None, 1 if silu else 0,
        vp(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, rc
    torch.cuda.synchronize()
    got = Od.float().cpu().numpy().astype(np.float64)
    x = Xd.float().cpu().numpy()
    r = Rd.float().cpu().numpy().astype(np.float64)
    if norm:
        y = ref.rms_norm_ref(x, gd.float().cpu().numpy(), 1e-5)
        x = torch.from_numpy(y).to(tdt).float().numpy()
    if silu:
        want, bound = _silu_mul_oracle(x, W, S, G)
        if xd == "bf16":
            bound = bound + 2.0 ** -8 * np.abs(want)
        assert (np.abs(got - want) <= bound).all()
        return
    want = ref.fast_numpy_matvec_int4(x, W, S, G).astype(np.float64)
    if res:
        want = want + r
    if xd == "f32":
        np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5 * max(1.0, float(np.abs(want).max())))
    else:
        np.testing.assert_allclose(got, want, rtol=1e-2, atol=1e-2 * max(1.0, float(np.abs(want).max())))
