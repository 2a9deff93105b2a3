"""GPU: the reference-side binding (locomp_amd.rocm_hook.try_launch) running
the kernels as locomp's _launch_rocm would hand them over: device tensors
with the reference's ROCmTensor attributes, and host ndarrays (whose outputs
the binding writes back).  fp32 activations / scales / outputs, the
reference's own dtypes (examples/38_quantized_matmul.py:30-40)."""

import numpy as np
import pytest

from locomp_amd import synth
from locomp_amd.rocm_hook import try_launch
from oracle import quant_ref as ref

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


class DevTensor:
    """A torch device tensor seen through ROCmTensor's attributes."""

    def __init__(self, a):
        self.t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
        self._hip_ptr, self.size, self.dtype = self.t.data_ptr(), a.size, a.dtype


def _close32(got, want):
    atol = 1e-5 * max(1.0, float(np.abs(want).max()))
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=atol)


@pytest.mark.parametrize("host", [False, True])
@pytest.mark.parametrize("wbits,N,K,G", [(4, 1024, 4096, 128), (8, 512, 512, 512), (8, 300, 2048, 64)])
def test_hook_matvec_fp32(host, wbits, N, K, G):
    X, W, S = synth.matvec_case(wbits, 1, N, K, G, 0.001, 0.01, x_dtype=np.float32,
                                s_dtype=np.float32, seed=N + K)
    X = X.reshape(K)
    O = np.zeros(N, np.float32)
    args = [X, W, S, O] if host else [DevTensor(X), DevTensor(W), DevTensor(S), DevTensor(O)]
    if wbits == 4:
        name, cx = "dequant_matvec_int4", {"K_dim": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    else:
        name, cx = "quant_matvec_int8", {"K_dim": K, "NUM_SCALES": K // G, "GROUP_SIZE": G}
    assert try_launch(name, (N,), (128,), args, cx)
    got = O if host else args[3].t.cpu().numpy()
    f = ref.fast_numpy_matvec_int4 if wbits == 4 else ref.fast_numpy_matvec_int8
    _close32(got, f(X.reshape(1, K), W, S, G).reshape(N))


def test_hook_dequant_int4_bit_exact_into_host_output():
    N, K, G = 128, 512, 32
    W, S = synth.dequant_case(4, N, K, G, 0.001, 0.01, s_dtype=np.float32, seed=4)
    OUT = np.zeros((N, K), np.float32)
    assert try_launch("dequant_int4", (N,), (128,), [W, DevTensor(S), OUT],
                      {"K": K, "HALF_K": K // 2, "NUM_SCALES": K // G, "GROUP_SIZE": G})
    want = ref.dequant_int4_ref(W, S, N, K, G)
    assert np.array_equal(OUT.view(np.uint32), want.astype(np.float32).view(np.uint32))
