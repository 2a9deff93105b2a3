"""GPU: the allocation-free dequant-matvec entry point
(locomp_amd_dequant_matvec_int4_noalloc) against the allocating one
(locomp_amd_dequant_matvec_int4), through the C ABI on the same inputs.

Both run the same kernels; the split-K prefill partials of the first live in
the library's fixed per-GPU scratch array (as do the bf16 part rows of fp32
activations at M <= 4), so the outputs must be bit-identical, including on a
second, smaller call right after the first (the array keeps the first call's
contents)."""

import ctypes

import numpy as np
import pytest

from locomp_amd import _lib, synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
vp = ctypes.c_void_p


def _run(fn, X, W, S, M, N, K, G, xd=None):
    stream = torch.cuda.current_stream()
    Xd, Wd, Sd = (torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in (X, W, S))
    Od = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    rc = fn(vp(Xd.data_ptr()), vp(Wd.data_ptr()), vp(Sd.data_ptr()), vp(Od.data_ptr()),
            K, K // 2, K // G, G, N, M, _lib.F16 if xd is None else xd, _lib.F16, _lib.F16,
            vp(stream.cuda_stream))
    torch.cuda.synchronize()
    return rc, Od.cpu().numpy()


# (M, N, K, G) pairs: a split-K prefill, then a smaller one; decode shapes need
# no scratch and must match too
CASES = [
    ((128, 4096, 4096, 128), (100, 2048, 4096, 128)),   # 8-way split, then 4-way
    ((512, 4096, 4096, 128), (200, 1024, 2048, 64)),
    ((1, 11008, 4096, 128), (4, 4096, 4096, 32)),
    ((64, 4096, 11008, 128), (24, 4096, 10240, 32)),   # decode M on the split-K GEMM, uneven runs
]


@pytest.mark.parametrize("first,second", CASES)
def test_noalloc_matches_allocating_entry(first, second):
    lib = _lib.load()
    for seed, (M, N, K, G) in enumerate((first, second)):
        print(f"noalloc case M={M} N={N} K={K} G={G}", flush=True)
        X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=seed)
        rc_a, want = _run(lib.locomp_amd_dequant_matvec_int4, X, W, S, M, N, K, G)
        rc_b, got = _run(lib.locomp_amd_dequant_matvec_int4_noalloc, X, W, S, M, N, K, G)
        assert rc_a == 0 and rc_b == 0, (rc_a, rc_b)
        assert not np.isnan(got).any()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_noalloc_fp32_activations_matches_allocating_entry():
    """fp32 activations at 2 <= M <= 4 are split into bf16 part rows first:
    in the fixed array here, in the stream's workspace for the allocating
    entry.  The second call has fewer rows, so the array still holds the first
    call's part rows past it; they must not be read."""
    lib = _lib.load()
    for seed, (M, N, K, G) in enumerate(((4, 11008, 4096, 128), (2, 3000, 2048, 64))):
        print(f"noalloc fp32 case M={M} N={N} K={K} G={G}", flush=True)
        X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=10 + seed)
        X = X.astype(np.float32)
        rc_a, want = _run(lib.locomp_amd_dequant_matvec_int4, X, W, S, M, N, K, G, _lib.F32)
        rc_b, got = _run(lib.locomp_amd_dequant_matvec_int4_noalloc, X, W, S, M, N, K, G, _lib.F32)
        assert rc_a == 0 and rc_b == 0, (rc_a, rc_b)
        assert not np.isnan(got).any()
        assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_noalloc_runs_unsplit_when_the_optional_split_does_not_fit():
    """512 x 14336 x 4096 int4 takes 256-row tiles with k split in two in the
    allocating entry (58.7 MB of partials); the split is only for speed, so
    with the fixed 32 MiB array the unsplit GEMM runs instead: different
    summation order, the same results to the matmul tolerance.  A second,
    smaller call follows."""
    from oracle import quant_ref as ref
    lib = _lib.load()
    for seed, (M, N, K, G) in enumerate(((512, 14336, 4096, 128), (512, 11008, 4096, 128))):
        print(f"noalloc unsplit case M={M} N={N} K={K} G={G}", flush=True)
        X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=20 + seed)
        rc, got = _run(lib.locomp_amd_dequant_matvec_int4_noalloc, X, W, S, M, N, K, G)
        assert rc == 0
        np.testing.assert_allclose(got.astype(np.float32), ref.fast_numpy_matvec_int4(X, W, S, G),
                                   rtol=1e-2, atol=1e-2)


def test_noalloc_rejects_required_splits_beyond_the_scratch():
    # bf16 activations post-scale their groups per split, which holds at most
    # 64 groups: K = 8192 with G = 32 (256 groups) needs 4 splits, and
    # 1024 x 4096 x 4 B x 4 = 64 MiB of partials exceed the fixed array
    lib = _lib.load()
    M, N, K, G = 1024, 4096, 8192, 32
    X, W, S = synth.matvec_case(4, M, N, K, G, 0.001, 0.01, seed=3)
    Xb = (X.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)   # bf16 bits (truncated)
    rc, _ = _run(lib.locomp_amd_dequant_matvec_int4_noalloc, Xb, W, S, M, N, K, G, _lib.BF16)
    assert rc == _lib.ERR_SCRATCH
    rc, _ = _run(lib.locomp_amd_dequant_matvec_int4, Xb, W, S, M, N, K, G, _lib.BF16)
    assert rc == 0
