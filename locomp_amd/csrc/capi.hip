// C ABI entry points: argument validation and kernel selection.
// Declarations and conventions: include/locomp_amd.h.
#include <algorithm>
#include <atomic>
#include <string>

#include "lq_common.h"

namespace lq {
int launch_dequant_int4(const void*, const void*, void*, int64_t, int64_t, int64_t, int, int, bool,
                        hipStream_t);
int launch_dequant_int8(const void*, const void*, void*, int64_t, int64_t, int64_t, int, int, bool,
                        hipStream_t);
template <int WBITS>
int launch_skinny(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                  int, int, hipStream_t);
template <int WBITS>
int launch_gemm_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                  int, int, int, hipStream_t, const FixedScratch*);
template <int WBITS, bool EPI>
int launch_gemm_pairs(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                      int64_t, int, int, hipStream_t);
template <int WBITS, bool EPI>
int launch_group_valu(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                      int64_t, int, int, int, hipStream_t, const FixedScratch*);
template <bool EPI>
int launch_rows_g16(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                    int, int, int, hipStream_t);
template <int WBITS, int XD, bool EPI>
int launch_tile_rows_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                       int64_t, int, int, hipStream_t);
int launch_gemm_silu_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                       int64_t, int, int, hipStream_t);
template <int WBITS>
int launch_skinny_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                    int64_t, int, int, int, hipStream_t, const FixedScratch*);
template <int WBITS>
int launch_generic(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                   int, int, int, hipStream_t);
template <int WBITS>
int launch_gemm(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t, int64_t,
                int, int, hipStream_t, const FixedScratch*);
template <int WBITS>
int launch_tile_xl_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                     int64_t, int, int, hipStream_t);
template <int WBITS>
int launch_gemm_split_only(const void*, const void*, const void*, void*, int64_t, int64_t,
                           int64_t, int64_t, int, int, hipStream_t, const FixedScratch*);
int launch_zero_fill(void*, int64_t, int, hipStream_t);
int launch_split_f32_rows(const float*, void*, int64_t, int64_t, hipStream_t);
int launch_rows_silu_x(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                       int64_t, int, int, int, hipStream_t);
int launch_rms_norm(void*, const void*, const void*, void*, int64_t, int64_t, float, int,
                    hipStream_t);
int launch_matvec_fused(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                        int64_t, int, int, int, const void*, float, const void*, bool, hipStream_t);
int launch_add_rows(const float*, const void*, void*, int64_t, int, hipStream_t);
int launch_quantize(int, const void*, void*, float*, int64_t, int64_t, int64_t, int, bool,
                    hipStream_t);
int launch_silu_fast(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                     int64_t, int, int, hipStream_t);
int launch_gemm_silu(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                     int64_t, int, int, hipStream_t);
void* stream_workspace(int, size_t, hipStream_t);
int release_workspaces(hipStream_t, bool);
int launch_silu_pairs(const float*, void*, int64_t, int64_t, int, hipStream_t);
int launch_generic_silu(const void*, const void*, const void*, void*, int64_t, int64_t, int64_t,
                        int64_t, int, int, int, hipStream_t);

static std::atomic<int> g_policy{LQ_POLICY_AUTO};

static inline bool dtype_ok(int d) { return d == LQ_F32 || d == LQ_F16 || d == LQ_BF16; }
static inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

// Largest problem the 32-bit index arithmetic of the fast kernels accepts.
constexpr int64_t kMax32 = (int64_t(1) << 31) - 1;

// Checks shared by every entry point; returns LQ_OK or an error code.
static int check_common(int64_t K, int64_t num_scales, int64_t G, int64_t N) {
  if (K < 0 || N < 0 || num_scales < 0) return LQ_ERR_SHAPE;
  if (G <= 0) return LQ_ERR_SHAPE;
  if (num_scales * G != K) return LQ_ERR_SHAPE;
  return LQ_OK;
}

static bool fast_allowed() { return g_policy.load(std::memory_order_relaxed) == LQ_POLICY_AUTO; }

}  // namespace lq

using namespace lq;

template <int WBITS>
static int matmul_dispatch(const void* X, const void* W, const void* S, void* O, int64_t K,
                           int64_t G, int64_t N, int64_t M, int xd, int sd, int od, hipStream_t st,
                           const FixedScratch* fixed = nullptr);

// fp32 activations at M > 4 (and gate|up beyond the row kernel): each row
// split into two bf16 parts with round to nearest (hi = RN(x), lo = RN(x -
// hi): |x - hi - lo| <= 2^-16 |x|), as 2 M bf16 rows in the stream's
// workspace slot 2 (row 2i + p = part p of row i), run on the bf16 kernels:
// the decode kernels for 2 M <= 64, else the MFMA GEMM (G % 32), whose
// stores add each row's two part products (EPI: then silu(gate) * up of the
// interleaved gate/up rows, O [M, N / 2]).  Each part times an integer
// weight is exact in fp32, so the result differs from an fp32 dot product by
// at most 2^-16 sum_k |x_k w_nk| beyond the summation order: no more than
// fp32 accumulation's own worst case (K 2^-24 sum_k |x_k w_nk|) for
// K >= 256.  Row blocks keep the part rows within the workspace cap.
// LQ_ERR_SHAPE (the caller falls back; it rewrites every row) when no fast
// kernel takes the shape or the workspace is missing (a capture on a stream
// that has none yet).
template <int WBITS, bool EPI>
static int f32_pair_rows(const void* X, const void* W, const void* S, void* O, int64_t K,
                         int64_t G, int64_t N, int64_t M, int sd, int od, hipStream_t st) {
  // below ~2^24 multiply-adds its two launches cost more than the generic
  // kernel (16 x 576 x 576 with three parts: 20 us against 11)
  if (M * N * K < (int64_t(1) << 24)) return LQ_ERR_SHAPE;
  constexpr int64_t kCap = int64_t(256) << 20;          // bytes per workspace slot
  const int64_t mb = std::min(M, std::max<int64_t>(1, kCap / (2 * K * 2)));
  void* parts = stream_workspace(2, size_t(2 * mb * K * 2), st);
  if (parts == nullptr) return LQ_ERR_SHAPE;
  const size_t orow = size_t(EPI ? N / 2 : N) * (od == LQ_F32 ? 4 : 2);
  // few long rows at N = 4096-class widths: the split-K GEMM beats the
  // activation-in-LDS kernel, as for bf16 activations
  const bool gemm_first = N > 3072 && N <= 4096 && K >= 10240;
  for (int64_t m0 = 0; m0 < M; m0 += mb) {
    const int64_t m = std::min(mb, M - m0);
    uint8_t* out = static_cast<uint8_t*>(O) + size_t(m0) * orow;
    int rc = launch_split_f32_rows(static_cast<const float*>(X) + m0 * K, parts, m, K, st);
    if (rc != LQ_OK) return rc;
    rc = LQ_ERR_SHAPE;
    if (2 * m <= 64 && !(2 * m > 16 && gemm_first))
      rc = launch_tile_rows_x<WBITS, kXPairs, EPI>(parts, W, S, out, 2 * m, N, K, G, sd, od, st);
    if (rc == LQ_ERR_SHAPE)
      rc = launch_gemm_pairs<WBITS, EPI>(parts, W, S, out, 2 * m, N, K, G, sd, od, st);
    if (rc != LQ_OK) return rc;
  }
  return LQ_OK;
}

// Kernel choice for the dequant-matmul entries (WBITS = 4 or 8).
// `fixed`: scratch lent by the caller for split-K partials (no allocation);
// nullptr = the per-stream workspace.
template <int WBITS>
static int matmul_dispatch(const void* X, const void* W, const void* S, void* O, int64_t K,
                           int64_t G, int64_t N, int64_t M, int xd, int sd, int od, hipStream_t st,
                           const FixedScratch* fixed) {
  if (!dtype_ok(xd) || !dtype_ok(sd) || !dtype_ok(od)) return LQ_ERR_DTYPE;
  if (M < 0) return LQ_ERR_SHAPE;
  if (M == 0 || N == 0) return LQ_OK;
  if (!O) return LQ_ERR_NULL;
  if (K == 0) return launch_zero_fill(O, M * N, od, st);
  if (!X || !W || !S) return LQ_ERR_NULL;
  const int64_t row_bytes = WBITS == 4 ? K / 2 : K;
  const bool small_enough = M * K <= kMax32 && N * row_bytes <= kMax32 && M * N <= kMax32 &&
                            N * (K / G) <= kMax32;
  // the fast kernels stage scale rows as dwords and load 16-byte pieces
  const bool fast_common = fast_allowed() && small_enough && aligned(X, 16) && aligned(W, 16) &&
                           aligned(S, 4) && K % 8 == 0;
  if (fast_common && (xd == LQ_BF16 || xd == LQ_F32) && M <= 16) {
    // bf16 activations (M <= 16) and fp32 (M <= 4) on bf16 MFMAs
    const int rc = launch_skinny_x<WBITS>(X, W, S, O, M, N, K, G, xd, sd, od, st, fixed);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  if (fast_common && xd == LQ_F32 && M > 4 && fixed == nullptr) {
    // fp32 beyond the decode kernels' 4 rows: two bf16 parts on the bf16 route
    const int rc = f32_pair_rows<WBITS, false>(X, W, S, O, K, G, N, M, sd, od, st);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  if (fast_common && xd == LQ_BF16 && M > 16 && M <= 64 &&
      !(N > 3072 && N <= 4096 && K >= 10240)) {
    // bf16 decode / verify sizes: the activation-in-LDS kernel (bf16 MFMAs);
    // few long rows (the split-GEMM shapes of the fp16 route) and other
    // shapes it does not take go to the GEMM below
    const int rc = launch_tile_xl_x<WBITS>(X, W, S, O, M, N, K, G, sd, od, st);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  if (fast_common && xd == LQ_BF16 && M > 16 && K % 64 == 0) {
    // bf16 prefill: the MFMA GEMM on exact integer weights (G % 32)
    const int rc = launch_gemm_x<WBITS>(X, W, S, O, M, N, K, G, xd, sd, od, st, fixed);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  const bool fast = fast_common && xd == LQ_F16;
  if (fast) {
    // Skinny (decode) kernel: 16-byte weight chunks per lane must lie in one
    // group and in one row.
    const int64_t lane_k = WBITS == 4 ? 32 : 16;
    // 16 < M <= 64 (int8: 32 < M) at N = 4096-class widths with long rows:
    // the GEMM with k split 8 ways fills the CUs, while the decode kernel
    // streams the whole activation block per workgroup (1 x 4096 x 11008
    // int4: 36.0 -> 28.6 us at M = 64, 27.1 -> 26.7 at M = 32; 4096 x 14336
    // M = 64: 45.3 -> 33.7; int8 M = 64 34.2 -> 29.3).  The split needs its
    // workspace; without one the decode kernel runs.
    if (M > (WBITS == 4 ? 16 : 32) && M <= 64 && N > 3072 && N <= 4096 && K >= 10240 &&
        K % 64 == 0 && G % 32 == 0) {
      const int rc = launch_gemm_split_only<WBITS>(X, W, S, O, M, N, K, G, sd, od, st, fixed);
      if (rc != LQ_ERR_SHAPE) return rc;
    }
    if (M <= 64 && K % lane_k == 0 && G % lane_k == 0)
      return launch_skinny<WBITS>(X, W, S, O, M, N, K, G, sd, od, st);
    // Prefill MFMA GEMM: each loader thread's 32 k (int4) / 16 k (int8)
    // inside one group.
    // int8 post-scales per group: whole 32-k halves per group (scale rows
    // beyond what LDS holds split K; a shape no split fits, or a capturing
    // stream without the workspace that needs, takes the generic kernel).
    const bool gemm_ok = G % 32 == 0;
    if (M > 64 && K % 64 == 0 && gemm_ok) {
      const int rc = launch_gemm<WBITS>(X, W, S, O, M, N, K, G, sd, od, st, fixed);
      if (rc != LQ_ERR_SHAPE) return rc;
    }
  }
  if (fast_common && WBITS == 4 && M <= 2 && G % 32 != 0 && G % 16 == 0) {
    // scale groups of 16-k multiples at M <= 2: the row kernel with a scale
    // per 16 k
    const int rc = launch_rows_g16<false>(X, W, S, O, M, N, K, G, xd, sd, od, st);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  if (fast_allowed() && small_enough) {
    // scale groups the MFMA kernels do not take (G % 32 != 0), unaligned
    // operands, and what else is left: fp32 FMAs on the VALU kernel
    const int rc = launch_group_valu<WBITS, false>(X, W, S, O, M, N, K, G, xd, sd, od, st, fixed);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  return launch_generic<WBITS>(X, W, S, O, M, N, K, G, xd, sd, od, st);
}

extern "C" {

int locomp_amd_abi_version(void) { return LOCOMP_AMD_ABI_VERSION; }

const char* locomp_amd_strerror(int code) {
  switch (code) {
    case LQ_OK: return "success";
    case LQ_ERR_SHAPE: return "inconsistent or unsupported sizes";
    case LQ_ERR_DTYPE: return "unknown dtype code";
    case LQ_ERR_NULL: return "null pointer for a non-empty problem";
    case LQ_ERR_POLICY: return "unknown kernel policy";
    case LQ_ERR_SCRATCH:
      return "problem needs scratch memory that is not available (the fixed buffer is too small, "
             "or a workspace cannot be allocated during stream capture)";
    case LQ_ERR_NAME: return "unknown kernel name";
    default: break;
  }
  if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
  return "unknown error";
}

int locomp_amd_set_policy(int policy) {
  if (policy != LQ_POLICY_AUTO && policy != LQ_POLICY_GENERIC) return LQ_ERR_POLICY;
  g_policy.store(policy);
  return LQ_OK;
}

int locomp_amd_get_policy(void) { return g_policy.load(); }

int locomp_amd_release_workspaces(void* stream, int all_streams) {
  return release_workspaces(static_cast<hipStream_t>(stream), all_streams != 0);
}

int locomp_amd_dequant_int4(const void* W, const void* SCALES, void* OUT, int64_t K, int64_t HALF_K,
                            int64_t NUM_SCALES, int64_t GROUP_SIZE, int64_t N, int scale_dtype,
                            int out_dtype, void* stream) {
  int rc = check_common(K, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  if (HALF_K * 2 != K) return LQ_ERR_SHAPE;
  if (!dtype_ok(scale_dtype) || !dtype_ok(out_dtype)) return LQ_ERR_DTYPE;
  if (N == 0 || K == 0) return LQ_OK;
  if (!W || !SCALES || !OUT) return LQ_ERR_NULL;
  const bool fast = fast_allowed() && HALF_K % 4 == 0 && GROUP_SIZE % 8 == 0 &&
                    N * (HALF_K / 4) <= kMax32 && aligned(W, 4) && aligned(OUT, 16) &&
                    N * NUM_SCALES <= kMax32;
  return launch_dequant_int4(W, SCALES, OUT, N, K, GROUP_SIZE, scale_dtype, out_dtype, fast,
                             static_cast<hipStream_t>(stream));
}

int locomp_amd_dequant_int8(const void* W, const void* SCALES, void* OUT, int64_t K,
                            int64_t NUM_SCALES, int64_t GROUP_SIZE, int64_t N, int scale_dtype,
                            int out_dtype, void* stream) {
  int rc = check_common(K, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  if (!dtype_ok(scale_dtype) || !dtype_ok(out_dtype)) return LQ_ERR_DTYPE;
  if (N == 0 || K == 0) return LQ_OK;
  if (!W || !SCALES || !OUT) return LQ_ERR_NULL;
  const bool fast = fast_allowed() && K % 8 == 0 && GROUP_SIZE % 8 == 0 &&
                    N * (K / 8) <= kMax32 && aligned(W, 8) && aligned(OUT, 16) &&
                    N * NUM_SCALES <= kMax32;
  return launch_dequant_int8(W, SCALES, OUT, N, K, GROUP_SIZE, scale_dtype, out_dtype, fast,
                             static_cast<hipStream_t>(stream));
}

int locomp_amd_dequant_matvec_int4(const void* X, const void* W, const void* scales, void* O,
                                   int64_t K_dim, int64_t HALF_K, int64_t NUM_SCALES,
                                   int64_t GROUP_SIZE, int64_t N, int64_t M, int x_dtype,
                                   int scale_dtype, int out_dtype, void* stream) {
  int rc = check_common(K_dim, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  if (HALF_K * 2 != K_dim) return LQ_ERR_SHAPE;
  return matmul_dispatch<4>(X, W, scales, O, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                            out_dtype, static_cast<hipStream_t>(stream));
}

int locomp_amd_dequant_matvec_int4_noalloc(const void* X, const void* W, const void* scales,
                                           void* O, int64_t K_dim, int64_t HALF_K,
                                           int64_t NUM_SCALES, int64_t GROUP_SIZE, int64_t N,
                                           int64_t M, int x_dtype, int scale_dtype, int out_dtype,
                                           void* stream) {
  int rc = check_common(K_dim, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  if (HALF_K * 2 != K_dim) return LQ_ERR_SHAPE;
  FixedScratch fixed{nullptr, kStaticScratchBytes};
  // the device's scratch address (looked up on the device's first call that
  // may launch; argument errors and empty problems return before)
  if (dtype_ok(x_dtype) && dtype_ok(scale_dtype) && dtype_ok(out_dtype) && M > 0 && N > 0 &&
      K_dim > 0 && X && W && scales && O) {
    rc = static_scratch(&fixed.p);
    if (rc != LQ_OK) return rc;
  }
  return matmul_dispatch<4>(X, W, scales, O, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                            out_dtype, static_cast<hipStream_t>(stream), &fixed);
}

int locomp_amd_dequant_matvec_int8(const void* X, const void* W, const void* scales, void* O,
                                   int64_t K_dim, int64_t NUM_SCALES, int64_t GROUP_SIZE,
                                   int64_t N, int64_t M, int x_dtype, int scale_dtype,
                                   int out_dtype, void* stream) {
  int rc = check_common(K_dim, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  return matmul_dispatch<8>(X, W, scales, O, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                            out_dtype, static_cast<hipStream_t>(stream));
}

int locomp_amd_dequant_matvec_int4_silu_mul(const void* X, const void* W, const void* scales,
                                            void* O, int64_t K_dim, int64_t HALF_K,
                                            int64_t NUM_SCALES, int64_t GROUP_SIZE, int64_t I,
                                            int64_t M, int x_dtype, int scale_dtype, int out_dtype,
                                            void* stream) {
  int rc = check_common(K_dim, NUM_SCALES, GROUP_SIZE, I);
  if (rc) return rc;
  if (HALF_K * 2 != K_dim) return LQ_ERR_SHAPE;
  if (!dtype_ok(x_dtype) || !dtype_ok(scale_dtype) || !dtype_ok(out_dtype)) return LQ_ERR_DTYPE;
  if (M < 0) return LQ_ERR_SHAPE;
  if (M == 0 || I == 0) return LQ_OK;
  if (!O) return LQ_ERR_NULL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K_dim == 0) return launch_zero_fill(O, M * I, out_dtype, st);   // silu(0) * 0
  if (!X || !W || !scales) return LQ_ERR_NULL;
  const int64_t N = 2 * I;
  const bool fast = fast_allowed() && aligned(X, 16) && aligned(W, 16) && aligned(scales, 4) &&
                    M * K_dim <= kMax32 && N * HALF_K <= kMax32 && N * NUM_SCALES <= kMax32;
  // the fp16 fused epilogues are instantiated for fp16 / fp32 scales and
  // outputs; bf16 / fp32 activations have their own (any of the three
  // scale / output dtypes); fp16 activations with bf16 scales or outputs,
  // and shapes no fused kernel takes, take the staged path below (fast
  // matvec, then the pairwise epilogue)
  const bool fused = x_dtype == LQ_F16 && scale_dtype != LQ_BF16 && out_dtype != LQ_BF16;
  if (fast) {
    rc = LQ_ERR_SHAPE;
    if (fused && M > 64 && K_dim % 64 == 0)   // prefill: the MFMA GEMM with the epilogue
      rc = launch_gemm_silu(X, W, scales, O, M, N, K_dim, GROUP_SIZE, scale_dtype, out_dtype, st);
    else if (fused)
      rc = launch_silu_fast(X, W, scales, O, M, N, K_dim, GROUP_SIZE, scale_dtype, out_dtype, st);
    if (rc != LQ_ERR_SHAPE) return rc;
    if (GROUP_SIZE % 32 != 0 && GROUP_SIZE % 16 == 0 && M <= 2 && K_dim % 8 == 0) {
      // scale groups of 16-k multiples: the row kernel with a scale per 16 k
      rc = launch_rows_g16<true>(X, W, scales, O, M, N, K_dim, GROUP_SIZE, x_dtype, scale_dtype,
                                 out_dtype, st);
      if (rc != LQ_ERR_SHAPE) return rc;
    }
    if (!fused && K_dim % 8 == 0) {
      // bf16 / fp32 activations or bf16 dtypes, M <= 2: the row kernel
      rc = launch_rows_silu_x(X, W, scales, O, M, N, K_dim, GROUP_SIZE, x_dtype, scale_dtype,
                              out_dtype, st);
      // bf16 activations: the decode kernels (M <= 64), else the MFMA GEMM
      if (rc == LQ_ERR_SHAPE && x_dtype == LQ_BF16 && M <= 64)
        rc = launch_tile_rows_x<4, LQ_BF16, true>(X, W, scales, O, M, N, K_dim, GROUP_SIZE,
                                                  scale_dtype, out_dtype, st);
      if (rc == LQ_ERR_SHAPE && x_dtype == LQ_BF16)
        rc = launch_gemm_silu_x(X, W, scales, O, M, N, K_dim, GROUP_SIZE, scale_dtype, out_dtype,
                                st);
      // fp32 activations: their two bf16 part rows on the same kernels
      if (rc == LQ_ERR_SHAPE && x_dtype == LQ_F32)
        rc = f32_pair_rows<4, true>(X, W, scales, O, K_dim, GROUP_SIZE, N, M, scale_dtype,
                                    out_dtype, st);
    }
    if (rc != LQ_ERR_SHAPE) return rc;
    // No fused kernel for this shape: the fast matvec into an fp32 staging
    // buffer (slot 1 of the stream's workspace), then the pairwise epilogue.
    void* P = stream_workspace(1, size_t(M) * size_t(N) * sizeof(float), st);
    if (P != nullptr) {
      rc = matmul_dispatch<4>(X, W, scales, P, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                              LQ_F32, st);
      if (rc != LQ_OK) return rc;
      return launch_silu_pairs(static_cast<const float*>(P), O, M, N, out_dtype, st);
    }
  }
  if (fast_allowed() && M * K_dim <= kMax32 && N * K_dim <= kMax32 && M * N <= kMax32) {
    rc = launch_group_valu<4, true>(X, W, scales, O, M, N, K_dim, GROUP_SIZE, x_dtype, scale_dtype,
                                    out_dtype, st, nullptr);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  return launch_generic_silu(X, W, scales, O, M, N, K_dim, GROUP_SIZE, x_dtype, scale_dtype,
                             out_dtype, st);
}

// The reference's generated-launcher convention (args = device pointers of
// the pointer parameters in signature order), with the integer parameters
// the reference bakes into each generated launcher passed as values.
int locomp_amd_launch(const char* name, int grid_x, int grid_y, int block_x, int block_y,
                      void** args, const int64_t* constexprs, int n_constexprs,
                      const int* dtypes, int64_t m, void* stream) {
  if (name == nullptr) return LQ_ERR_NAME;
  if (grid_x < 0 || grid_y != 1 || block_x <= 0 || block_y <= 0 ||
      int64_t(block_x) * block_y > 1024)
    return LQ_ERR_SHAPE;
  const std::string n(name);
  const int64_t N = grid_x;
  // every kernel here has pointer arguments and integer parameters
  auto need = [&](int nc) {
    return args != nullptr && dtypes != nullptr && constexprs != nullptr && n_constexprs == nc;
  };
  if (n == "dequant_int4") {        // (W, SCALES, OUT; K, HALF_K, NUM_SCALES, GROUP_SIZE)
    if (!need(4)) return LQ_ERR_SHAPE;
    return locomp_amd_dequant_int4(args[0], args[1], args[2], constexprs[0], constexprs[1],
                                   constexprs[2], constexprs[3], N, dtypes[1], dtypes[2], stream);
  }
  if (n == "dequant_int8") {        // (W, SCALES, OUT; K, NUM_SCALES, GROUP_SIZE)
    if (!need(3)) return LQ_ERR_SHAPE;
    return locomp_amd_dequant_int8(args[0], args[1], args[2], constexprs[0], constexprs[1],
                                   constexprs[2], N, dtypes[1], dtypes[2], stream);
  }
  if (n == "dequant_matvec_int4") { // (X, W, scales, O; K_dim, HALF_K, NUM_SCALES, GROUP_SIZE)
    if (!need(4)) return LQ_ERR_SHAPE;
    return locomp_amd_dequant_matvec_int4(args[0], args[1], args[2], args[3], constexprs[0],
                                          constexprs[1], constexprs[2], constexprs[3], N, m,
                                          dtypes[0], dtypes[2], dtypes[3], stream);
  }
  if (n == "dequant_matvec_int8" || n == "quant_matvec_int8") {   // (X, W, scales, O; K_dim, NUM_SCALES, GROUP_SIZE)
    if (!need(3)) return LQ_ERR_SHAPE;
    return locomp_amd_dequant_matvec_int8(args[0], args[1], args[2], args[3], constexprs[0],
                                          constexprs[1], constexprs[2], N, m, dtypes[0],
                                          dtypes[2], dtypes[3], stream);
  }
  return LQ_ERR_NAME;
}

// Quantizers.  mode: 0 = examples/38 quantize_int4, 1 = examples/52
// quantize_int4_ref, 2 = examples/38 quantize_int8.
static int quantize_common(int mode, const void* W, void* Q, float* S, int64_t N, int64_t K,
                           int64_t G, int in_dtype, void* stream) {
  if (!dtype_ok(in_dtype)) return LQ_ERR_DTYPE;
  if (N < 0 || K < 0 || G <= 0 || K % G != 0) return LQ_ERR_SHAPE;
  if (mode != 2 && G % 2 != 0) return LQ_ERR_SHAPE;   // int4 packs pairs inside a group
  if (N == 0 || K == 0) return LQ_OK;
  if (!W || !Q || !S) return LQ_ERR_NULL;
  if (N * K > kMax32 * 4) return LQ_ERR_SHAPE;
  const bool vec_ok = fast_allowed() && K % 8 == 0 && aligned(W, 16) &&
                      aligned(Q, mode == 2 ? 8 : 4);
  return launch_quantize(mode, W, Q, S, N, K, G, in_dtype, vec_ok,
                         static_cast<hipStream_t>(stream));
}

int locomp_amd_quantize_int4(const void* W, void* PACKED, float* SCALES, int64_t N, int64_t K,
                             int64_t GROUP_SIZE, int variant, int in_dtype, void* stream) {
  if (variant != LQ_QUANT_EX38 && variant != LQ_QUANT_EX52) return LQ_ERR_SHAPE;
  return quantize_common(variant == LQ_QUANT_EX38 ? 0 : 1, W, PACKED, SCALES, N, K, GROUP_SIZE,
                         in_dtype, stream);
}

int locomp_amd_quantize_int8(const void* W, void* Q, float* SCALES, int64_t N, int64_t K,
                             int64_t GROUP_SIZE, int in_dtype, void* stream) {
  return quantize_common(2, W, Q, SCALES, N, K, GROUP_SIZE, in_dtype, stream);
}

int locomp_amd_rms_norm(void* H, const void* R, const void* gamma, void* Y, int64_t M, int64_t K,
                        float eps, int dtype, void* stream) {
  if (!dtype_ok(dtype)) return LQ_ERR_DTYPE;
  if (M < 0 || K < 0 || M > kMax32 || K > kMax32) return LQ_ERR_SHAPE;
  if (M == 0 || K == 0) return LQ_OK;
  if (!H || !gamma || !Y) return LQ_ERR_NULL;
  return launch_rms_norm(H, R, gamma, Y, M, K, eps, dtype, static_cast<hipStream_t>(stream));
}

int locomp_amd_dequant_matvec_int4_fused(const void* X, const void* W, const void* scales, void* O,
                                         int64_t K_dim, int64_t HALF_K, int64_t NUM_SCALES,
                                         int64_t GROUP_SIZE, int64_t N, int64_t M, int x_dtype,
                                         int scale_dtype, int out_dtype, const void* norm_weight,
                                         float norm_eps, const void* residual, int silu_mul,
                                         void* stream) {
  int rc = check_common(K_dim, NUM_SCALES, GROUP_SIZE, N);
  if (rc) return rc;
  if (HALF_K * 2 != K_dim) return LQ_ERR_SHAPE;
  if (!dtype_ok(x_dtype) || !dtype_ok(scale_dtype) || !dtype_ok(out_dtype)) return LQ_ERR_DTYPE;
  if (M < 0 || (silu_mul && (residual || N % 2 != 0))) return LQ_ERR_SHAPE;
  const int64_t on = silu_mul ? N / 2 : N;   // output columns
  if (M == 0 || on == 0) return LQ_OK;
  if (!O) return LQ_ERR_NULL;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (!norm_weight && !residual) {
    if (silu_mul)
      return locomp_amd_dequant_matvec_int4_silu_mul(X, W, scales, O, K_dim, HALF_K, NUM_SCALES,
                                                     GROUP_SIZE, N / 2, M, x_dtype, scale_dtype,
                                                     out_dtype, stream);
    return matmul_dispatch<4>(X, W, scales, O, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                              out_dtype, st);
  }
  if (K_dim > 0 && (!X || !W || !scales)) return LQ_ERR_NULL;
  if (fast_allowed() && K_dim > 0 && aligned(X, 16) && aligned(W, 16) && aligned(scales, 4) &&
      (!norm_weight || aligned(norm_weight, 16))) {
    rc = launch_matvec_fused(X, W, scales, O, M, N, K_dim, GROUP_SIZE, x_dtype, scale_dtype,
                             out_dtype, norm_weight, norm_eps, residual, silu_mul != 0, st);
    if (rc != LQ_ERR_SHAPE) return rc;
  }
  // Staged: the normalized activations in workspace slot 4, the product in
  // fp32 in slot 3 when a residual follows, then the residual add.
  const void* Xn = X;
  if (norm_weight && K_dim > 0) {
    const size_t xs = x_dtype == LQ_F32 ? 4 : 2;
    void* Y = stream_workspace(4, size_t(M) * size_t(K_dim) * xs, st);
    if (Y == nullptr) return LQ_ERR_SCRATCH;
    rc = launch_rms_norm(const_cast<void*>(X), nullptr, norm_weight, Y, M, K_dim, norm_eps,
                         x_dtype, st);
    if (rc != LQ_OK) return rc;
    Xn = Y;
  }
  if (silu_mul)
    return locomp_amd_dequant_matvec_int4_silu_mul(Xn, W, scales, O, K_dim, HALF_K, NUM_SCALES,
                                                   GROUP_SIZE, N / 2, M, x_dtype, scale_dtype,
                                                   out_dtype, stream);
  if (!residual)
    return matmul_dispatch<4>(Xn, W, scales, O, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype,
                              out_dtype, st);
  void* P = stream_workspace(3, size_t(M) * size_t(N) * sizeof(float), st);
  if (P == nullptr) return LQ_ERR_SCRATCH;
  rc = matmul_dispatch<4>(Xn, W, scales, P, K_dim, GROUP_SIZE, N, M, x_dtype, scale_dtype, LQ_F32,
                          st);
  if (rc != LQ_OK) return rc;
  return launch_add_rows(static_cast<const float*>(P), residual, O, M * N, out_dtype, st);
}

}  // extern "C"
