// Decode-step fusions on the row kernel (int4, M = 1, G % 32, K <= 4096):
// rmsnorm of the activations in its prologue, the residual add in its
// store, with or without the gate|up SiLU * mul epilogue; and the residual
// add kernel of the fallback.  See gemv_rows.h (FUSE).
#include "gemv_impl.h"

namespace lq {

template <int NSEG, int RW, bool EPI, int XD, int FUSE, int OCC>
static int launch_fused_t(const void* X, const void* W, const void* S, void* O, int64_t N,
                          int64_t K, int64_t G, int sd, int od, const void* gamma, float eps,
                          const void* R, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_rows_kernel<1, NSEG, RW, kRT, kRT, EPI, OCC, XD, FUSE>), dim3(blocks),
                     dim3(256), 0, st, X, static_cast<const uint8_t*>(W), S, O, 1, int(N), int(K),
                     int(K / G), int(G), sd, od, gamma, eps, R);
  return check_launch();
}

// Segment counts and rows per wave as the plain row kernel takes them.
template <int XD, bool EPI, int FUSE>
static int launch_fused_x(const void* X, const void* W, const void* S, void* O, int64_t N,
                          int64_t K, int64_t G, int sd, int od, const void* gamma, float eps,
                          const void* R, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  constexpr int kSmallRW = EPI ? 2 : 1;   // (gate / up pairs stay in one wave)
  if (nseg <= 2 && N <= 3072) {
    if (nseg <= 1)
      return launch_fused_t<1, kSmallRW, EPI, XD, FUSE, 3>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);
    return launch_fused_t<2, kSmallRW, EPI, XD, FUSE, 3>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);
  }
  if (nseg <= 1)
    return launch_fused_t<1, 4, EPI, XD, FUSE, 3>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);
  return launch_fused_t<2, 4, EPI, XD, FUSE, 2>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);
}

// M = 1, K <= 4096, G % 32: one launch.  `gamma` (X's dtype): rmsnorm
// prologue; `R` (O's dtype, may be O): residual add; `epi`: SiLU * mul
// (not with R).  LQ_ERR_SHAPE where the row kernel does not apply.
int launch_matvec_fused(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                        int64_t K, int64_t G, int xd, int sd, int od, const void* gamma, float eps,
                        const void* R, bool epi, hipStream_t st) {
  if (M != 1 || K % 32 != 0 || G % 32 != 0 || K < 32 || K > 4096 || (epi && (R || N % 2 != 0)))
    return LQ_ERR_SHAPE;
  if (!gamma && !R) return LQ_ERR_SHAPE;
  const int fuse = (gamma ? kFuseNorm : 0) | (R ? kFuseRes : 0);
#define LQ_FX(XD_)                                                                                     \
  do {                                                                                                 \
    if (epi && fuse == kFuseNorm)                                                                      \
      return launch_fused_x<XD_, true, kFuseNorm>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);   \
    if (!epi && fuse == kFuseNorm)                                                                     \
      return launch_fused_x<XD_, false, kFuseNorm>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);  \
    if (!epi && fuse == kFuseRes)                                                                      \
      return launch_fused_x<XD_, false, kFuseRes>(X, W, S, O, N, K, G, sd, od, gamma, eps, R, st);   \
    if (!epi && fuse == (kFuseNorm | kFuseRes))                                                        \
      return launch_fused_x<XD_, false, kFuseNorm | kFuseRes>(X, W, S, O, N, K, G, sd, od, gamma, eps, \
                                                              R, st);                                  \
  } while (0)
  if (xd == LQ_F16) LQ_FX(LQ_F16);
  else if (xd == LQ_BF16) LQ_FX(LQ_BF16);
  else if (xd == LQ_F32) LQ_FX(LQ_F32);
#undef LQ_FX
  return LQ_ERR_SHAPE;
}

// O [M, N] (od) = P (fp32) + R (od); R may be O.
__global__ __launch_bounds__(256) void add_rows_kernel(const float* __restrict__ P, const void* R,
                                                       void* O, int64_t count, int od) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= count) return;
  store_out<kRT>(O, size_t(i), P[i] + load_f32_rt<kRT>(R, size_t(i), od), od);
}

int launch_add_rows(const float* P, const void* R, void* O, int64_t count, int od, hipStream_t st) {
  if (count == 0) return LQ_OK;
  hipLaunchKernelGGL(add_rows_kernel, dim3(unsigned((count + 255) / 256)), dim3(256), 0, st, P, R, O,
                     count, od);
  return check_launch();
}

}  // namespace lq
