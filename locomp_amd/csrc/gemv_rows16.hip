// Scale groups of 16-k multiples that are not 32-k multiples (G = 16, 48,
// ...) on the row-contiguous kernel (gemv_rows.h, G16): int4, M <= 2 (fp32
// activations M = 1, K <= 4096), every activation / scale / output dtype,
// optionally with the gate|up SiLU * mul epilogue.
#include "gemv_impl.h"

namespace lq {

template <int M_, int NSEG, int RW, bool EPI, int OCC, int XD>
static int launch_rows16_t(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                           int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_rows_kernel<M_, NSEG, RW, kRT, kRT, EPI, OCC, XD, 0, true>), dim3(blocks),
                     dim3(256), 0, st, X, static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),
                     int(K / G), int(G), sd, od, nullptr, 0.f, nullptr);
  return check_launch();
}

// Segment counts and rows per wave as the G % 32 row kernel takes them, with
// one row per wave from 5 segments (the epilogue's gate / up pairs keep two)
// since the second scale per lane k-range costs registers.
template <int M_, int XD, bool EPI>
static int launch_rows16_m(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                           int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  constexpr int kSmallRW = EPI ? 2 : 1;   // (gate / up pairs stay in one wave)
  constexpr int kLongRW = EPI ? 2 : 1;
  if (nseg <= 2 && N <= 3072) {
    if (nseg <= 1) return launch_rows16_t<M_, 1, kSmallRW, EPI, 3, XD>(X, W, S, O, M, N, K, G, sd, od, st);
    return launch_rows16_t<M_, 2, kSmallRW, EPI, 3, XD>(X, W, S, O, M, N, K, G, sd, od, st);
  }
  if (nseg <= 1) return launch_rows16_t<M_, 1, 4, EPI, 3, XD>(X, W, S, O, M, N, K, G, sd, od, st);
  if (nseg <= 2)
    return launch_rows16_t<M_, 2, 4, EPI, (M_ == 2 || XD == LQ_F32) ? 2 : 3, XD>(X, W, S, O, M, N, K, G, sd, od, st);
  if constexpr (M_ == 1 && XD != LQ_F32) {
    if (nseg <= 4) return launch_rows16_t<M_, 4, 2, EPI, 3, XD>(X, W, S, O, M, N, K, G, sd, od, st);
    if (nseg <= 6) return launch_rows16_t<M_, 6, kLongRW, EPI, 2, XD>(X, W, S, O, M, N, K, G, sd, od, st);
    // (8 segments with the epilogue's 2 rows per wave spill: not taken)
    if constexpr (!EPI) return launch_rows16_t<M_, 8, kLongRW, EPI, 2, XD>(X, W, S, O, M, N, K, G, sd, od, st);
  }
  return LQ_ERR_SHAPE;
}

// LQ_ERR_SHAPE where it does not apply: G % 16 != 0, M > 2 (fp32: M > 1 or
// K > 4096), K % 32 != 0, K beyond 16384 (M = 2: 4096; EPI: 12288), odd N
// with EPI.
template <bool EPI>
int launch_rows_g16(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N, int64_t K,
                    int64_t G, int xd, int sd, int od, hipStream_t st) {
  if (G % 16 != 0 || K % 32 != 0 || K < 32 || M < 1 || M > (xd == LQ_F32 ? 1 : 2) ||
      K > (M == 1 && xd != LQ_F32 ? 16384 : 4096) || (EPI && N % 2 != 0))
    return LQ_ERR_SHAPE;
#define LQ_R16(XD_)                                                                                \
  do {                                                                                             \
    if (M == 1) return launch_rows16_m<1, XD_, EPI>(X, W, S, O, M, N, K, G, sd, od, st);          \
    if constexpr (XD_ != LQ_F32) return launch_rows16_m<2, XD_, EPI>(X, W, S, O, M, N, K, G, sd, od, st); \
  } while (0)
  if (xd == LQ_F16) LQ_R16(LQ_F16);
  else if (xd == LQ_BF16) LQ_R16(LQ_BF16);
  else if (xd == LQ_F32) LQ_R16(LQ_F32);
#undef LQ_R16
  return LQ_ERR_SHAPE;
}

template int launch_rows_g16<false>(const void*, const void*, const void*, void*, int64_t, int64_t,
                                    int64_t, int64_t, int, int, int, hipStream_t);
template int launch_rows_g16<true>(const void*, const void*, const void*, void*, int64_t, int64_t,
                                   int64_t, int64_t, int, int, int, hipStream_t);

}  // namespace lq
