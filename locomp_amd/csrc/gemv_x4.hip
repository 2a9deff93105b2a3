// bf16 / fp32-activation decode kernels for int4 weights; see gemv_x.h.
#include "gemv_x.h"

namespace lq {

// fp32 rows X [M, K] (K % 8 == 0) -> their round-to-nearest bf16 parts
// P [2 M, K], row 2 m + p = part p of row m.
int launch_split_f32_rows(const float* X, void* P, int64_t M, int64_t K, hipStream_t st) {
  const int64_t threads = M * (K / 8);
  hipLaunchKernelGGL(split_f32_parts_kernel<2>, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, st,
                     X, static_cast<uint16_t*>(P), int(M), int(K), 2, 1);
  return check_launch();
}

template int launch_tile_xl_x<4>(const void*, const void*, const void*, void*, int64_t,
                                  int64_t, int64_t, int64_t, int, int, hipStream_t);
template int launch_tile_rows_x<4, kXPairs, false>(const void*, const void*, const void*, void*,
                                                   int64_t, int64_t, int64_t, int64_t, int, int,
                                                   hipStream_t);
// Gate / up rows interleaved with the SiLU * mul epilogue on the row kernel
// for what the fp16 fused kernels do not take (bf16 / fp32 activations,
// bf16 scales or outputs), M <= 2 (fp32: M = 1, K <= 4096).
int launch_rows_silu_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                       int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st) {
  return launch_rows_x<true>(X, W, S, O, M, N, K, G, xd, sd, od, st);
}

template int launch_skinny_x<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                                int64_t, int64_t, int, int, int, hipStream_t,
                                const FixedScratch*);
}  // namespace lq
