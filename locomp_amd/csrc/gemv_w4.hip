// Decode (skinny) dequant-matmul kernels for int4 weights; see gemv_impl.h.
#include "gemv_impl.h"

namespace lq {
template int launch_skinny<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, hipStream_t);
int launch_silu_fast(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                     int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  return launch_rows_silu<>(X, W, S, O, M, N, K, G, sd, od, st);
}
}  // namespace lq
