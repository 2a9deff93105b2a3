// Gate|up decode kernels with the SiLU * mul epilogue for bf16 activations
// and fp32 part-row pairs (int4); see gemv_x.h.
#include "gemv_x.h"

namespace lq {
template int launch_tile_rows_x<4, LQ_BF16, true>(const void*, const void*, const void*, void*,
                                                  int64_t, int64_t, int64_t, int64_t, int, int,
                                                  hipStream_t);
template int launch_tile_rows_x<4, kXPairs, true>(const void*, const void*, const void*, void*,
                                                  int64_t, int64_t, int64_t, int64_t, int, int,
                                                  hipStream_t);
}  // namespace lq
