// bf16 / fp32-activation decode kernels for int8 weights; see gemv_x.h.
#include "gemv_x.h"

namespace lq {
template int launch_tile_xl_x<8>(const void*, const void*, const void*, void*, int64_t,
                                  int64_t, int64_t, int64_t, int, int, hipStream_t);
template int launch_tile_rows_x<8, kXPairs, false>(const void*, const void*, const void*, void*,
                                                   int64_t, int64_t, int64_t, int64_t, int, int,
                                                   hipStream_t);
template int launch_skinny_x<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                                int64_t, int64_t, int, int, int, hipStream_t,
                                const FixedScratch*);
}  // namespace lq
