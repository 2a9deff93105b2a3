// Decode (skinny) dequant-matmul kernels for int8 weights; see gemv_impl.h.
#include "gemv_impl.h"

namespace lq {
template int launch_skinny<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, hipStream_t);
}  // namespace lq
