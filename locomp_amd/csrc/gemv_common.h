// Shared constants and helpers of the decode GEMV kernels (gemv_*.h).
#pragma once
#include <type_traits>

#include "lq_common.h"

namespace lq {

constexpr int kSkThreads = 256;
constexpr int kSkWaves = 4;
constexpr int kSkBatch = 4;  // k-steps whose weight loads are issued together

template <int WBITS> struct SkinnyGeom;
template <> struct SkinnyGeom<4> { static constexpr int kLane = 32; static constexpr int kStep = 128; };
template <> struct SkinnyGeom<8> { static constexpr int kLane = 16; static constexpr int kStep = 64; };

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ h8 make_h8(half2_t a, half2_t b, half2_t c, half2_t d) {
  h8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

// Row of a 16-byte X chunk: c / kc via an fp32 reciprocal (exact for the
// chunk counts used here: c < 2^20, kc <= 2^14).
__device__ __forceinline__ int chunk_row(int c, int kc, float inv_kc) {
  int m = int((float(c) + 0.5f) * inv_kc);
  return m;
}

}  // namespace lq
