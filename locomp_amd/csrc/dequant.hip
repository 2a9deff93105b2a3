// Standalone dequantize kernels (gfx950): packed int4 / int8 -> fp32/fp16/bf16.
//
// Semantics follow locomp examples/52_dequantize.py:27-53 (int4) and :60-74
// (int8): OUT[r, k] = float32(q - 8) * float32(S[r, k / G]) (int4) or
// float32(q) * float32(S[r, k / G]) (int8), rounded once to the output dtype.
//
// The work is a flat, HBM-bound elementwise map: packed byte b of the
// row-major [N, K/2] weight feeds OUT elements 2b and 2b+1 of the row-major
// [N, K] output.  The fast kernels give each lane one dword (8 int4 / 4 int8
// weights) per step; consecutive lanes take consecutive dwords, so each wave
// instruction reads 256 contiguous bytes and writes 4 KB (fp16) contiguous.
#include "lq_common.h"

namespace lq {

constexpr int kDeqThreads = 256;
constexpr int kDeqUnroll = 4;

// ------------------------------------------------------------------ int4 --

template <int SD, int OD>
__global__ __launch_bounds__(kDeqThreads) void dequant_int4_dword_kernel(
    const uint32_t* __restrict__ W, const void* __restrict__ S, void* __restrict__ OUT,
    uint32_t total_dwords, uint32_t dwords_per_row, uint32_t num_scales, uint32_t group) {
  const uint32_t base = blockIdx.x * (kDeqThreads * kDeqUnroll) + threadIdx.x;
  uint32_t w[kDeqUnroll];
  uint32_t d[kDeqUnroll];
#pragma unroll
  for (int j = 0; j < kDeqUnroll; ++j) {
    d[j] = base + j * kDeqThreads;
    w[j] = d[j] < total_dwords ? __builtin_nontemporal_load(W + d[j]) : 0u;
  }
#pragma unroll
  for (int j = 0; j < kDeqUnroll; ++j) {
    if (d[j] >= total_dwords) continue;
    const uint32_t row = d[j] / dwords_per_row;
    const uint32_t k0 = (d[j] - row * dwords_per_row) * 8u;
    const size_t sidx = size_t(row) * num_scales + k0 / group;
    const size_t o = size_t(d[j]) * 8u;
    if constexpr (SD == LQ_F16 && OD == LQ_F16) {
      // fp16 path: exact (q - 8) in fp16, then one correctly rounded fp16
      // multiply == RNE of the exact fp32 product.
      const half_t s = static_cast<const half_t*>(S)[sidx];
      const half2_t s2 = {s, s};
      half2_t h[4];
      int4x8_to_h2(w[j], h);
      u32x4_t v;
      v.x = as_u32(h[0] * s2);
      v.y = as_u32(h[1] * s2);
      v.z = as_u32(h[2] * s2);
      v.w = as_u32(h[3] * s2);
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<half_t*>(OUT) + o));
    } else {
      const float s = load_f32<SD>(S, sidx);
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int q = int((w[j] >> (4 * e)) & 0xFu);
        f[e] = round_f32(float(q - 8) * s);
      }
      if constexpr (OD == LQ_F32) {
        float4_t a = {f[0], f[1], f[2], f[3]};
        float4_t b = {f[4], f[5], f[6], f[7]};
        float4_t* p = reinterpret_cast<float4_t*>(static_cast<float*>(OUT) + o);
        __builtin_nontemporal_store(a, p);
        __builtin_nontemporal_store(b, p + 1);
      } else {
        u32x4_t v;
        uint32_t u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (OD == LQ_F16) {
            const half2_t hh = {half_t(f[2 * e]), half_t(f[2 * e + 1])};
            u[e] = as_u32(hh);
          } else {
            u[e] = uint32_t(f32_to_bf16(f[2 * e])) | (uint32_t(f32_to_bf16(f[2 * e + 1])) << 16);
          }
        }
        v.x = u[0]; v.y = u[1]; v.z = u[2]; v.w = u[3];
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(OUT) + o));
      }
    }
  }
}

// Any shape / group size: one lane per packed byte, 64-bit indexing.
template <int SD, int OD>
__global__ __launch_bounds__(kDeqThreads) void dequant_int4_byte_kernel(
    const uint8_t* __restrict__ W, const void* __restrict__ S, void* __restrict__ OUT,
    int64_t total_bytes, int64_t half_k, int64_t num_scales, int64_t group) {
  const int64_t stride = int64_t(gridDim.x) * kDeqThreads;
  for (int64_t b = int64_t(blockIdx.x) * kDeqThreads + threadIdx.x; b < total_bytes; b += stride) {
    const int64_t row = b / half_k;
    const int64_t j = b - row * half_k;
    const uint32_t packed = W[b];
    const int64_t klo = 2 * j, khi = 2 * j + 1;
    const float slo = load_f32<SD>(S, size_t(row * num_scales + klo / group));
    const float shi = load_f32<SD>(S, size_t(row * num_scales + khi / group));
    store_f32<OD>(OUT, size_t(2 * b), round_f32(float(int(packed & 0xFu) - 8) * slo));
    store_f32<OD>(OUT, size_t(2 * b + 1), round_f32(float(int(packed >> 4) - 8) * shi));
  }
}

// ------------------------------------------------------------------ int8 --

template <int SD, int OD>
__global__ __launch_bounds__(kDeqThreads) void dequant_int8_qword_kernel(
    const u32x2_t* __restrict__ W, const void* __restrict__ S, void* __restrict__ OUT,
    uint32_t total_qwords, uint32_t qwords_per_row, uint32_t num_scales, uint32_t group) {
  const uint32_t base = blockIdx.x * (kDeqThreads * kDeqUnroll) + threadIdx.x;
  u32x2_t w[kDeqUnroll];
  uint32_t d[kDeqUnroll];
#pragma unroll
  for (int j = 0; j < kDeqUnroll; ++j) {
    d[j] = base + j * kDeqThreads;
    w[j] = d[j] < total_qwords ? __builtin_nontemporal_load(W + d[j]) : u32x2_t{0u, 0u};
  }
#pragma unroll
  for (int j = 0; j < kDeqUnroll; ++j) {
    if (d[j] >= total_qwords) continue;
    const uint32_t row = d[j] / qwords_per_row;
    const uint32_t k0 = (d[j] - row * qwords_per_row) * 8u;
    const size_t sidx = size_t(row) * num_scales + k0 / group;
    const size_t o = size_t(d[j]) * 8u;
    if constexpr (SD == LQ_F16 && OD == LQ_F16) {
      const half_t s = static_cast<const half_t*>(S)[sidx];
      const half2_t s2 = {s, s};
      half2_t h[4];
      int8x4_to_h2(w[j].x, h);
      int8x4_to_h2(w[j].y, h + 2);
      u32x4_t v;
      v.x = as_u32(h[0] * s2);
      v.y = as_u32(h[1] * s2);
      v.z = as_u32(h[2] * s2);
      v.w = as_u32(h[3] * s2);
      __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<half_t*>(OUT) + o));
    } else {
      const float s = load_f32<SD>(S, sidx);
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t word = e < 4 ? w[j].x : w[j].y;
        const int q = int(int8_t((word >> (8 * (e & 3))) & 0xFFu));
        f[e] = round_f32(float(q) * s);
      }
      if constexpr (OD == LQ_F32) {
        float4_t a = {f[0], f[1], f[2], f[3]};
        float4_t b = {f[4], f[5], f[6], f[7]};
        float4_t* p = reinterpret_cast<float4_t*>(static_cast<float*>(OUT) + o);
        __builtin_nontemporal_store(a, p);
        __builtin_nontemporal_store(b, p + 1);
      } else {
        u32x4_t v;
        uint32_t u[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (OD == LQ_F16) {
            const half2_t hh = {half_t(f[2 * e]), half_t(f[2 * e + 1])};
            u[e] = as_u32(hh);
          } else {
            u[e] = uint32_t(f32_to_bf16(f[2 * e])) | (uint32_t(f32_to_bf16(f[2 * e + 1])) << 16);
          }
        }
        v.x = u[0]; v.y = u[1]; v.z = u[2]; v.w = u[3];
        __builtin_nontemporal_store(v, reinterpret_cast<u32x4_t*>(static_cast<uint16_t*>(OUT) + o));
      }
    }
  }
}

template <int SD, int OD>
__global__ __launch_bounds__(kDeqThreads) void dequant_int8_elem_kernel(
    const int8_t* __restrict__ W, const void* __restrict__ S, void* __restrict__ OUT,
    int64_t total, int64_t k_dim, int64_t num_scales, int64_t group) {
  const int64_t stride = int64_t(gridDim.x) * kDeqThreads;
  for (int64_t i = int64_t(blockIdx.x) * kDeqThreads + threadIdx.x; i < total; i += stride) {
    const int64_t row = i / k_dim;
    const int64_t k = i - row * k_dim;
    const float s = load_f32<SD>(S, size_t(row * num_scales + k / group));
    store_f32<OD>(OUT, size_t(i), round_f32(float(int(W[i])) * s));
  }
}

// ------------------------------------------------------------ launchers --

static inline unsigned grid_stride_blocks(int64_t total) {
  int64_t b = (total + kDeqThreads - 1) / kDeqThreads;
  if (b > 65536) b = 65536;
  return unsigned(b < 1 ? 1 : b);
}

template <int SD, int OD>
static int launch_dequant_int4_t(const void* W, const void* S, void* OUT, int64_t N, int64_t K,
                                 int64_t G, bool fast, hipStream_t st) {
  const int64_t half_k = K / 2;
  const int64_t num_scales = K / G;
  if (fast) {
    const uint32_t dpr = uint32_t(half_k / 4);
    const uint32_t total = uint32_t(N * (half_k / 4));
    const unsigned blocks = (total + kDeqThreads * kDeqUnroll - 1) / (kDeqThreads * kDeqUnroll);
    hipLaunchKernelGGL((dequant_int4_dword_kernel<SD, OD>), dim3(blocks), dim3(kDeqThreads), 0, st,
                       static_cast<const uint32_t*>(W), S, OUT, total, dpr, uint32_t(num_scales),
                       uint32_t(G));
  } else {
    const int64_t total = N * half_k;
    hipLaunchKernelGGL((dequant_int4_byte_kernel<SD, OD>), dim3(grid_stride_blocks(total)),
                       dim3(kDeqThreads), 0, st, static_cast<const uint8_t*>(W), S, OUT, total,
                       half_k, num_scales, G);
  }
  return check_launch();
}

template <int SD, int OD>
static int launch_dequant_int8_t(const void* W, const void* S, void* OUT, int64_t N, int64_t K,
                                 int64_t G, bool fast, hipStream_t st) {
  const int64_t num_scales = K / G;
  if (fast) {
    const uint32_t qpr = uint32_t(K / 8);
    const uint32_t total = uint32_t(N * (K / 8));
    const unsigned blocks = (total + kDeqThreads * kDeqUnroll - 1) / (kDeqThreads * kDeqUnroll);
    hipLaunchKernelGGL((dequant_int8_qword_kernel<SD, OD>), dim3(blocks), dim3(kDeqThreads), 0, st,
                       static_cast<const u32x2_t*>(W), S, OUT, total, qpr, uint32_t(num_scales),
                       uint32_t(G));
  } else {
    const int64_t total = N * K;
    hipLaunchKernelGGL((dequant_int8_elem_kernel<SD, OD>), dim3(grid_stride_blocks(total)),
                       dim3(kDeqThreads), 0, st, static_cast<const int8_t*>(W), S, OUT, total, K,
                       num_scales, G);
  }
  return check_launch();
}

#define LQ_DISPATCH_SD_OD(FN, SD, OD, ...)                                  \
  do {                                                                      \
    if ((SD) == LQ_F32 && (OD) == LQ_F32) return FN<LQ_F32, LQ_F32>(__VA_ARGS__);   \
    if ((SD) == LQ_F32 && (OD) == LQ_F16) return FN<LQ_F32, LQ_F16>(__VA_ARGS__);   \
    if ((SD) == LQ_F32 && (OD) == LQ_BF16) return FN<LQ_F32, LQ_BF16>(__VA_ARGS__); \
    if ((SD) == LQ_F16 && (OD) == LQ_F32) return FN<LQ_F16, LQ_F32>(__VA_ARGS__);   \
    if ((SD) == LQ_F16 && (OD) == LQ_F16) return FN<LQ_F16, LQ_F16>(__VA_ARGS__);   \
    if ((SD) == LQ_F16 && (OD) == LQ_BF16) return FN<LQ_F16, LQ_BF16>(__VA_ARGS__); \
    if ((SD) == LQ_BF16 && (OD) == LQ_F32) return FN<LQ_BF16, LQ_F32>(__VA_ARGS__);   \
    if ((SD) == LQ_BF16 && (OD) == LQ_F16) return FN<LQ_BF16, LQ_F16>(__VA_ARGS__);   \
    if ((SD) == LQ_BF16 && (OD) == LQ_BF16) return FN<LQ_BF16, LQ_BF16>(__VA_ARGS__); \
    return LQ_ERR_DTYPE;                                                    \
  } while (0)

int launch_dequant_int4(const void* W, const void* S, void* OUT, int64_t N, int64_t K, int64_t G,
                        int sd, int od, bool fast, hipStream_t st) {
  LQ_DISPATCH_SD_OD(launch_dequant_int4_t, sd, od, W, S, OUT, N, K, G, fast, st);
}

int launch_dequant_int8(const void* W, const void* S, void* OUT, int64_t N, int64_t K, int64_t G,
                        int sd, int od, bool fast, hipStream_t st) {
  LQ_DISPATCH_SD_OD(launch_dequant_int8_t, sd, od, W, S, OUT, N, K, G, fast, st);
}

}  // namespace lq
