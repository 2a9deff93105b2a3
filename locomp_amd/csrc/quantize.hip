// Weight producers on the GPU: float weights -> packed int4 / int8 plus
// per-group scales, bit-exact with the reference's NumPy quantizers
//   quantize_int4      examples/38_quantized_matmul.py:248-271
//   quantize_int8      examples/38_quantized_matmul.py:274-291
//   quantize_int4_ref  examples/52_dequantize.py:110-126
//
// Arithmetic, step by step as NumPy does it on float32 arrays (Python float
// constants are cast to float32):
//   amax  = max |w| over the group (exact)
//   38:   s = amax > 0 ? amax / 7 (or / 127) : 1        q = round(w / s)
//   52:   s = max(amax, 1e-10f) / 7                      q = round(w / (s + 1e-10f))
//   int4: q = clip(q + 8, 0, 15), byte j = q[2j] | q[2j+1] << 4;  int8: clip(q, -128, 127)
// Division is IEEE correctly rounded (HIP's float '/', or the shared-
// reciprocal form below, which gives the same result); rounding
// is half-to-even (v_rndne_f32 = np.round).
//
// Layout: lane = 8 consecutive weights of one row (two 16-byte loads for
// fp32 input), groups of G = 8 .. 512 (a power of two) are G / 8 adjacent
// lanes of one wave, their amax a shuffle-xor reduction.  Other G take a
// one-thread-per-group kernel.  HBM-bound: 4 (fp32) or 2 (16-bit) bytes in,
// 0.5 (int4) or 1 (int8) byte + 4 / G bytes out per weight.
#include "lq_common.h"

namespace lq {

enum { kQ4Ref38 = 0, kQ4Ref52 = 1, kQ8Ref38 = 2 };

template <int DT>
__device__ __forceinline__ void load8(const void* p, size_t i, float (&w)[8]) {
  if constexpr (DT == LQ_F32) {
    const u32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p) + i));
    const u32x4_t b = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const float*>(p) + i + 4));
    // Elements are copied to scalars before the bit_cast: this clang reads
    // element 0 for __builtin_bit_cast of a vector element expression (a[e]).
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t ua = a[e], ub = b[e];
      w[e] = __builtin_bit_cast(float, ua);
      w[4 + e] = __builtin_bit_cast(float, ub);
    }
  } else {
    const u32x4_t a = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(p) + i));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint16_t lo = uint16_t(a[e] & 0xFFFFu), hi = uint16_t(a[e] >> 16);
      if constexpr (DT == LQ_F16) {
        w[2 * e] = float(__builtin_bit_cast(half_t, lo));
        w[2 * e + 1] = float(__builtin_bit_cast(half_t, hi));
      } else {
        w[2 * e] = bf16_to_f32(lo);
        w[2 * e + 1] = bf16_to_f32(hi);
      }
    }
  }
}

// scale and divisor of a group from its amax
template <int MODE>
__device__ __forceinline__ void group_scale(float amax, float& s, float& div) {
  if constexpr (MODE == kQ4Ref52) {
    s = fmaxf(amax, 1e-10f) / 7.0f;
    div = s + 1e-10f;
  } else {
    s = amax > 0.0f ? amax / (MODE == kQ8Ref38 ? 127.0f : 7.0f) : 1.0f;
    div = s;
  }
}

// w / d correctly rounded with y = RN(1 / d) shared by the lane's 8 weights
// (Markstein's correction: q0 = RN(w y), r = w - q0 d exactly by an fma,
// RN(q0 + r y) = RN(w / d)); one correctly rounded division per lane
// instead of eight.  The caller keeps d and 1 / d normal and finite.
__device__ __forceinline__ float div_shared(float w, float d, float y) {
  const float q0 = w * y;
  const float r = __builtin_fmaf(-q0, d, w);
  return __builtin_fmaf(r, y, q0);
}

template <int MODE, int DT, int LPG>   // LPG = lanes per group = G / 8
__global__ __launch_bounds__(256) void quantize_lane8_kernel(
    const void* __restrict__ W, uint8_t* __restrict__ Q, float* __restrict__ S, int N, int K,
    int G) {
  const int k8s = K >> 3;                              // lanes per row
  const size_t e = size_t(blockIdx.x) * 256 + threadIdx.x;
  const size_t total = size_t(N) * k8s;
  // Every lane of a wave takes part in the shuffles; lanes past the end work
  // on a clamped copy and store nothing.
  const bool live = e < total;
  const size_t ec = live ? e : total - 1;
  const size_t row = ec / k8s;
  const int k8 = int(ec - row * k8s);
  float w[8];
  load8<DT>(W, row * K + size_t(k8) * 8, w);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(w[i]));
#pragma unroll
  for (int d = 1; d < LPG; d <<= 1) amax = fmaxf(amax, __shfl_xor(amax, d, 64));
  float s, div;
  group_scale<MODE>(amax, s, div);
  // shared reciprocal where d and 1 / d are comfortably normal, else divide
  const bool shared = div > 1e-30f && div < 1e30f;
  float qv[8];
  if (shared) {
    const float y = 1.0f / div;
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] = div_shared(w[i], div, y);
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) qv[i] = w[i] / div;
  }
  if constexpr (MODE == kQ8Ref38) {
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q = fminf(fmaxf(__builtin_rintf(qv[i]), -128.0f), 127.0f);
      const uint32_t b = uint32_t(int(q)) & 0xFFu;
      if (i < 4) lo |= b << (8 * i);
      else hi |= b << (8 * (i - 4));
    }
    if (live) *reinterpret_cast<u32x2_t*>(Q + row * K + size_t(k8) * 8) = u32x2_t{lo, hi};
  } else {
    uint32_t p = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float q = fminf(fmaxf(__builtin_rintf(qv[i]) + 8.0f, 0.0f), 15.0f);
      p |= uint32_t(q) << (4 * i);
    }
    if (live) *reinterpret_cast<uint32_t*>(Q + row * (K >> 1) + size_t(k8) * 4) = p;
  }
  if (live && (k8 % LPG) == 0) S[row * (K / G) + k8 / LPG] = s;
}

// Any G with K % G == 0 (even for int4): one thread per (row, group).
template <int MODE, int DT>
__global__ __launch_bounds__(256) void quantize_group_kernel(
    const void* __restrict__ W, uint8_t* __restrict__ Q, float* __restrict__ S, int N, int K,
    int G) {
  const int ng = K / G;
  const size_t t = size_t(blockIdx.x) * 256 + threadIdx.x;
  if (t >= size_t(N) * ng) return;
  const size_t row = t / ng;
  const int g = int(t - row * ng);
  const size_t base = row * K + size_t(g) * G;
  float amax = 0.0f;
  for (int i = 0; i < G; ++i) amax = fmaxf(amax, fabsf(load_f32<DT>(W, base + i)));
  float s, div;
  group_scale<MODE>(amax, s, div);
  S[t] = s;
  if constexpr (MODE == kQ8Ref38) {
    for (int i = 0; i < G; ++i) {
      const float q = fminf(fmaxf(__builtin_rintf(load_f32<DT>(W, base + i) / div), -128.0f), 127.0f);
      Q[base + i] = uint8_t(int(q));
    }
  } else {
    for (int i = 0; i < G; i += 2) {       // G is even for int4 (checked on the host)
      float q0 = __builtin_rintf(load_f32<DT>(W, base + i) / div);
      float q1 = __builtin_rintf(load_f32<DT>(W, base + i + 1) / div);
      q0 = fminf(fmaxf(q0 + 8.0f, 0.0f), 15.0f);
      q1 = fminf(fmaxf(q1 + 8.0f, 0.0f), 15.0f);
      Q[(base + i) >> 1] = uint8_t(uint32_t(q0) | (uint32_t(q1) << 4));
    }
  }
}

template <int MODE, int DT>
static int launch_quantize_dt(const void* W, void* Q, float* S, int64_t N, int64_t K, int64_t G,
                              bool vec_ok, hipStream_t st) {
  uint8_t* q = static_cast<uint8_t*>(Q);
  const int lpg = int(G / 8);
  if (vec_ok && G % 8 == 0 && lpg <= 64 && (lpg & (lpg - 1)) == 0) {
    const size_t lanes = size_t(N) * (K / 8);
    const unsigned blocks = unsigned((lanes + 255) / 256);
#define LQ_QL(L_)                                                                           \
  case L_:                                                                                  \
    hipLaunchKernelGGL((quantize_lane8_kernel<MODE, DT, L_>), dim3(blocks), dim3(256), 0, st, \
                       W, q, S, int(N), int(K), int(G));                                    \
    break
    switch (lpg) {
      LQ_QL(1); LQ_QL(2); LQ_QL(4); LQ_QL(8); LQ_QL(16); LQ_QL(32); LQ_QL(64);
    }
#undef LQ_QL
  } else {
    const size_t groups = size_t(N) * (K / G);
    hipLaunchKernelGGL((quantize_group_kernel<MODE, DT>), dim3(unsigned((groups + 255) / 256)),
                       dim3(256), 0, st, W, q, S, int(N), int(K), int(G));
  }
  return check_launch();
}

int launch_quantize(int mode, const void* W, void* Q, float* S, int64_t N, int64_t K, int64_t G,
                    int in_dtype, bool vec_ok, hipStream_t st) {
#define LQ_QM(M_, D_) \
  if (mode == M_ && in_dtype == D_) return launch_quantize_dt<M_, D_>(W, Q, S, N, K, G, vec_ok, st)
  LQ_QM(kQ4Ref38, LQ_F32); LQ_QM(kQ4Ref38, LQ_F16); LQ_QM(kQ4Ref38, LQ_BF16);
  LQ_QM(kQ4Ref52, LQ_F32); LQ_QM(kQ4Ref52, LQ_F16); LQ_QM(kQ4Ref52, LQ_BF16);
  LQ_QM(kQ8Ref38, LQ_F32); LQ_QM(kQ8Ref38, LQ_F16); LQ_QM(kQ8Ref38, LQ_BF16);
#undef LQ_QM
  return LQ_ERR_DTYPE;
}

}  // namespace lq
