// Decode-shaped dequant-matmul (M <= 64) for gfx950, and the shape-generic
// fallback used for every case the fast kernels do not cover.
//
// Reference semantics: locomp examples/38_quantized_matmul.py:30-87 (int4)
// and :94-134 (int8): O[m, n] = sum_k X[m, k] * w[n, k], fp32 accumulation.
//
// Fast kernel ("skinny"): fp16 activations, CDNA4 v_mfma_f32_16x16x32_f16.
//   * A workgroup of 4 waves owns 16 weight rows and all M; the 4 waves split
//     K (wave w takes k-steps w, w+4, ...) and their partial 16x(16*MT)
//     tiles are summed through LDS at the end.
//   * Lane l = (n = l % 16, quarter = l / 16) loads 16 packed bytes of row n
//     per k-step with one 128-bit load; a wave instruction therefore covers
//     16 rows x 64 contiguous bytes, and the 4 waves together stream 256
//     contiguous bytes of every row.  Weights are touched exactly once.
//   * The 16 bytes are dequantised in registers to exact fp16 (q - 8) (int4)
//     or q (int8) and fed to the MFMA B operand as-is; the MFMA's K order is
//     the same for A and B, so lane l's A operand is X[m = l % 16, same k].
//   * Scales: when every k-step lies in one group (G % step == 0) the step's
//     MFMA result is multiplied by s[n, g] in fp32 ("post-scale"); otherwise
//     B is multiplied by its lane's scale in fp16 before the MFMA.
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

template <int WBITS, int MT, bool POST, int SD, int OD>
__global__ __launch_bounds__(kSkThreads) void skinny_mfma_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  typedef SkinnyGeom<WBITS> Geo;
  constexpr int kMfmaPerLoad = Geo::kLane / 8;
  __shared__ float4_t red[kSkWaves][MT][64];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nl = lane & 15;
  const int quarter = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int n = n0 + nl;
  const bool row_ok = n < N;
  const int row_bytes = (WBITS == 4) ? (K >> 1) : K;
  const uint8_t* wrow = W + size_t(row_ok ? n : 0) * row_bytes;
  const int nsteps = (K + Geo::kStep - 1) / Geo::kStep;

  float4_t acc[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};

  for (int s0 = wave; s0 < nsteps; s0 += kSkWaves * kSkBatch) {
    u32x4_t wv[kSkBatch];
#pragma unroll
    for (int b = 0; b < kSkBatch; ++b) {
      const int s = s0 + b * kSkWaves;
      const int k = s * Geo::kStep + quarter * Geo::kLane;
      if (row_ok && s < nsteps && k < K) {
        wv[b] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4_t*>(wrow + (size_t(k) * WBITS >> 3)));
      } else {
        wv[b] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int b = 0; b < kSkBatch; ++b) {
      const int s = s0 + b * kSkWaves;
      if (s >= nsteps) break;
      const int kl = s * Geo::kStep + quarter * Geo::kLane;  // lane's first k
      const bool k_ok = kl < K;
      float sc = 0.f;
      half2_t sc2 = {half_t(0.f), half_t(0.f)};
      if (POST) {
        const int g = (s * Geo::kStep) / group;
        sc = row_ok ? load_f32<SD>(S, size_t(n) * num_scales + g) : 0.f;
      } else {
        const int g = (k_ok ? kl : 0) / group;
        const half_t h = row_ok ? half_t(load_f32<SD>(S, size_t(n) * num_scales + g)) : half_t(0.f);
        sc2 = half2_t{h, h};
      }
      float4_t part[MT];
#pragma unroll
      for (int t = 0; t < MT; ++t) part[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kMfmaPerLoad; ++i) {
        half2_t hb[4];
        if constexpr (WBITS == 4) {
          const uint32_t word = wv[b][i];
          int4x8_to_h2(word, hb);
        } else {
          int8x4_to_h2(wv[b][2 * i], hb);
          int8x4_to_h2(wv[b][2 * i + 1], hb + 2);
        }
        if (!POST) {
#pragma unroll
          for (int p = 0; p < 4; ++p) hb[p] = hb[p] * sc2;
        }
        const h8 bop = make_h8(hb[0], hb[1], hb[2], hb[3]);
        const int ka = kl + i * 8;
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const int m = t * 16 + nl;
          h8 aop = {};
          if (m < M && k_ok) aop = *reinterpret_cast<const h8*>(X + size_t(m) * K + ka);
          if (POST)
            part[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, part[t], 0, 0, 0);
          else
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc[t], 0, 0, 0);
        }
      }
      if (POST) {
#pragma unroll
        for (int t = 0; t < MT; ++t) acc[t] += part[t] * sc;
      }
    }
  }

#pragma unroll
  for (int t = 0; t < MT; ++t) red[wave][t][lane] = acc[t];
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      float4_t v = red[0][t][lane] + red[1][t][lane] + red[2][t][lane] + red[3][t][lane];
      // D layout of v_mfma_f32_16x16x32: lane holds rows 4*(lane/16)+r, column lane%16.
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = t * 16 + quarter * 4 + r;
        if (m < M && row_ok) store_f32<OD>(O, size_t(m) * N + n, v[r]);
      }
    }
  }
}

// ------------------------------------------------------ generic fallback --
// One workgroup of 256 lanes per weight row; lanes stride over K, each wave
// takes every 4th activation row; fp32 math; wave reduction by shuffles.
template <int WBITS, int XD, int SD, int OD>
__global__ __launch_bounds__(256) void generic_matvec_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int64_t M, int64_t N, int64_t K, int64_t num_scales, int64_t group) {
  const int64_t n = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t row_bytes = (WBITS == 4) ? K / 2 : K;
  const uint8_t* wrow = W + n * row_bytes;
  for (int64_t m = wave; m < M; m += 4) {
    float acc = 0.f;
    for (int64_t k = lane; k < K; k += 64) {
      int q;
      if constexpr (WBITS == 4) {
        const uint32_t b = wrow[k >> 1];
        q = int((k & 1) ? (b >> 4) : (b & 0xFu)) - 8;
      } else {
        q = int(int8_t(wrow[k]));
      }
      const float w = float(q) * load_f32<SD>(S, size_t(n * num_scales + k / group));
      acc += load_f32<XD>(X, size_t(m * K + k)) * w;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if (lane == 0) store_f32<OD>(O, size_t(m * N + n), acc);
  }
}

// Writes zeros to O (K == 0: empty reduction).
template <int OD>
__global__ void zero_fill_kernel(void* O, int64_t count) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
    store_f32<OD>(O, size_t(i), 0.f);
}

// ------------------------------------------------------------ launchers --

template <int WBITS, int MT, bool POST, int SD, int OD>
static int launch_skinny_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                           int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const unsigned blocks = unsigned((N + 15) / 16);
  hipLaunchKernelGGL((skinny_mfma_kernel<WBITS, MT, POST, SD, OD>), dim3(blocks), dim3(kSkThreads),
                     0, st, static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O,
                     int(M), int(N), int(K), int(K / G), int(G));
  return check_launch();
}

template <int WBITS, int MT, int SD, int OD>
static int launch_skinny_mt(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, hipStream_t st) {
  if (G % SkinnyGeom<WBITS>::kStep == 0)
    return launch_skinny_t<WBITS, MT, true, SD, OD>(X, W, S, O, M, N, K, G, st);
  return launch_skinny_t<WBITS, MT, false, SD, OD>(X, W, S, O, M, N, K, G, st);
}

template <int WBITS, int SD, int OD>
static int launch_skinny_sd_od(const void* X, const void* W, const void* S, void* O, int64_t M,
                               int64_t N, int64_t K, int64_t G, hipStream_t st) {
  if (M <= 16) return launch_skinny_mt<WBITS, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
  if (M <= 32) return launch_skinny_mt<WBITS, 2, SD, OD>(X, W, S, O, M, N, K, G, st);
  return launch_skinny_mt<WBITS, 4, SD, OD>(X, W, S, O, M, N, K, G, st);
}

template <int WBITS>
int launch_skinny(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                  int64_t K, int64_t G, int sd, int od, hipStream_t st) {
#define LQ_SK(SD_, OD_) \
  if (sd == SD_ && od == OD_) return launch_skinny_sd_od<WBITS, SD_, OD_>(X, W, S, O, M, N, K, G, st)
  LQ_SK(LQ_F16, LQ_F16);
  LQ_SK(LQ_F16, LQ_F32);
  LQ_SK(LQ_F16, LQ_BF16);
  LQ_SK(LQ_F32, LQ_F16);
  LQ_SK(LQ_F32, LQ_F32);
  LQ_SK(LQ_F32, LQ_BF16);
  LQ_SK(LQ_BF16, LQ_F16);
  LQ_SK(LQ_BF16, LQ_F32);
  LQ_SK(LQ_BF16, LQ_BF16);
#undef LQ_SK
  return LQ_ERR_DTYPE;
}

template int launch_skinny<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, hipStream_t);
template int launch_skinny<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, hipStream_t);

template <int WBITS, int XD, int SD, int OD>
static int launch_generic_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, hipStream_t st) {
  hipLaunchKernelGGL((generic_matvec_kernel<WBITS, XD, SD, OD>), dim3(unsigned(N)), dim3(256), 0,
                     st, X, static_cast<const uint8_t*>(W), S, O, M, N, K, K / G, G);
  return check_launch();
}

template <int WBITS, int XD>
static int launch_generic_x(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
#define LQ_GN(SD_, OD_) \
  if (sd == SD_ && od == OD_) return launch_generic_t<WBITS, XD, SD_, OD_>(X, W, S, O, M, N, K, G, st)
  LQ_GN(LQ_F32, LQ_F32);
  LQ_GN(LQ_F32, LQ_F16);
  LQ_GN(LQ_F32, LQ_BF16);
  LQ_GN(LQ_F16, LQ_F32);
  LQ_GN(LQ_F16, LQ_F16);
  LQ_GN(LQ_F16, LQ_BF16);
  LQ_GN(LQ_BF16, LQ_F32);
  LQ_GN(LQ_BF16, LQ_F16);
  LQ_GN(LQ_BF16, LQ_BF16);
#undef LQ_GN
  return LQ_ERR_DTYPE;
}

template <int WBITS>
int launch_generic(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                   int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st) {
  if (xd == LQ_F32) return launch_generic_x<WBITS, LQ_F32>(X, W, S, O, M, N, K, G, sd, od, st);
  if (xd == LQ_F16) return launch_generic_x<WBITS, LQ_F16>(X, W, S, O, M, N, K, G, sd, od, st);
  if (xd == LQ_BF16) return launch_generic_x<WBITS, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
  return LQ_ERR_DTYPE;
}

template int launch_generic<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                               int64_t, int64_t, int, int, int, hipStream_t);
template int launch_generic<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                               int64_t, int64_t, int, int, int, hipStream_t);

int launch_zero_fill(void* O, int64_t count, int od, hipStream_t st) {
  unsigned blocks = unsigned(count / 256 + 1);
  if (blocks > 4096) blocks = 4096;
  if (od == LQ_F32) hipLaunchKernelGGL((zero_fill_kernel<LQ_F32>), dim3(blocks), dim3(256), 0, st, O, count);
  else if (od == LQ_F16) hipLaunchKernelGGL((zero_fill_kernel<LQ_F16>), dim3(blocks), dim3(256), 0, st, O, count);
  else if (od == LQ_BF16) hipLaunchKernelGGL((zero_fill_kernel<LQ_BF16>), dim3(blocks), dim3(256), 0, st, O, count);
  else return LQ_ERR_DTYPE;
  return check_launch();
}

}  // namespace lq
