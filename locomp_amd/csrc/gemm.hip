// Prefill-shaped dequant-matmul for gfx950: O[M, N] = X[M, K] @ deq(W)^T with
// fp16 activations, int4 group-wise weights, fp16 MFMA and fp32 accumulation.
//
// The reference has no GEMM for this path; it would run one matvec launch per
// activation row (locomp examples/38_quantized_matmul.py:154).  Values follow
// the same definition: w = (q - 8) * s[n, k / G].
//
// Tiling: a 256-lane workgroup owns a BM x BN output tile and walks K in BK
// steps.  Per step, X[BM, BK] is copied to LDS as-is and the packed weights
// W[BN, BK/2] are loaded (one 128-bit load per lane = 32 k of one row),
// dequantised in registers to fp16 (q - 8) * s (exact (q - 8), one rounding
// of the product) and written to LDS, so each weight is dequantised once
// per workgroup.  LDS is double-buffered: the global loads for step t + 1 are
// issued before the MFMAs of step t.  Four waves in a 2 x 2 arrangement each
// compute a (BM/2) x (BN/2) sub-tile with v_mfma_f32_16x16x32_f16.
#include "lq_common.h"

namespace lq {

constexpr int kGmThreads = 256;
constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kBK = 64;
constexpr int kLdsStride = kBK + 8;  // halves; 144-byte rows spread ds_read_b128 over banks
constexpr int kWM = kBM / 2;          // wave tile
constexpr int kWN = kBN / 2;
constexpr int kTM = kWM / 16;         // 16x16 MFMA tiles per wave
constexpr int kTN = kWN / 16;

typedef _Float16 h8 __attribute__((ext_vector_type(8)));

template <int SD, int OD>
__global__ __launch_bounds__(kGmThreads, 2) void gemm_w4_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  __shared__ __attribute__((aligned(16))) half_t As[2][kBM * kLdsStride];
  __shared__ __attribute__((aligned(16))) half_t Bs[2][kBN * kLdsStride];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int r16 = lane & 15;
  const int q4 = lane >> 4;

  const int m0 = blockIdx.y * kBM;
  const int n0 = blockIdx.x * kBN;
  const int half_k = K >> 1;

  // Global -> register assignment.
  // A: 4 chunks of 16 B per lane; chunk j covers row (tid / 8) + 32 j, halves (tid % 8) * 8.
  const int a_row = tid >> 3;
  const int a_col = (tid & 7) * 8;
  // B: row tid / 2, packed bytes (tid % 2) * 16 .. +16 (= 32 k).
  const int b_row = tid >> 1;
  const int b_half = tid & 1;
  const int bn = n0 + b_row;
  const bool b_ok = bn < N;
  const uint8_t* wrow = W + size_t(b_ok ? bn : 0) * half_k;

  u32x4_t a_reg[4];
  u32x4_t b_reg;
  float b_scale = 0.f;

  auto load_tile = [&](int kt) {
    const int k0 = kt * kBK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = m0 + a_row + 32 * j;
      if (m < M)
        a_reg[j] = *reinterpret_cast<const u32x4_t*>(X + size_t(m) * K + k0 + a_col);
      else
        a_reg[j] = u32x4_t{0u, 0u, 0u, 0u};
    }
    const int kb = k0 + b_half * 32;
    if (b_ok) {
      b_reg = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + (kb >> 1)));
      b_scale = load_f32<SD>(S, size_t(bn) * num_scales + kb / group);
    } else {
      b_reg = u32x4_t{0u, 0u, 0u, 0u};
      b_scale = 0.f;
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<u32x4_t*>(&As[buf][(a_row + 32 * j) * kLdsStride + a_col]) = a_reg[j];
    const half_t hs = half_t(b_scale);
    const half2_t s2 = {hs, hs};
    half_t* dst = &Bs[buf][b_row * kLdsStride + b_half * 32];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      half2_t h[4];
      int4x8_to_h2(b_reg[i], h);
      u32x4_t v;
      v.x = as_u32(h[0] * s2);
      v.y = as_u32(h[1] * s2);
      v.z = as_u32(h[2] * s2);
      v.w = as_u32(h[3] * s2);
      *reinterpret_cast<u32x4_t*>(dst + i * 8) = v;
    }
  };

  float4_t acc[kTM][kTN];
#pragma unroll
  for (int i = 0; i < kTM; ++i)
#pragma unroll
    for (int j = 0; j < kTN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const int ktiles = K / kBK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  for (int kt = 0; kt < ktiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < ktiles) load_tile(kt + 1);
    const half_t* as = As[cur];
    const half_t* bs = Bs[cur];
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 32) {
      h8 a[kTM], b[kTN];
#pragma unroll
      for (int i = 0; i < kTM; ++i)
        a[i] = *reinterpret_cast<const h8*>(as + (wm * kWM + i * 16 + r16) * kLdsStride + kk + q4 * 8);
#pragma unroll
      for (int j = 0; j < kTN; ++j)
        b[j] = *reinterpret_cast<const h8*>(bs + (wn * kWN + j * 16 + r16) * kLdsStride + kk + q4 * 8);
#pragma unroll
      for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < ktiles) store_tile(cur ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds rows 4*(lane/16)+r, column lane%16 of each 16x16 tile.
#pragma unroll
  for (int i = 0; i < kTM; ++i) {
#pragma unroll
    for (int j = 0; j < kTN; ++j) {
      const int n = n0 + wn * kWN + j * 16 + r16;
      if (n >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * kWM + i * 16 + q4 * 4 + r;
        if (m < M) store_f32<OD>(O, size_t(m) * N + n, acc[i][j][r]);
      }
    }
  }
}

template <int SD, int OD>
static int launch_gemm_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                         int64_t N, int64_t K, int64_t G, hipStream_t st) {
  dim3 grid(unsigned((N + kBN - 1) / kBN), unsigned((M + kBM - 1) / kBM));
  hipLaunchKernelGGL((gemm_w4_kernel<SD, OD>), grid, dim3(kGmThreads), 0, st,
                     static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                     int(N), int(K), int(K / G), int(G));
  return check_launch();
}

template <int WBITS>
int launch_gemm(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  static_assert(WBITS == 4, "prefill GEMM is int4-only");
#define LQ_GM(SD_, OD_) \
  if (sd == SD_ && od == OD_) return launch_gemm_t<SD_, OD_>(X, W, S, O, M, N, K, G, st)
  LQ_GM(LQ_F16, LQ_F16);
  LQ_GM(LQ_F16, LQ_F32);
  LQ_GM(LQ_F16, LQ_BF16);
  LQ_GM(LQ_F32, LQ_F16);
  LQ_GM(LQ_F32, LQ_F32);
  LQ_GM(LQ_F32, LQ_BF16);
  LQ_GM(LQ_BF16, LQ_F16);
  LQ_GM(LQ_BF16, LQ_F32);
  LQ_GM(LQ_BF16, LQ_BF16);
#undef LQ_GM
  return LQ_ERR_DTYPE;
}

template int launch_gemm<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                            int64_t, int64_t, int, int, hipStream_t);

}  // namespace lq
