// Shape-generic dequant-matmul fallback (any M, N, K, G, dtype) and the
// K == 0 zero fill.  fp32 VALU math; used for every case the MFMA kernels
// do not cover and, under LQ_POLICY_GENERIC, for everything.
#include "lq_common.h"

namespace lq {

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

// Gate|up dequant-matmul with the SiLU * mul epilogue, any shape and dtype:
// block i computes rows 2i (gate_i) and 2i + 1 (up_i) of the interleaved
// int4 weights and stores silu(gate_i) * up_i to O [M, N / 2]
// (examples/54_smollm2_inference.py:113-120, 545-548).
template <int XD, int SD, int OD>
__global__ __launch_bounds__(256) void generic_silu_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int64_t M, int64_t N, int64_t K, int64_t num_scales, int64_t group) {
  const int64_t i = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const uint8_t* wg = W + (2 * i) * (K / 2);
  const uint8_t* wu = wg + K / 2;
  for (int64_t m = wave; m < M; m += 4) {
    float ag = 0.f, au = 0.f;
    for (int64_t k = lane; k < K; k += 64) {
      const uint32_t bg = wg[k >> 1], bu = wu[k >> 1];
      const int qg = int((k & 1) ? (bg >> 4) : (bg & 0xFu)) - 8;
      const int qu = int((k & 1) ? (bu >> 4) : (bu & 0xFu)) - 8;
      const float x = load_f32<XD>(X, size_t(m * K + k));
      ag += x * (float(qg) * load_f32<SD>(S, size_t((2 * i) * num_scales + k / group)));
      au += x * (float(qu) * load_f32<SD>(S, size_t((2 * i + 1) * num_scales + k / group)));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      ag += __shfl_xor(ag, off, 64);
      au += __shfl_xor(au, off, 64);
    }
    if (lane == 0) store_f32<OD>(O, size_t(m * (N / 2) + i), ag / (1.0f + expf(-ag)) * au);
  }
}

template <int XD, int SD, int OD>
static int launch_generic_silu_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                                 int64_t N, int64_t K, int64_t G, hipStream_t st) {
  hipLaunchKernelGGL((generic_silu_kernel<XD, SD, OD>), dim3(unsigned(N / 2)), dim3(256), 0, st, X,
                     static_cast<const uint8_t*>(W), S, O, M, N, K, K / G, G);
  return check_launch();
}

int launch_generic_silu(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                        int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st) {
#define LQ_GS(XD_, SD_, OD_) \
  if (xd == XD_ && sd == SD_ && od == OD_) return launch_generic_silu_t<XD_, SD_, OD_>(X, W, S, O, M, N, K, G, st)
#define LQ_GS_X(XD_) \
  LQ_GS(XD_, LQ_F32, LQ_F32); LQ_GS(XD_, LQ_F32, LQ_F16); LQ_GS(XD_, LQ_F32, LQ_BF16); \
  LQ_GS(XD_, LQ_F16, LQ_F32); LQ_GS(XD_, LQ_F16, LQ_F16); LQ_GS(XD_, LQ_F16, LQ_BF16); \
  LQ_GS(XD_, LQ_BF16, LQ_F32); LQ_GS(XD_, LQ_BF16, LQ_F16); LQ_GS(XD_, LQ_BF16, LQ_BF16)
  LQ_GS_X(LQ_F32);
  LQ_GS_X(LQ_F16);
  LQ_GS_X(LQ_BF16);
#undef LQ_GS_X
#undef LQ_GS
  return LQ_ERR_DTYPE;
}

// Writes zeros to O (K == 0: empty reduction).
template <int OD>
__global__ void zero_fill_kernel(void* O, int64_t count) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
    store_f32<OD>(O, size_t(i), 0.f);
}

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
