// Residual add + RMSNorm for the decode stack around the quantized linears
// (one row of hidden size K per workgroup):
//   H[m] += R[m]                         (when R is given; H updated in place)
//   Y[m, i] = H[m, i] * rsqrt(sum_i H[m, i]^2 / K + eps) * gamma[i]
// The norm restates rms_norm_kernel (locomp examples/54_smollm2_inference.py
// :40-73: sum of squares, rsqrt(total / N + eps), val * rms * w) and the
// residual add its add_inplace_kernel (:164-167), fused so that the decode
// step launches one kernel between linears instead of two.  Arithmetic in
// fp32; H, R, gamma and Y share one dtype (fp16, bf16 or fp32).
#include "lq_common.h"

namespace lq {

template <int DT>
__global__ __launch_bounds__(256) void rms_norm_kernel(void* __restrict__ H, const void* __restrict__ R,
                                                       const void* __restrict__ gamma,
                                                       void* __restrict__ Y, int K, float eps) {
  const size_t row = size_t(blockIdx.x) * K;
  __shared__ float part[4];
  float ss = 0.f;
  for (int i = threadIdx.x; i < K; i += 256) {
    float v = load_f32<DT>(H, row + i);
    if (R) {
      v += load_f32<DT>(R, row + i);
      store_f32<DT>(H, row + i, v);
      v = load_f32<DT>(H, row + i);   // the stored hidden state is what the norm reads
    }
    ss += v * v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float rms = rsqrtf((part[0] + part[1] + part[2] + part[3]) / float(K) + eps);
  for (int i = threadIdx.x; i < K; i += 256)
    store_f32<DT>(Y, row + i, load_f32<DT>(H, row + i) * rms * load_f32<DT>(gamma, i));
}

int launch_rms_norm(void* H, const void* R, const void* gamma, void* Y, int64_t M, int64_t K,
                    float eps, int dt, hipStream_t st) {
  if (M == 0) return LQ_OK;
#define LQ_RN(DT_)                                                                                \
  hipLaunchKernelGGL((rms_norm_kernel<DT_>), dim3(unsigned(M)), dim3(256), 0, st, H, R, gamma, Y, \
                     int(K), eps)
  if (dt == LQ_F16) LQ_RN(LQ_F16);
  else if (dt == LQ_BF16) LQ_RN(LQ_BF16);
  else if (dt == LQ_F32) LQ_RN(LQ_F32);
  else return LQ_ERR_DTYPE;
#undef LQ_RN
  return check_launch();
}

}  // namespace lq
