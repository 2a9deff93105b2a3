// gemv_diag_kernel: MFMA-diagonal int4 decode GEMV (M <= 4, G % 128).
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_common.h"

namespace lq {

// ------------------------------------ decode GEMV, MFMA diagonal (M <= 4) --
// int4, G % 128 == 0.  Each wave owns RW whole weight rows.  Lane l = (j, q)
// (j = l % 16, q = l / 16) takes the 32 k at position p = 4j + q of every
// 2048-k segment c, so one wave load instruction still reads 1 KB contiguous
// of one row (lanes permuted).  The lane keeps its own activations for those
// k in registers, shared by all rows.
//
// Decode, 5 VALU ops per 8 weights: t0 = (w & 0x000F000F) | 0x6400.. gives
// (k0, k4) as 1024 + q; t1 = (w & 0x00F000F0) | .. gives (k1, k5) as
// 1024 + 16q; t2, t3 the same on w >> 8 for (k2, k6), (k3, k7).  The matching
// activations are k-permuted the same way and those multiplying a 16q half are
// pre-divided by 16 (exact), so x' . v = x (q - 8) + x * BIAS with BIAS = 1032
// or 72; the lane's BIAS * x sums are subtracted after the MFMA.
//
// Dot products run on the matrix core: MFMA t (t = 0..3, one per dword of the
// lane's 16 bytes) computes D = A B with A[i][8q + e] = lane (i, q)'s
// activations and B[8q + e][j] = lane (j, q)'s weights, so the diagonal
// D[i][i] sums lanes (i, 0..3) = the 128 k of group i of the segment; the
// other entries are discarded.  The diagonal element of group i sits in lane
// i + 16 * (i / 4), accumulator register i % 4, where it is un-biased and
// multiplied by the group scale; rows are then reduced across lanes.
template <int M_, int NSEG, int RW, int SD, int OD>
__global__ __launch_bounds__(256, 2) void gemv_diag_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  typedef typename Elem<SD>::T stype;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  const int half_k = K >> 1;
  const int j = lane & 15, q = lane >> 4;
  const int pos = 4 * j + q;
  const bool diag = q == (j >> 2);
  const int dreg = j & 3;

  // 1. activations for this lane's k-ranges
  u32x4_t xv[M_][NSEG][4];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + pos * 32, K - 32);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xv[m][c][e] = *reinterpret_cast<const u32x4_t*>(X + size_t(m < M ? m : 0) * K + k0 + e * 8);
    }
  // 2. scales of (row, segment): one group per lane quad
  const stype* sp = static_cast<const stype*>(S);
  stype sv[RW][NSEG];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + pos * 32, K - 32);
      const int n = min(n0 + r, N - 1);
      sv[r][c] = sp[size_t(n) * num_scales + k0 / group];
    }
  __builtin_amdgcn_sched_barrier(0);
  // 3. all weights of this wave
  u32x4_t wv[RW][NSEG];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + pos * 32, K - 32);
      const int n = min(n0 + r, N - 1);
      wv[r][c] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(W + size_t(n) * half_k + (k0 >> 1)));
    }
  __builtin_amdgcn_sched_barrier(0);

  // 4. activation operands: k-permute, /16 on the 16q pairs, bias sums
  const half2_t sixteenth = {half_t(0.0625f), half_t(0.0625f)};
  const half2_t ones = {half_t(1.f), half_t(1.f)};
  float corr[M_][NSEG];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const bool valid = (m < M) && (c * 2048 + pos * 32 < K);
      float s0 = 0.f, s1 = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        u32x4_t v = xperm8(xv[m][c][e]);
        if (!valid) v = u32x4_t{0u, 0u, 0u, 0u};
        s0 = __builtin_amdgcn_fdot2(as_h2(v.x), ones, s0, false);
        s0 = __builtin_amdgcn_fdot2(as_h2(v.z), ones, s0, false);
        s1 = __builtin_amdgcn_fdot2(as_h2(v.y), ones, s1, false);
        s1 = __builtin_amdgcn_fdot2(as_h2(v.w), ones, s1, false);
        v.y = as_u32(as_h2(v.y) * sixteenth);
        v.w = as_u32(as_h2(v.w) * sixteenth);
        xv[m][c][e] = v;
      }
      float cs = s0 * 1032.0f + s1 * 72.0f;
      // sum over the lane quad (j, q = 0..3) that forms one diagonal entry
      cs += __shfl_xor(cs, 16, 64);
      cs += __shfl_xor(cs, 32, 64);
      corr[m][c] = cs;
    }

  // 5. all rows at once: the RW * NSEG * M_ MFMA chains are interleaved so
  // their latencies overlap (one wait for the wave's weights).
  const uint32_t magic = opaque_u32(0x64006400u);
  float4_t d[M_][RW][NSEG];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int c = 0; c < NSEG; ++c) d[m][r][c] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
      for (int c = 0; c < NSEG; ++c) {
        const uint32_t w = wv[r][c][e];
        const uint32_t w8 = w >> 8;
        u32x4_t b;
        b.x = and_or(w, 0x000F000Fu, magic);
        b.y = and_or(w, 0x00F000F0u, magic);
        b.z = and_or(w8, 0x000F000Fu, magic);
        b.w = and_or(w8, 0x00F000F0u, magic);
        const h8 bop = __builtin_bit_cast(h8, b);
#pragma unroll
        for (int m = 0; m < M_; ++m)
          d[m][r][c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(h8, xv[m][c][e]), bop, d[m][r][c], 0, 0, 0);
      }
  }
  // un-bias and scale every accumulator register, pick the diagonal once
  float acc[M_][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    float4_t a4[M_];
    float ac[M_];
#pragma unroll
    for (int m = 0; m < M_; ++m) { a4[m] = float4_t{0.f, 0.f, 0.f, 0.f}; ac[m] = 0.f; }
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      float sc;
      if constexpr (SD == LQ_F32) sc = sv[r][c];
      else if constexpr (SD == LQ_F16) sc = float(sv[r][c]);
      else sc = bf16_to_f32(sv[r][c]);
      sc = (diag && c * 2048 + pos * 32 < K) ? sc : 0.f;
#pragma unroll
      for (int m = 0; m < M_; ++m) {
        a4[m] += d[m][r][c] * sc;
        ac[m] += corr[m][c] * sc;
      }
    }
#pragma unroll
    for (int m = 0; m < M_; ++m) {
      const float dv = dreg == 0 ? a4[m][0] : dreg == 1 ? a4[m][1] : dreg == 2 ? a4[m][2] : a4[m][3];
      acc[m][r] = dv - ac[m];
    }
  }

  // 6. reduce each row over the lanes (non-diagonal lanes hold 0)
#pragma unroll
  for (int m = 0; m < M_; ++m) {
    float v[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) v[r] = acc[m][r];
    int cnt = RW;
    int width = 32;
#pragma unroll
    for (; cnt > 1; cnt >>= 1, width >>= 1) {
      const bool upper = (lane & width) != 0;
      const int h = cnt >> 1;
#pragma unroll
      for (int i = 0; i < h; ++i) {
        const float keep = upper ? v[i + h] : v[i];
        const float send = upper ? v[i] : v[i + h];
        v[i] = keep + __shfl_xor(send, width, 64);
      }
    }
#pragma unroll
    for (; width > 0; width >>= 1) v[0] += __shfl_xor(v[0], width, 64);
    int row = 0;
    {
      int w2 = 32;
#pragma unroll
      for (int c2 = RW; c2 > 1; c2 >>= 1, w2 >>= 1) row = row * 2 + ((lane & w2) ? 1 : 0);
    }
    const int lowmask = (64 / RW) - 1;
    if ((lane & lowmask) == 0 && m < M && n0 + row < N) store_f32<OD>(O, size_t(m) * N + n0 + row, v[0]);
  }
}

}  // namespace lq
