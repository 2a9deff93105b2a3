// gemv_seg_kernel: the 2048-k segment decode GEMV (int4, M <= 4, G % 128; the headline M = 1).
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_traits.h"

namespace lq {

// --------------------------- decode GEMV, MFMA diagonal, 2048-k segments --
// Same scheme as gemv_diag_kernel with the overhead removed:
//   * buffer loads (SGPR resource, 32-bit lane offsets, row offset in the
//     scalar operand); rows past N read as zeros;
//   * the bias correction is computed by 4 MFMAs per segment (A = the lane's
//     activations, B = the bias constants 1032 / 1152) and enters each row's
//     MFMA chain as its initial accumulator (negated), so the chain ends
//     holding x . (q - 8) directly;
//   * the diagonal is selected once per (row, segment), scaled, summed;
//   * PART (K % 2048 != 0, K % 128 == 0): the last segments take buffer
//     offsets past the end for k >= K: activations, weights and scales read
//     as zeros there (and cost no memory traffic), so those k add nothing;
//     a separate instantiation, so whole-segment rows skip the selects.
// lane offset past every buffer's end (sizes < 2^31 - 2^30 are checked on the host)
constexpr int kSegOob = 0x40000000;

// XD: activation dtype.  bf16 / fp32 activations run bf16 MFMAs on weights
// decoded to bf16 128 + q (0x4300 | q, 7 VALU ops per dword); fp32 ones as
// two bf16 parts (hi = RN(x), lo = RN(x - hi), |x - hi - lo| <= 2^-16 |x|)
// whose MFMAs chain into the same accumulator.  SD / OD = kRT take the
// dtypes from sd_rt / od_rt.
template <int M_, int NSEG, int RW, int SD, int OD, bool PART, int XD = LQ_F16>
__global__ __launch_bounds__(256, 2) void gemv_seg_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0) {
  constexpr bool kH = XD == LQ_F16;
  constexpr int NP = XD == LQ_F32 ? 2 : 1;     // bf16 parts per activation
  constexpr int kXB = XD == LQ_F32 ? 4 : 2;    // activation element bytes
  // load the output pointer now (else its kernel-argument load sits between
  // the final reduction and the store)
  __asm__ volatile("" ::"s"(reinterpret_cast<uint64_t>(O)));
  const int sd = SD == kRT ? sd_rt : SD;
  const int ssz = sd == LQ_F32 ? 4 : 2;
  const float rgroup = 1.0f / float(group);    // for div_rcp (K <= 16384 here)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  const int half_k = K >> 1;
  const int j = lane & 15, q = lane >> 4;
  const int pos = 4 * j + q;
  const bool diag = q == (j >> 2);
  const int dreg = j & 3;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(X), 0, M * K * kXB, 0x00020000);
  const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(W), 0, N * half_k, 0x00020000);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void*>(S), 0, N * num_scales * ssz, 0x00020000);

  // 1. activations (rows m >= M read as zeros): thread t fetches the chunk
  // lane t / 4 of every wave uses as its operand e = t % 4
  u32x4_t xv2[M_][NSEG][kXB / 2];   // 8 activations: one (2-byte) or two (fp32) loads
  {
    const int tl = threadIdx.x >> 2, te = threadIdx.x & 3;
    const int tpos = 4 * (tl & 15) + (tl >> 4);
#pragma unroll
    for (int m = 0; m < M_; ++m)
#pragma unroll
      for (int c = 0; c < NSEG; ++c)
#pragma unroll
        for (int h = 0; h < kXB / 2; ++h)
          xv2[m][c][h] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
              rx, !PART || c * 2048 + tpos * 32 < K ? (m * K + c * 2048 + tpos * 32 + te * 8) * kXB + 16 * h
                                                    : kSegOob,
              0, 0));
  }
  // 2. scales
  uint32_t sv[RW][NSEG];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const bool kin = !PART || c * 2048 + pos * 32 < K;
      const int g = div_rcp(c * 2048 + pos * 32, group, rgroup);
      if (ssz == 2)
        sv[r][c] = __builtin_amdgcn_raw_buffer_load_b16(rs, kin ? g * 2 : kSegOob, ((n0 + r) * num_scales) * 2, 0);
      else
        sv[r][c] = __builtin_amdgcn_raw_buffer_load_b32(rs, kin ? g * 4 : kSegOob, ((n0 + r) * num_scales) * 4, 0);
    }
  __builtin_amdgcn_sched_barrier(0);
  // 3. weights: the first kEarly chunks now, the rest after the operand
  // barrier below.  A wave reaches a barrier only once it has issued every
  // load before it, and issue stalls while the CU's memory queue is full, so
  // issuing all weights here made each workgroup wait for its slowest issuer
  // (with two barriers; with one, 4 of 8 early chunks measured best at M = 1,
  // 5.86 against 6.00 us, while M = 2 keeps 2: 8.0 against 8.7 us).
  constexpr int kEarly = M_ == 1 ? 4 : 2;
  u32x4_t wv[RW][NSEG];
  auto wload = [&](int r, int c) {
    wv[r][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
        rw, !PART || c * 2048 + pos * 32 < K ? c * 1024 + pos * 16 : kSegOob, (n0 + r) * half_k,
        2 /* nontemporal */));
  };
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c)
      if (r * NSEG + c < kEarly) wload(r, c);
  __builtin_amdgcn_sched_barrier(0);

  // 4. activation operands, built once per workgroup in LDS: every thread
  // converts M_ * NSEG of the 16-byte chunks (chunk (m, c, lane, e) -> slot);
  // then the bias chains, the remaining weight loads, and every wave reads
  // its operands back.
  __shared__ u32x4_t xs_l[M_ * NSEG * NP * 256];
  const half2_t sixteenth = {half_t(0.0625f), half_t(0.0625f)};
  {
    const int t = threadIdx.x;
#pragma unroll
    for (int m = 0; m < M_; ++m)
#pragma unroll
      for (int c = 0; c < NSEG; ++c) {
        // thread t converts the chunk that lane t / 4 uses as its e = t % 4 operand
        if constexpr (kH) {
          u32x4_t v = xperm8(xv2[m][c][0]);
          v.y = as_u32(as_h2(v.y) * sixteenth);
          v.w = as_u32(as_h2(v.w) * sixteenth);
          xs_l[(m * NSEG + c) * 256 + t] = v;
        } else if constexpr (XD == LQ_BF16) {
          xs_l[(m * NSEG + c) * 256 + t] = xperm8(xv2[m][c][0]);
        } else {
          const u32x8_t x8 = {xv2[m][c][0].x, xv2[m][c][0].y, xv2[m][c][0].z, xv2[m][c][0].w,
                              xv2[m][c][1].x, xv2[m][c][1].y, xv2[m][c][1].z, xv2[m][c][1].w};
#pragma unroll
          for (int p = 0; p < NP; ++p)
            xs_l[((m * NSEG + c) * NP + p) * 256 + t] =
                __builtin_bit_cast(u32x4_t, TileMfma<4, LQ_F32>::prep_x2(x8, p));
        }
      }
  }
  __syncthreads();
  // -bias * x per (row, segment), 4 MFMAs (x NP parts) each: fp16 activations
  // at M = 1 form them in every wave (no second barrier before the remaining
  // weight loads; measured faster also at 8 segments of one row per wave,
  // where the chains equal the row's own MFMAs); M = 2 (twice the chains:
  // 8.7 against 7.8 us at 11008 x 4096) and bf16 / fp32 activations, whose
  // chains are longer, once per workgroup in LDS (waves 0.. one (m, c) each).
  constexpr bool kOwnBias = kH && M_ == 1;
  auto bias_chain = [&](const u32x4_t* xe /* [NP][4] */) {
    float4_t cr = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kH) {
      const half2_t b1032 = {half_t(1032.f), half_t(1032.f)};
      const half2_t b1152 = {half_t(1152.f), half_t(1152.f)};
      u32x4_t bias_w;
      bias_w.x = as_u32(b1032); bias_w.y = as_u32(b1152); bias_w.z = as_u32(b1032); bias_w.w = as_u32(b1152);
      const h8 bias_op = __builtin_bit_cast(h8, bias_w);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        cr = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, xe[e]), bias_op, cr, 0, 0, 0);
    } else {
      const u32x4_t b136 = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};   // 128 + 8
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          cr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, xe[p * 4 + e]),
                                                       __builtin_bit_cast(bf8_t, b136), cr, 0, 0, 0);
    }
    return -cr;
  };
  __shared__ float4_t nc_l[kOwnBias ? 1 : M_ * NSEG * 64];
  if constexpr (!kOwnBias) {
    for (int mc = wave; mc < M_ * NSEG; mc += 4) {
      u32x4_t xe[NP * 4];
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 4; ++e) xe[p * 4 + e] = xs_l[(mc * NP + p) * 256 + lane * 4 + e];
      nc_l[mc * 64 + lane] = bias_chain(xe);
    }
    __syncthreads();
  }
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c)
      if (r * NSEG + c >= kEarly) wload(r, c);
  __builtin_amdgcn_sched_barrier(0);
  u32x4_t xv[M_][NSEG][NP][4];
  float4_t negcorr[M_][NSEG];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[m][c][p][e] = xs_l[((m * NSEG + c) * NP + p) * 256 + lane * 4 + e];
      if constexpr (kOwnBias) negcorr[m][c] = bias_chain(&xv[m][c][0][0]);
      else negcorr[m][c] = nc_l[(m * NSEG + c) * 64 + lane];
    }

  // 5. rows: decode (5 ops / 8 weights) + MFMA, chains start at -bias
  const uint32_t magic = opaque_u32(kH ? 0x64006400u : 0x43004300u);
  // acc4 keeps all four MFMA result registers scaled by the lane's scale;
  // only element dreg (the lane's diagonal entry) is used, picked once per
  // row after the last segment (a per-segment pick compiles to branches).
  float4_t acc4[M_][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M_; ++m) acc4[m][r] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      float4_t d[M_];
#pragma unroll
      for (int m = 0; m < M_; ++m) d[m] = negcorr[m][c];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = wv[r][c][e];
        if constexpr (kH) {
          const uint32_t w8 = w >> 8;
          u32x4_t b;
          b.x = and_or(w, 0x000F000Fu, magic);
          b.y = and_or(w, 0x00F000F0u, magic);
          b.z = and_or(w8, 0x000F000Fu, magic);
          b.w = and_or(w8, 0x00F000F0u, magic);
          const h8 bop = __builtin_bit_cast(h8, b);
#pragma unroll
          for (int m = 0; m < M_; ++m)
            d[m] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, xv[m][c][0][e]),
                                                          bop, d[m], 0, 0, 0);
        } else {
          const bf8_t bop = __builtin_bit_cast(bf8_t, int4x8_biased_kperm_m(w, magic));
#pragma unroll
          for (int m = 0; m < M_; ++m)
#pragma unroll
            for (int p = 0; p < NP; ++p)
              d[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf8_t, xv[m][c][p][e]),
                                                             bop, d[m], 0, 0, 0);
        }
      }
      float sc;
      if (sd == LQ_F32) sc = __uint_as_float(sv[r][c]);
      else if (sd == LQ_F16) sc = float(__builtin_bit_cast(half_t, uint16_t(sv[r][c])));
      else sc = bf16_to_f32(uint16_t(sv[r][c]));
#pragma unroll
      for (int m = 0; m < M_; ++m) acc4[m][r] += d[m] * sc;
    }
  }
  float acc[M_][RW];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      float dv = acc4[m][r][0];
      dv = dreg == 1 ? acc4[m][r][1] : dv;
      dv = dreg == 2 ? acc4[m][r][2] : dv;
      dv = dreg == 3 ? acc4[m][r][3] : dv;
      acc[m][r] = dv;
    }

  // 6. reduce each row over the 16 diagonal lanes
#pragma unroll
  for (int m = 0; m < M_; ++m) {
    float v[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) v[r] = diag ? acc[m][r] : 0.f;
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
    // the remaining full sum: LDS shuffles across the 16-lane rows, then an
    // in-row prefix sum by DPP row shifts (VALU latency instead of one LDS
    // round trip per step), which leaves the sum of each span of 2 width
    // lanes in its last lane
#pragma unroll
    for (; width >= 16; width >>= 1) v[0] += __shfl_xor(v[0], width, 64);
    if (width >= 1) v[0] += dpp_row_shr<1>(v[0]);
    if (width >= 2) v[0] += dpp_row_shr<2>(v[0]);
    if (width >= 4) v[0] += dpp_row_shr<4>(v[0]);
    if (width >= 8) v[0] += dpp_row_shr<8>(v[0]);
    int row = 0;
    {
      int w2 = 32;
#pragma unroll
      for (int c2 = RW; c2 > 1; c2 >>= 1, w2 >>= 1) row = row * 2 + ((lane & w2) ? 1 : 0);
    }
    const int lowmask = (64 / RW) - 1;
    if ((lane & lowmask) == lowmask && m < M && n0 + row < N)
      store_out<OD>(O, size_t(m) * N + n0 + row, v[0], od_rt);
  }
}

}  // namespace lq
