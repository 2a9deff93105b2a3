// skinny_mfma_kernel (M <= 64, any shape) and gemv_lds_kernel (M <= 16, LDS-staged).
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_common.h"

namespace lq {

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

// -------------------------------------------- decode GEMV, LDS-staged --
// M <= 16.  Latency-oriented design:
//   * A workgroup of WAVES waves owns 16 * WAVES / KSPLIT weight rows; the
//     KSPLIT waves of a 16-row tile take interleaved k-steps (wave ks takes
//     steps ks, ks + KSPLIT, ...) and reduce through LDS at the end.  Many
//     short waves (a few k-steps each) keep several waves per SIMD resident,
//     which hides the MFMA and LDS latencies of each wave's chain.
//   * Each wave issues *all* of its 128-bit weight loads (at most MAXJ per
//     lane) before consuming any, so the whole weight matrix is in flight.
//   * Activations and the workgroup's scale rows (contiguous in memory) are
//     copied to LDS as raw 16-byte chunks whose global loads are issued
//     before the weight loads: the vmcnt counter retires loads in order, so
//     anything issued after the weights would wait for all of them.
//   * Every load is unconditional (out-of-range lanes re-read a valid
//     address) so the compiler counts outstanding loads down instead of
//     draining them; the surplus values are neutralised (zero A operand, or
//     an output column that is never written).
//   * Per k-step: the LDS reads of the A operands come first, then the
//     dequantisation, then two independent MFMA chains; with post-scaling
//     the step's scale multiply is deferred by one step so it does not wait
//     on the MFMA just issued.
constexpr int kGvXPre = 2;        // 16-byte X chunks per lane prefetched before W
constexpr int kGvSPre = 1;        // 16-byte scale chunks per lane prefetched before W

template <int WBITS, bool POST, int SD, int OD, int WAVES, int KSPLIT, int MAXJ>
__global__ __launch_bounds__(64 * WAVES) void gemv_lds_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  typedef SkinnyGeom<WBITS> Geo;
  typedef typename Elem<SD>::T stype;
  constexpr int kThreads = 64 * WAVES;
  constexpr int kMfmaPerLoad = Geo::kLane / 8;
  constexpr int kRows = 16 * WAVES / KSPLIT;
  constexpr int kSPerChunk = 16 / sizeof(stype);
  extern __shared__ __attribute__((aligned(16))) unsigned char lds_raw[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int nl = lane & 15;
  const int quarter = lane >> 4;
  const int tile = wave / KSPLIT;
  const int ks = wave % KSPLIT;
  const int n0 = blockIdx.x * kRows;
  const int n = n0 + tile * 16 + nl;
  const bool row_ok = n < N;
  const int xs = K + 8;                       // LDS row stride (halves), breaks bank aliasing
  half_t* xl = reinterpret_cast<half_t*>(lds_raw);
  stype* sl = reinterpret_cast<stype*>(lds_raw + size_t(M) * xs * 2);
  const int rows_here = min(kRows, N - n0);
  const int nsc = rows_here * num_scales;                // scale elements of this workgroup
  const int schunks = (nsc + kSPerChunk - 1) / kSPerChunk;
  float4_t* red = reinterpret_cast<float4_t*>(
      lds_raw + size_t(M) * xs * 2 + ((size_t(kRows) * num_scales * sizeof(stype) + 15) & ~size_t(15)));
  float* corr = reinterpret_cast<float*>(red + WAVES * 64);   // [nsteps][16]: BIAS * sum_k x[m, k]

  // 1. activation / scale loads first (raw 16-byte chunks, clamped indices)
  const int kc = K >> 3;                      // 16-byte chunks per X row
  const int xchunks = M * kc;
  const float inv_kc = 1.0f / float(kc);
  u32x4_t xr[kGvXPre];
#pragma unroll
  for (int i = 0; i < kGvXPre; ++i) {
    const int c = min(tid + i * kThreads, xchunks - 1);
    xr[i] = *reinterpret_cast<const u32x4_t*>(X + size_t(c) * 8);
  }
  const stype* sg = static_cast<const stype*>(S) + size_t(n0) * num_scales;
  u32x4_t sr[kGvSPre];
#pragma unroll
  for (int i = 0; i < kGvSPre; ++i) {
    const int c = min(tid + i * kThreads, schunks - 1);
    sr[i] = *reinterpret_cast<const u32x4_t*>(sg + size_t(c) * kSPerChunk);
  }
  // Keep the scheduler from interleaving the phases (it would otherwise hoist
  // the LDS stores above the weight loads and wait for the X loads there).
  __builtin_amdgcn_sched_barrier(0);

  // 2. all weight loads of this wave
  const int row_bytes = (WBITS == 4) ? (K >> 1) : K;
  const uint8_t* wrow = W + size_t(row_ok ? n : n0) * row_bytes;
  const int nsteps = (K + Geo::kStep - 1) / Geo::kStep;
  const int kmax = K - Geo::kLane;           // last valid lane start
  u32x4_t wv[MAXJ];
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int s = ks + j * KSPLIT;
    const int k = min(s * Geo::kStep + quarter * Geo::kLane, kmax);
    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(wrow + (size_t(k) * WBITS >> 3)));
  }
  __builtin_amdgcn_sched_barrier(0);

  // 3. stage X and scales in LDS.  Unconditional stores at the clamped chunk
  // index: lanes past the end rewrite the last chunk with the identical value.
#pragma unroll
  for (int i = 0; i < kGvXPre; ++i) {
    const int c = min(tid + i * kThreads, xchunks - 1);
    const int m = chunk_row(c, kc, inv_kc);
    *reinterpret_cast<u32x4_t*>(xl + m * xs + (c - m * kc) * 8) = xperm8(xr[i]);
  }
  for (int c = tid + kGvXPre * kThreads; c < xchunks; c += kThreads) {
    const int m = chunk_row(c, kc, inv_kc);
    *reinterpret_cast<u32x4_t*>(xl + m * xs + (c - m * kc) * 8) =
        xperm8(*reinterpret_cast<const u32x4_t*>(X + size_t(c) * 8));
  }
#pragma unroll
  for (int i = 0; i < kGvSPre; ++i) {
    const int c = min(tid + i * kThreads, schunks - 1);
    *reinterpret_cast<u32x4_t*>(sl + c * kSPerChunk) = sr[i];
  }
  for (int c = tid + kGvSPre * kThreads; c < schunks; c += kThreads)
    *reinterpret_cast<u32x4_t*>(sl + c * kSPerChunk) =
        *reinterpret_cast<const u32x4_t*>(sg + size_t(c) * kSPerChunk);
  __syncthreads();

  const int nsteps_all = nsteps;
  if constexpr (POST) {
    // BIAS * sum of each activation row over each k-step (runs while the
    // weight loads are still in flight).
    const half2_t ones = {half_t(1.f), half_t(1.f)};
    for (int t = tid; t < nsteps_all * 16; t += kThreads) {
      const int st = t >> 4, m = t & 15;
      float sum = 0.f;
      if (m < M) {
        const int k0 = st * Geo::kStep;
        const int k1 = min(k0 + Geo::kStep, K);
        for (int k = k0; k < k1; k += 8) {
          const u32x4_t v = *reinterpret_cast<const u32x4_t*>(xl + m * xs + k);
          sum = __builtin_amdgcn_fdot2(as_h2(v.x), ones, sum, false);
          sum = __builtin_amdgcn_fdot2(as_h2(v.y), ones, sum, false);
          sum = __builtin_amdgcn_fdot2(as_h2(v.z), ones, sum, false);
          sum = __builtin_amdgcn_fdot2(as_h2(v.w), ones, sum, false);
        }
      }
      corr[t] = sum * (WBITS == 4 ? kInt4Bias : kInt8Bias);
    }
    __syncthreads();
  }

  // 4. consume the weights in load order
  const bool a_ok = nl < M;
  const half_t* xrow = xl + nl * xs;
  const int srow_i = (row_ok ? tile * 16 + nl : 0) * num_scales;
  const half_t bias = half_t(WBITS == 4 ? kInt4Bias : kInt8Bias);
  const half2_t bias2 = {bias, bias};
  float4_t acc = {0.f, 0.f, 0.f, 0.f};
  float4_t pend = {0.f, 0.f, 0.f, 0.f};   // previous step's unscaled partial (POST)
  float pend_s = 0.f;
#pragma unroll
  for (int j = 0; j < MAXJ; ++j) {
    const int s = ks + j * KSPLIT;
    if (s >= nsteps) break;
    const int kl = s * Geo::kStep + quarter * Geo::kLane;
    const bool k_ok = kl < K;
    h8 aop[kMfmaPerLoad];
#pragma unroll
    for (int i = 0; i < kMfmaPerLoad; ++i) {
      aop[i] = h8{};
      if (a_ok && k_ok) aop[i] = *reinterpret_cast<const h8*>(xrow + kl + i * 8);
    }
    h8 bop[kMfmaPerLoad];
#pragma unroll
    for (int i = 0; i < kMfmaPerLoad; ++i) {
      u32x4_t bw;
      if constexpr (WBITS == 4) bw = int4x8_biased_kperm(wv[j][i]);
      else bw = int8x8_biased_kperm(wv[j][2 * i], wv[j][2 * i + 1]);
      if constexpr (!POST) {
        const half_t h = half_t(load_f32<SD>(sl, srow_i + (k_ok ? kl : 0) / group));
        const half2_t sc2 = {h, h};
        bw.x = as_u32((as_h2(bw.x) - bias2) * sc2);
        bw.y = as_u32((as_h2(bw.y) - bias2) * sc2);
        bw.z = as_u32((as_h2(bw.z) - bias2) * sc2);
        bw.w = as_u32((as_h2(bw.w) - bias2) * sc2);
      }
      bop[i] = __builtin_bit_cast(h8, bw);
    }
    if constexpr (POST) {
      float4_t p0 = {0.f, 0.f, 0.f, 0.f}, p1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < kMfmaPerLoad; i += 2) {
        p0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i], bop[i], p0, 0, 0, 0);
        p1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i + 1], bop[i + 1], p1, 0, 0, 0);
      }
      acc += pend * pend_s;
      pend = p0 + p1 - *reinterpret_cast<const float4_t*>(corr + s * 16 + quarter * 4);
      pend_s = load_f32<SD>(sl, srow_i + (s * Geo::kStep) / group);
    } else {
#pragma unroll
      for (int i = 0; i < kMfmaPerLoad; ++i)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop[i], bop[i], acc, 0, 0, 0);
    }
  }
  if constexpr (POST) acc += pend * pend_s;

  // 5. reduce the KSPLIT partial tiles, write O
  if constexpr (KSPLIT > 1) {
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (ks != 0) return;
#pragma unroll
    for (int k2 = 1; k2 < KSPLIT; ++k2) acc += red[(wave + k2) * 64 + lane];
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = quarter * 4 + r;
    if (m < M && row_ok) store_f32<OD>(O, size_t(m) * N + n, acc[r]);
  }
}

}  // namespace lq
