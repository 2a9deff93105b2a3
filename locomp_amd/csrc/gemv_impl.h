#pragma once
// Decode-shaped dequant-matmul kernels (M <= 64) for gfx950.  Included by
// gemv_w4.hip / gemv_w8.hip, which instantiate launch_skinny<WBITS>.
//
// Reference semantics: locomp examples/38_quantized_matmul.py:30-87 (int4)
// and :94-134 (int8): O[m, n] = sum_k X[m, k] * w[n, k], fp32 accumulation.
//
// Kernel choice (launch_skinny_sd_od, fp16 activations), first that applies:
//   gemv_tile_kernel    2 <= M <= 16, 512-byte row chunks, weights by DMA
//                       through an LDS ring, activations in registers
//   gemv_tile_xl_kernel 16 < M <= 64, K % 256, activations and weights by DMA
//   gemv_seg_kernel     int4, M <= 4, G % 128 == 0, K % 2048 == 0 (headline M = 1)
//   gemv_diag_kernel    int4, M <= 4, G % 128 == 0, K % 128 == 0
//   gemv_rows_kernel    int4, M <= 2, G % 32 == 0 (also the gate|up SiLU epilogue)
//   gemv_lds_kernel     M <= 16, activations + scales staged in LDS
//   skinny_mfma_kernel  M <= 64 (and everything the above reject)
//
// skinny_mfma_kernel: a workgroup of 4 waves owns 16 weight rows and all M;
// the waves split K (wave w takes k-steps w, w+4, ...) and reduce through
// LDS.  Lane l = (n = l % 16, quarter = l / 16) loads 16 packed bytes of row
// n per k-step; the bytes are dequantised in registers to exact fp16 and fed
// to the MFMA B operand; the MFMA's K order is the same for A and B, so lane
// l's A operand is X[m = l % 16, same k].  Scales: post-scale in fp32 when a
// k-step lies in one group, else the B operand is scaled in fp16.
#include "lq_common.h"
#include <type_traits>

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


// ------------------------------------------ decode GEMV, row-contiguous --
// int4, M <= 2.  Each wave owns RW whole weight rows; lane l covers the 32 k
// starting at c * 2048 + 32 * l of every row (segment c < NSEG), so each wave
// load instruction reads 1 KB contiguous of one row.  The lane's activations
// for its k-range are loaded once (k-permuted to match the decoder) and reused
// for all RW rows; their sum is kept to remove the decoder's +1032 bias.  Per
// 16 bytes of weights: 7 VALU ops decode 4 x 8 weights to biased fp16 pairs,
// 16 v_dot2_f32_f16 accumulate in fp32, and the 32-k partial is un-biased and
// scaled (the 32 k lie in one group).  Rows are reduced across the wave with a
// transposed butterfly (log2(RW) exchange stages, then 6 - log2(RW) plain
// stages).  Load order: activations, scales, then all weights, so the
// in-order vmcnt lets each row start as soon as its own bytes arrive.
// EPI: the weight rows are gate / up interleaved (row 2i = gate_i, 2i + 1 =
// up_i) and the kernel stores silu(gate_i) * up_i to O [M, N / 2] instead of
// the N dot products (examples/54_smollm2_inference.py:113-120, 545-548).
template <int M_, int NSEG, int RW, int SD, int OD, bool EPI = false>
__global__ __launch_bounds__(256, 3) void gemv_rows_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  typedef typename Elem<SD>::T stype;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  const int half_k = K >> 1;

  // 1. activations (k-permuted) for this lane's k-ranges
  u32x4_t xv[M_][NSEG][4];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + lane * 32, K - 32);
#pragma unroll
      for (int e = 0; e < 4; ++e)
        xv[m][c][e] = *reinterpret_cast<const u32x4_t*>(X + size_t(m < M ? m : 0) * K + k0 + e * 8);
    }
  // 2. scales of (row, segment)
  const stype* sp = static_cast<const stype*>(S);
  stype sv[RW][NSEG];
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + lane * 32, K - 32);
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
      const int k0 = min(c * 2048 + lane * 32, K - 32);
      const int n = min(n0 + r, N - 1);
      wv[r][c] = __builtin_nontemporal_load(
          reinterpret_cast<const u32x4_t*>(W + size_t(n) * half_k + (k0 >> 1)));
    }
  __builtin_amdgcn_sched_barrier(0);

  // 4. permute activations, bias correction per (m, segment)
  const half2_t ones = {half_t(1.f), half_t(1.f)};
  float corr[M_][NSEG];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      float sum = 0.f;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[m][c][e] = xperm8(xv[m][c][e]);
        sum = __builtin_amdgcn_fdot2(as_h2(xv[m][c][e].x), ones, sum, false);
        sum = __builtin_amdgcn_fdot2(as_h2(xv[m][c][e].y), ones, sum, false);
        sum = __builtin_amdgcn_fdot2(as_h2(xv[m][c][e].z), ones, sum, false);
        sum = __builtin_amdgcn_fdot2(as_h2(xv[m][c][e].w), ones, sum, false);
      }
      const bool valid = (m < M) && (c * 2048 + lane * 32 < K);
      corr[m][c] = valid ? sum * kInt4Bias : 0.f;
    }

  // 5. rows
  float acc[M_][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M_; ++m) acc[m][r] = 0.f;
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const bool valid = c * 2048 + lane * 32 < K;
      // four independent dot2 chains (one per dword) keep the VALU pipeline
      // busy instead of waiting on one 16-long accumulate chain
      float pe[M_][4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const u32x4_t b = int4x8_biased_kperm(wv[r][c][e]);
#pragma unroll
        for (int m = 0; m < M_; ++m) {
          float t = __builtin_amdgcn_fdot2(as_h2(b.x), as_h2(xv[m][c][e].x), 0.f, false);
          t = __builtin_amdgcn_fdot2(as_h2(b.y), as_h2(xv[m][c][e].y), t, false);
          t = __builtin_amdgcn_fdot2(as_h2(b.z), as_h2(xv[m][c][e].z), t, false);
          pe[m][e] = __builtin_amdgcn_fdot2(as_h2(b.w), as_h2(xv[m][c][e].w), t, false);
        }
      }
      float part[M_];
#pragma unroll
      for (int m = 0; m < M_; ++m) part[m] = (pe[m][0] + pe[m][1]) + (pe[m][2] + pe[m][3]);
      float sc;
      if constexpr (SD == LQ_F32) sc = sv[r][c];
      else if constexpr (SD == LQ_F16) sc = float(sv[r][c]);
      else sc = bf16_to_f32(sv[r][c]);
      sc = valid ? sc : 0.f;
#pragma unroll
      for (int m = 0; m < M_; ++m) acc[m][r] += (part[m] - corr[m][c]) * sc;
      // consume in load order: no hoisting of later rows' decode (register
      // pressure) and no early waits on their loads
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  // 6. reduce each row over the 64 lanes: transposed butterfly
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
    // lane bits 5..(6 - log2 RW) name the row
    int row = 0;
    {
      int w2 = 32;
#pragma unroll
      for (int c2 = RW; c2 > 1; c2 >>= 1, w2 >>= 1) row = row * 2 + ((lane & w2) ? 1 : 0);
    }
    const int lowmask = (64 / RW) - 1;
    if constexpr (EPI) {
      static_assert(RW % 2 == 0, "gate / up pairs within one wave");
      // row r and r ^ 1 sit in lanes that differ in bit log2(64 / RW)
      const float other = __shfl_xor(v[0], 64 / RW, 64);
      if ((lane & lowmask) == 0 && (row & 1) == 0 && m < M && n0 + row + 1 < N) {
        const float g = v[0];
        store_f32<OD>(O, size_t(m) * (N >> 1) + ((n0 + row) >> 1), g / (1.0f + expf(-g)) * other);
      }
    } else {
      if ((lane & lowmask) == 0 && m < M && n0 + row < N) store_f32<OD>(O, size_t(m) * N + n0 + row, v[0]);
    }
  }
}


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


// MFMA operand traits of the tile kernels, by weight bits and activation
// dtype XD.  kSpan = k per MFMA block (one weight dword per lane), kXLoads =
// 16-byte activation loads per lane per block, kMagic = the OR mask of the
// biased weight decode.  fp16 activations feed fp16 MFMAs.  bf16 activations
// feed bf16 MFMAs with exact integer weights: int4 as bf16 128 + q
// (0x4300 | q), int8 as 128 + q via an exact byte -> float conversion, the
// bias removed by a bias chain and the scale applied in fp32 per group.
// fp32 activations are split exactly into three bf16 parts, x = hi + mid +
// lo (hi = x truncated to bf16, mid = the residual truncated, lo = the rest,
// which has at most 8 significant bits), fed as separate MFMA rows
// (m + 4 part) whose sums are added in fp32: every product of a part and an
// integer weight is exact in fp32.
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));
typedef short s4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));
template <int WBITS, int XD = LQ_F16> struct TileMfma;
template <> struct TileMfma<4, LQ_F16> {
  static constexpr int kSpan = 32;      // k per MFMA block (one dword of int4)
  static constexpr int kXLoads = 1;
  static constexpr uint32_t kMagic = 0x64006400u;
  static constexpr bool kBiased = true;
  typedef h8 op_t;
  typedef u32x4_t x_t;                  // 8 activations per lane per block
  // (k0, k4) (k1, k5) (k2, k6) (k3, k7) as 1024 + q, 1024 + 16 q, 1024 + q, 1024 + 16 q
  __device__ static op_t decode(uint32_t w, uint32_t magic) {
    const uint32_t w8 = w >> 8;
    u32x4_t b;
    b.x = and_or(w, 0x000F000Fu, magic);
    b.y = and_or(w, 0x00F000F0u, magic);
    b.z = and_or(w8, 0x000F000Fu, magic);
    b.w = and_or(w8, 0x00F000F0u, magic);
    return __builtin_bit_cast(h8, b);
  }
  // activations in the same order, the 16 q slots divided by 16 (exact)
  __device__ static op_t prep_x(const x_t& x, int = 0) {
    const half2_t sixteenth = {half_t(0.0625f), half_t(0.0625f)};
    u32x4_t v = xperm8(x);
    v.y = as_u32(as_h2(v.y) * sixteenth);
    v.w = as_u32(as_h2(v.w) * sixteenth);
    return __builtin_bit_cast(h8, v);
  }
  // -(bias) per slot: x * (1024 + q) - 1032 x = x (q - 8); (x / 16)(1024 + 16 q) - 1152 (x / 16) = x (q - 8)
  __device__ static op_t neg_bias() {
    const half2_t a = {half_t(-1032.f), half_t(-1032.f)};
    const half2_t b = {half_t(-1152.f), half_t(-1152.f)};
    u32x4_t v;
    v.x = as_u32(a); v.y = as_u32(b); v.z = as_u32(a); v.w = as_u32(b);
    return __builtin_bit_cast(h8, v);
  }
  __device__ static float4_t mfma(const op_t& a, const op_t& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
template <> struct TileMfma<8, LQ_F16> {
  static constexpr int kSpan = 16;      // k per MFMA block (one dword of int8)
  static constexpr int kXLoads = 1;
  static constexpr uint32_t kMagic = 0x64006400u;
  static constexpr bool kBiased = false;
  typedef h4 op_t;
  typedef u32x2_t x_t;                  // 4 activations per lane per block
  __device__ static op_t decode(uint32_t w, uint32_t) {
    half2_t hb[2];
    int8x4_to_h2(w, hb);
    h4 r;
    r[0] = hb[0][0]; r[1] = hb[0][1]; r[2] = hb[1][0]; r[3] = hb[1][1];
    return r;
  }
  __device__ static op_t prep_x(const x_t& x, int = 0) { return __builtin_bit_cast(h4, x); }
  __device__ static op_t neg_bias() { return op_t{}; }
  __device__ static float4_t mfma(const op_t& a, const op_t& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
};

// int4 -> bf16 pairs (k_i, k_{i+4}) = 128 + q: nibble i of bytes 0 and 2.
__device__ __forceinline__ u32x4_t int4x8_bf16_biased(uint32_t w, uint32_t magic) {
  return int4x8_biased_kperm_m(w, magic);
}
// int8 -> four bf16 128 + q, k order kept (u = q ^ 0x80 = q + 128 is exact as
// a float and as bf16: at most 8 significant bits, so the float's low half is 0).
__device__ __forceinline__ u32x2_t int8x4_bf16_biased(uint32_t w) {
  const uint32_t u = w ^ 0x80808080u;
  const float f0 = float(u & 0xFFu), f1 = float((u >> 8) & 0xFFu);
  const float f2 = float((u >> 16) & 0xFFu), f3 = float(u >> 24);
  u32x2_t r;
  r.x = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  return r;
}
// Part `part` (0 hi, 1 mid, 2 lo) of the exact 3-way bf16 split of fp32 x,
// as the bf16 bit pattern in the high half of the returned dword.
__device__ __forceinline__ uint32_t f32_part_bits(uint32_t x, int part) {
  const uint32_t hi = x & 0xFFFF0000u;
  const float r1 = __uint_as_float(x) - __uint_as_float(hi);
  const uint32_t mid = __float_as_uint(r1) & 0xFFFF0000u;
  const float r2 = r1 - __uint_as_float(mid);
  return part == 0 ? hi : part == 1 ? mid : __float_as_uint(r2);
}

template <> struct TileMfma<4, LQ_BF16> {
  static constexpr int kSpan = 32;
  static constexpr int kXLoads = 1;
  static constexpr uint32_t kMagic = 0x43004300u;
  static constexpr bool kBiased = true;
  typedef bf8_t op_t;
  typedef u32x4_t x_t;
  __device__ static op_t decode(uint32_t w, uint32_t magic) {
    return __builtin_bit_cast(bf8_t, int4x8_bf16_biased(w, magic));
  }
  __device__ static op_t prep_x(const x_t& x, int = 0) { return __builtin_bit_cast(bf8_t, xperm8(x)); }
  __device__ static op_t neg_bias() {   // -136 = -(128 + 8)
    const u32x4_t v = {0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};
    return __builtin_bit_cast(bf8_t, v);
  }
  __device__ static float4_t mfma(const op_t& a, const op_t& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct TileMfma<8, LQ_BF16> {
  static constexpr int kSpan = 16;
  static constexpr int kXLoads = 1;
  static constexpr uint32_t kMagic = 0;
  static constexpr bool kBiased = true;
  typedef s4_t op_t;
  typedef u32x2_t x_t;
  __device__ static op_t decode(uint32_t w, uint32_t) {
    return __builtin_bit_cast(s4_t, int8x4_bf16_biased(w));
  }
  __device__ static op_t prep_x(const x_t& x, int = 0) { return __builtin_bit_cast(s4_t, x); }
  __device__ static op_t neg_bias() {   // -128
    const u32x2_t v = {0xC300C300u, 0xC300C300u};
    return __builtin_bit_cast(s4_t, v);
  }
  __device__ static float4_t mfma(const op_t& a, const op_t& b, const float4_t& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};
template <> struct TileMfma<4, LQ_F32> : TileMfma<4, LQ_BF16> {
  static constexpr int kXLoads = 2;
  typedef u32x8_t x_t;
  // 8 fp32 activations -> part `part` as bf16 in the decode's k order
  __device__ static op_t prep_x(const x_t& x, int part) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = f32_part_bits(x[i], part);
    u32x4_t v;
    v.x = __builtin_amdgcn_perm(b[4], b[0], 0x07060302u);
    v.y = __builtin_amdgcn_perm(b[5], b[1], 0x07060302u);
    v.z = __builtin_amdgcn_perm(b[6], b[2], 0x07060302u);
    v.w = __builtin_amdgcn_perm(b[7], b[3], 0x07060302u);
    return __builtin_bit_cast(bf8_t, v);
  }
};
template <> struct TileMfma<8, LQ_F32> : TileMfma<8, LQ_BF16> {
  typedef u32x4_t x_t;
  __device__ static op_t prep_x(const x_t& x, int part) {
    uint32_t b[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = f32_part_bits(x[i], part);
    u32x2_t v;
    v.x = __builtin_amdgcn_perm(b[1], b[0], 0x07060302u);
    v.y = __builtin_amdgcn_perm(b[3], b[2], 0x07060302u);
    return __builtin_bit_cast(s4_t, v);
  }
};

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
// three exact bf16 parts (hi + mid + lo) whose MFMAs chain into the same
// accumulator.  SD / OD = kRT take the dtypes from sd_rt / od_rt.
template <int M_, int NSEG, int RW, int SD, int OD, bool PART, int XD = LQ_F16>
__global__ __launch_bounds__(256, 2) void gemv_seg_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0) {
  constexpr bool kH = XD == LQ_F16;
  constexpr int NP = XD == LQ_F32 ? 3 : 1;     // bf16 parts per activation
  constexpr int kXB = XD == LQ_F32 ? 4 : 2;    // activation element bytes
  const int sd = SD == kRT ? sd_rt : SD;
  const int ssz = sd == LQ_F32 ? 4 : 2;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
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
      const int g = (c * 2048 + pos * 32) / group;
      if (ssz == 2)
        sv[r][c] = __builtin_amdgcn_raw_buffer_load_b16(rs, kin ? g * 2 : kSegOob, ((n0 + r) * num_scales) * 2, 0);
      else
        sv[r][c] = __builtin_amdgcn_raw_buffer_load_b32(rs, kin ? g * 4 : kSegOob, ((n0 + r) * num_scales) * 4, 0);
    }
  __builtin_amdgcn_sched_barrier(0);
  // 3. weights: the first kEarly chunks now, the rest after the operand
  // barriers below.  A wave reaches a barrier only once it has issued every
  // load before it, and issue stalls while the CU's memory queue is full, so
  // issuing all weights here made each workgroup wait for its slowest issuer
  // (operands ready 1.1-4.0 us after the start; 0.8-1.8 us this way).
  constexpr int kEarly = 2;
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

  // 4. activation operands and bias accumulators, built once per workgroup
  // in LDS: every thread converts M_ * NSEG of the 16-byte chunks (chunk
  // (m, c, lane, e) -> slot), then waves 0.. compute -bias for one (m, c)
  // each with 4 MFMAs, then every wave reads its operands back.
  __shared__ u32x4_t xs_l[M_ * NSEG * NP * 256];
  __shared__ float4_t nc_l[M_ * NSEG * 64];
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
                __builtin_bit_cast(u32x4_t, TileMfma<4, LQ_F32>::prep_x(x8, p));
        }
      }
  }
  __syncthreads();
  {
    for (int mc = wave; mc < M_ * NSEG; mc += 4) {
      float4_t cr = {0.f, 0.f, 0.f, 0.f};
      if constexpr (kH) {
        const half2_t b1032 = {half_t(1032.f), half_t(1032.f)};
        const half2_t b1152 = {half_t(1152.f), half_t(1152.f)};
        u32x4_t bias_w;
        bias_w.x = as_u32(b1032); bias_w.y = as_u32(b1152); bias_w.z = as_u32(b1032); bias_w.w = as_u32(b1152);
        const h8 bias_op = __builtin_bit_cast(h8, bias_w);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          cr = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              __builtin_bit_cast(h8, xs_l[mc * 256 + lane * 4 + e]), bias_op, cr, 0, 0, 0);
      } else {
        const u32x4_t b136 = {0x43084308u, 0x43084308u, 0x43084308u, 0x43084308u};   // 128 + 8
#pragma unroll
        for (int p = 0; p < NP; ++p)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            cr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf8_t, xs_l[(mc * NP + p) * 256 + lane * 4 + e]),
                __builtin_bit_cast(bf8_t, b136), cr, 0, 0, 0);
      }
      nc_l[mc * 64 + lane] = -cr;
    }
  }
  __syncthreads();
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
      negcorr[m][c] = nc_l[(m * NSEG + c) * 64 + lane];
    }

  // 5. rows: decode (5 ops / 8 weights) + MFMA, chains start at -bias
  const uint32_t magic = opaque_u32(kH ? 0x64006400u : 0x43004300u);
  float acc[M_][RW];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
#pragma unroll
    for (int m = 0; m < M_; ++m) acc[m][r] = 0.f;
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
      for (int m = 0; m < M_; ++m) {
        const float dv = dreg == 0 ? d[m][0] : dreg == 1 ? d[m][1] : dreg == 2 ? d[m][2] : d[m][3];
        acc[m][r] += dv * sc;
      }
    }
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
#pragma unroll
    for (; width > 0; width >>= 1) v[0] += __shfl_xor(v[0], width, 64);
    int row = 0;
    {
      int w2 = 32;
#pragma unroll
      for (int c2 = RW; c2 > 1; c2 >>= 1, w2 >>= 1) row = row * 2 + ((lane & w2) ? 1 : 0);
    }
    const int lowmask = (64 / RW) - 1;
    if ((lane & lowmask) == 0 && m < M && n0 + row < N) store_out<OD>(O, size_t(m) * N + n0 + row, v[0], od_rt);
  }
}


// ------------------------------------------- decode GEMV, 2 <= M <= 16 --
// A workgroup of 8 waves owns 16 T weight rows (T = 1 .. 4 16-row MFMA tiles,
// weight row = MFMA column; T is picked so the grid is at most one workgroup
// per CU) and all M <= 16 activation rows (the MFMA rows).  The weight rows
// stream through LDS in chunks of 512 bytes per row:
//   * a chunk (16 T rows, 8 T KB) is copied global -> LDS by direct-to-LDS
//     loads, 1 KB contiguous per wave instruction (two rows); 16-byte position
//     p of row r holds logical position p ^ (r & 15), so the 16 rows one LDS
//     read touches fall in 16 different bank groups;
//   * a 4-slot ring keeps chunks c + 1 .. c + 3 in flight while chunk c is
//     consumed, each together with its activations and scales (one "group"
//     of loads per chunk, issued three chunks ahead: under full load even L2
//     hits take microseconds); the loads are inline asm and every wait is
//     placed by hand;
//   * wave w takes k-eighth w of the chunk (64 bytes per row) for all row
//     tiles: 4 MFMA blocks per tile, each over one weight dword per lane
//     (int4: 16x16x32, 32 k; int8: 16x16x16, 16 k), so a group of G >= the
//     block is applied in fp32 to a chain of whole blocks;
//   * int4 weights are decoded biased (5 VALU per dword: 1024 + q, or
//     1024 + 16 q against an activation pre-divided by 16); the bias of a
//     scale group is one extra MFMA chain per wave (activations x constant),
//     shared by all tiles, that starts every tile's chain;
//   * the eight k-eighths are summed through LDS at the end.
constexpr int kTChunkB = 512;           // bytes per row per chunk
constexpr int kTSlots = 4;
constexpr int kTWaves = 8;
constexpr int kTBlocks = 4;             // MFMA blocks per wave per chunk

constexpr int kTScaleLds = 32 * 1024;  // LDS for one workgroup's scale rows

// Copies 16 bytes per lane from a raw buffer (offset voff) to LDS (lane L ->
// lds + 16 L); bytes past the buffer's size read as zero.
__device__ __forceinline__ void dma16_buf(i32x4_t rsrc, uint32_t voff, const void* lds) {
  const uint32_t a = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  __asm__ volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds"
                   :: "v"(voff), "s"(rsrc), "s"(a) : "memory", "m0");
}

// NSC = scale groups per wave k-eighth of a row (1, 2 or 4; 4 MFMA blocks);
// TILES = 16-row weight tiles per workgroup (1 .. 4); PART = the rows end in
// a partial chunk (the masked path below; whole-chunk rows skip its cost);
// EPI = gate/up rows interleaved (2i, 2i + 1): store silu(gate) * up to
// O [M, N / 2] instead of O [M, N].
// XD = activation dtype (fp16, bf16, or fp32 for M <= 4: MFMA row
// m + 4 part holds part `part` of activation row m); SD / OD = kRT take the
// scale / output dtype from sd_rt / od_rt.
template <int WBITS, int NSC, int TILES, int SD, int OD, bool PART, bool EPI = false,
          int XD = LQ_F16>
__global__ __launch_bounds__(512, 1) void gemv_tile_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0) {
  typedef TileMfma<WBITS, XD> Mf;
  typedef typename Mf::op_t op_t;
  typedef typename Mf::x_t x_t;
  constexpr int kSpan = Mf::kSpan;                      // k per MFMA block
  constexpr int kEighthK = kTBlocks * kSpan;            // k per wave per chunk
  constexpr int kChunkK = kTWaves * kEighthK;
  constexpr int kPerScale = kTBlocks / NSC;             // blocks sharing one scale
  constexpr int kXB = XD == LQ_F32 ? 4 : 2;             // activation element bytes
  constexpr bool kSplit = XD == LQ_F32;
  const int kSSize = scale_size<SD>(sd_rt);
  constexpr int kRows = 16 * TILES;
  constexpr int kDma = TILES;                           // DMA instructions per wave per chunk
  constexpr int kSlotB = kRows * kTChunkB;
  static_assert(kTSlots * kSlotB >= kTWaves * TILES * 64 * 16, "reduction reuses the ring");
  static_assert(kTSlots * kSlotB + kTScaleLds <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t wl[kTSlots * kSlotB];
  __shared__ __attribute__((aligned(16))) uint8_t sl[kTScaleLds];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int q4 = lane >> 4;
  const int n0 = blockIdx.x * kRows;
  const int row_bytes = (WBITS == 4) ? (K >> 1) : K;
  // The last chunk may be partial (row_bytes % 512 != 0): its 16-byte
  // positions past the row end take an out-of-range buffer offset and read
  // zeros, the matching activations are zeroed in compute(), and the scale
  // index is clamped to the row's last group.
  const int nchunks = (row_bytes + kTChunkB - 1) / kTChunkB;

  // DMA: wave w copies rows 2 T w .. 2 T w + 2 T - 1 of each chunk, 2 rows
  // per instruction (PART: from a raw buffer over W).
  const uint8_t* dsrc[kDma];
  const i32x4_t wrsrc = {int(uint32_t(reinterpret_cast<uint64_t>(W))),
                         int(uint32_t(reinterpret_cast<uint64_t>(W) >> 32) & 0xFFFFu),
                         int(uint32_t(N) * uint32_t(row_bytes)), 0x00020000};
  uint32_t doff[kDma];   // byte offset of the lane's 16 bytes in chunk 0
  int dpos[kDma];        // their position in the row's chunk
#pragma unroll
  for (int i = 0; i < kDma; ++i) {
    const int row = wave * 2 * kDma + 2 * i + (lane >> 5);
    const int n = min(n0 + row, N - 1);
    const int c = (lane & 31) ^ (row & 15);
    doff[i] = uint32_t(n) * uint32_t(row_bytes) + uint32_t(c * 16);
    dpos[i] = c * 16;
    dsrc[i] = W + size_t(n) * row_bytes + c * 16;
  }
  // Workgroups start at different chunks (step c reads chunk (c + rot) mod
  // nchunks) so that concurrent workgroups of one XCD read different
  // activation ranges instead of all hitting the same L2 lines.
  const int rot = (blockIdx.x >> 3) % nchunks;
  auto phys = [&](int c) { return c + rot < nchunks ? c + rot : c + rot - nchunks; };
  auto dma_chunk = [&](int slot, int c) {
    const int ch = phys(c);
#pragma unroll
    for (int i = 0; i < kDma; ++i) {
      void* dst = &wl[slot * kSlotB + (wave * 2 * kDma + 2 * i) * kTChunkB];
      if constexpr (PART)
        dma16_buf(wrsrc, ch * kTChunkB + dpos[i] < row_bytes ? doff[i] + uint32_t(ch * kTChunkB) : 0xFFFFFFF0u,
                  dst);
      else
        dma16(dsrc[i] + ch * kTChunkB, dst);
    }
  };

  // Lane (m = r16, q4) supplies activation row m, k = block * kSpan + q4 * kSpan / 4 + 0 ..
  // (fp32: MFMA row r16 = m + 4 part, m = r16 % 4)
  const int xm = kSplit ? (r16 & 3) : r16;
  const int xpart = kSplit ? (r16 >> 2) : 0;
  const uint8_t* xrow = static_cast<const uint8_t*>(X) +
                        (size_t(min(xm, M - 1)) * K + wave * kEighthK + q4 * (kSpan / 4)) * kXB;
  struct Batch {
    x_t x[kTBlocks];
  };
  // Lanes of activation rows m >= M (and fp32 part 3) load nothing (their
  // registers hold whatever they held): MFMA rows are independent and those
  // rows are never stored, so this only saves requests.
  const bool x_lane = xm < M && xpart < 3;
  auto load_batch = [&](Batch& bt, int c) {
    const int ch = phys(c);
    if (!x_lane) return;
    const int k0 = ch * kChunkK + wave * kEighthK + q4 * (kSpan / 4);
#pragma unroll
    for (int f = 0; f < kTBlocks; ++f) {
      // past K (partial last chunk): load from the row start, zeroed in compute()
      const uint8_t* px = !PART || k0 + f * kSpan < K ? xrow + size_t(ch * kChunkK + f * kSpan) * kXB
                                                       : static_cast<const uint8_t*>(X);
      if constexpr (sizeof(x_t) == 32) {
        u32x4_t a = gload_b128_cached(px), b = gload_b128_cached(px + 16);
        bt.x[f] = u32x8_t{a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      } else if constexpr (sizeof(x_t) == 16) {
        bt.x[f] = gload_b128_cached(px);
      } else {
        __asm__ volatile("global_load_dwordx2 %0, %1, off" : "=v"(bt.x[f]) : "v"(px) : "memory");
      }
    }
  };
  // A group = everything chunk c needs: its activation/scale batch and its
  // weight DMA.  Name the batch registers after the wait that covers them so
  // nothing reads them early.
  constexpr int kGroupLoads = kTBlocks * Mf::kXLoads + kDma;
  auto tie_batch = [&](Batch& bt) {
#pragma unroll
    for (int f = 0; f < kTBlocks; ++f) __asm__ volatile("" : "+v"(bt.x[f]));
  };
  // Wait until at most `pending` later groups are outstanding (vmcnt takes an
  // immediate, hence the branches).
  auto wait_group = [&](Batch& bt, int pending) {
    if (pending >= 2) __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kGroupLoads) : "memory");
    else if (pending == 1) __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(kGroupLoads) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    tie_batch(bt);
  };
  auto issue_group = [&](Batch& bt, int c) {
    load_batch(bt, c);
    dma_chunk(c & 3, c);
  };

  const uint32_t magic = opaque_u32(Mf::kMagic);
  float4_t acc[TILES];
#pragma unroll
  for (int t = 0; t < TILES; ++t) acc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
  auto compute = [&](int c, const Batch& bt) {
    const int slot = c & 3;
    const int kbase = phys(c) * kChunkK + wave * kEighthK;   // first k of this wave's eighth
    const uint8_t* lslot = &wl[slot * kSlotB];
    // All LDS reads first (weights: one dword per tile and block; scales),
    // so their latency overlaps; then the tile chains interleaved block by
    // block so consecutive MFMAs are independent.
    uint32_t w[TILES][kTBlocks];
    float sc[TILES][NSC];
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int row = t * 16 + r16;
      const uint8_t* lrow = lslot + row * kTChunkB + q4 * 4;
#pragma unroll
      for (int f = 0; f < kTBlocks; ++f) {
        const int lc = wave * kTBlocks + f;           // 16-byte position of block f
        w[t][f] = *reinterpret_cast<const uint32_t*>(lrow + ((lc ^ (row & 15)) << 4));
      }
#pragma unroll
      for (int sg = 0; sg < NSC; ++sg) {
        int g = (kbase + sg * kPerScale * kSpan) / group;
        if constexpr (PART) g = min(g, num_scales - 1);
        sc[t][sg] = load_scale<SD>(sl + (size_t(row) * num_scales + g) * kSSize, sd_rt);
      }
    }
    op_t xa[kTBlocks];
#pragma unroll
    for (int f = 0; f < kTBlocks; ++f) {
      xa[f] = Mf::prep_x(bt.x[f], xpart);
      if (PART && kbase + f * kSpan + q4 * (kSpan / 4) >= K) xa[f] = op_t{};
    }
#pragma unroll
    for (int sg = 0; sg < NSC; ++sg) {
      // bias chain of this scale group: one MFMA per block, shared by the tiles
      float4_t start = {0.f, 0.f, 0.f, 0.f};
      if constexpr (Mf::kBiased) {
        const op_t nb = Mf::neg_bias();
#pragma unroll
        for (int fb = 0; fb < kPerScale; ++fb) start = Mf::mfma(xa[sg * kPerScale + fb], nb, start);
      }
      float4_t part[TILES];
#pragma unroll
      for (int t = 0; t < TILES; ++t) part[t] = start;
#pragma unroll
      for (int fb = 0; fb < kPerScale; ++fb) {
        const int f = sg * kPerScale + fb;
#pragma unroll
        for (int t = 0; t < TILES; ++t) part[t] = Mf::mfma(xa[f], Mf::decode(w[t][f], magic), part[t]);
      }
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        acc[t] += part[t] * sc[t][sg];
        // Keep this read of the MFMA result in the block of its MFMA chain:
        // sunk past the step's branches and barrier, it was emitted without
        // the wait states an MFMA result needs before a VALU read.
        __asm__ volatile("" : "+v"(acc[t]));
      }
    }
  };

  // Step c issues group c + 3 (into ring slot and register batch (c + 3) % 4,
  // both released by step c - 1), consumes chunk c, then waits for group
  // c + 1, leaving groups c + 2 and c + 3 in flight.  Groups are issued in
  // chunk order and retire in order, so each wait is exact; no load is
  // issued for a chunk that does not exist.
  // The workgroup's scale rows n0 .. are contiguous: copy them to LDS first.
  // The buffer runs to the end of the scale array (a whole number of dwords,
  // checked by the launcher), so every wanted byte sits in an in-range dword
  // and whatever lies past the array reads as zero.
  {
    const int rows = min(kRows, N - n0);
    const uint32_t bytes = uint32_t(rows) * uint32_t(num_scales) * kSSize;
    const uint32_t avail = uint32_t(N - n0) * uint32_t(num_scales) * kSSize;
    const uint64_t base = reinterpret_cast<uint64_t>(S) + uint64_t(n0) * num_scales * kSSize;
    const i32x4_t rsrc = {int(uint32_t(base)), int(uint32_t(base >> 32) & 0xFFFFu), int(avail),
                          0x00020000};
    const int ninstr = int((bytes + 1023) >> 10);
    for (int j = wave; j < ninstr; j += kTWaves)
      dma16_buf(rsrc, uint32_t(j * 1024 + lane * 16), &sl[j * 1024]);
  }
  Batch bt0, bt1, bt2, bt3;
  issue_group(bt0, 0);
  if (nchunks > 1) issue_group(bt1, 1);
  if (nchunks > 2) issue_group(bt2, 2);
  wait_group(bt0, min(nchunks - 1, 2));
  __syncthreads();

  auto step = [&](int c, Batch& cur, Batch& next, Batch& ahead3) {
    if (c + 3 < nchunks) issue_group(ahead3, c + 3);
    compute(c, cur);
    if (c + 1 < nchunks) wait_group(next, min(nchunks - c - 2, 2));
    __syncthreads();
  };
  for (int c = 0; c < nchunks; c += 4) {
    step(c, bt0, bt1, bt3);
    if (c + 1 < nchunks) step(c + 1, bt1, bt2, bt0);
    if (c + 2 < nchunks) step(c + 2, bt2, bt3, bt1);
    if (c + 3 < nchunks) step(c + 3, bt3, bt0, bt2);
  }

  // Every load has been waited for and every wave has finished with the
  // ring (the last step ended in a barrier): reuse it for the cross-wave sum.
  float4_t* red = reinterpret_cast<float4_t*>(wl);
#pragma unroll
  for (int t = 0; t < TILES; ++t) red[(wave * TILES + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (wave < TILES) {
    const int t = wave;
    float4_t v = red[t * 64 + lane];
#pragma unroll
    for (int w = 1; w < kTWaves; ++w) v += red[(w * TILES + t) * 64 + lane];
    const int n = n0 + t * 16 + r16;
    if constexpr (kSplit) {
      // activation row m's three parts: MFMA rows m, m + 4, m + 8 = register
      // m of lanes r16, r16 + 16, r16 + 32
#pragma unroll
      for (int r = 0; r < 4; ++r) v[r] += __shfl(v[r], lane + 16, 64) + __shfl(v[r], lane + 32, 64);
      if (q4 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < M && n < N) store_out<OD>(O, size_t(r) * N + n, v[r], od_rt);
      }
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = q4 * 4 + r;
        if constexpr (EPI) {
          // rows 2i (gate) and 2i + 1 (up) sit in lanes r16 and r16 ^ 1
          const float up = __shfl_xor(v[r], 1, 64);
          const float g = v[r];
          if ((r16 & 1) == 0 && m < M && n < N)
            store_out<OD>(O, size_t(m) * (N / 2) + n / 2, g / (1.0f + expf(-g)) * up, od_rt);
        } else {
          if (m < M && n < N) store_out<OD>(O, size_t(m) * N + n, v[r], od_rt);
        }
      }
    }
  }
}

// ----------------------------- decode / verify GEMV, 16 < M <= 64, all-DMA ring --
// For 16 < M <= 64 the activations of a chunk are shared by the whole
// workgroup, so they are copied to LDS by DMA together with the weights
// instead of being loaded into each wave's registers (the M <= 16 design,
// whose registers would not hold 4 activation tiles).  A chunk is 256 k:
// 16 T weight rows (256 bytes int8 / 128 bytes int4 each) plus 64 activation
// rows x 512 bytes, all XOR-swizzled by row (16-byte positions) through the
// source addresses.  A 3-slot ring keeps chunks c + 1 and c + 2 in flight;
// the chunk's DMA instructions are dealt round-robin over the 8 waves, every
// load is a DMA, so a step's wait is a bare vmcnt of this wave's count.  Wave
// w takes k [32 w, 32 w + 32) of the chunk for all 4 x T (activation x
// weight) tiles: int8 two exact 16x16x16 blocks; int4 one 16x16x32 block
// with the 5-op biased decode, the bias one MFMA per activation tile shared
// by the T weight tiles.  The group scale (G % 32 == 0) is applied in fp32.
constexpr int kXChunkK = 256;
constexpr int kXSlots = 3;
// LDS of the ring (also the cross-wave sum) and of the scale rows: whatever
// the ring leaves of 160 KB, at most kTScaleLds.
constexpr int xl_ring_bytes(int wbits, int tiles) {
  const int slot = 16 * tiles * kXChunkK * wbits / 8 + 64 * kXChunkK * 2;
  return kXSlots * slot > 8 * 4 * tiles * 1024 ? kXSlots * slot : 8 * 4 * tiles * 1024;
}
constexpr int xl_scale_bytes(int wbits, int tiles) {
  const int left = 160 * 1024 - xl_ring_bytes(wbits, tiles);
  return (left > kTScaleLds ? kTScaleLds : left) & ~1023;
}

// EPI: gate/up rows interleaved; store silu(gate) * up to O [M, N / 2].
template <int WBITS, int TILES, int SD, int OD, bool EPI = false>
__global__ __launch_bounds__(512, 1) void gemv_tile_xl_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group) {
  typedef TileMfma<WBITS> Mf;
  typedef typename Mf::op_t op_t;
  constexpr int kRows = 16 * TILES;
  constexpr int kRowB = kXChunkK * WBITS / 8;             // weight bytes per row per chunk
  constexpr int kPos = kRowB / 16;                        // 16-byte positions per weight row
  constexpr int kWBytes = kRows * kRowB;
  constexpr int kXBytes = 64 * kXChunkK * 2;              // 64 activation rows, fp16
  constexpr int kSlotB = kWBytes + kXBytes;
  constexpr int kSSize = SD == LQ_F32 ? 4 : 2;
  constexpr int kWInstr = kWBytes / 1024;
  constexpr int kInstr = kWInstr + kXBytes / 1024;
  constexpr int kPerWaveMax = (kInstr + 7) / 8;
  static_assert(kWBytes % 1024 == 0, "whole weight DMA instructions");
  // the cross-wave sum reuses the ring (sized to hold it)
  constexpr int kRingB = xl_ring_bytes(WBITS, TILES);
  static_assert(kRingB >= kXSlots * kSlotB, "ring holds the slots");
  constexpr int kSclB = xl_scale_bytes(WBITS, TILES);
  static_assert(kRingB + kSclB <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRingB];
  __shared__ __attribute__((aligned(16))) uint8_t sl[kSclB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r16 = lane & 15;
  const int q4 = lane >> 4;
  const int n0 = blockIdx.x * kRows;
  const int row_bytes = K * WBITS / 8;
  const int nchunks = K / kXChunkK;

  // DMA instruction j = wave + 8 i: j < kWInstr copies weight rows
  // (1024 / kRowB) j .. (lane L -> row + L / kPos, position L % kPos), else
  // activation rows 2 (j - kWInstr) .. + 1 (lane L -> row + L / 32, position
  // L % 32); position p of a row holds logical 16-byte chunk p ^ (row & 15)
  // (^ (row & (kPos - 1)) for the shorter int4 weight rows).
  const int my_count = (kInstr - wave + 7) / 8;
  const uint8_t* src[kPerWaveMax];
  int dst[kPerWaveMax];
  bool is_w[kPerWaveMax];
#pragma unroll
  for (int i = 0; i < kPerWaveMax; ++i) {
    const int j = min(wave + 8 * i, kInstr - 1);
    is_w[i] = j < kWInstr;
    if (j < kWInstr) {
      const int row = (1024 / kRowB) * j + lane / kPos;
      const int n = min(n0 + row, N - 1);
      src[i] = W + size_t(n) * row_bytes + (((lane % kPos) ^ (row & (kPos - 1))) << 4);
      dst[i] = j * 1024;
    } else {
      const int row = 2 * (j - kWInstr) + (lane >> 5);
      const int m = min(row, M - 1);
      src[i] = reinterpret_cast<const uint8_t*>(X + size_t(m) * K) + (((lane & 31) ^ (row & 15)) << 4);
      dst[i] = kWBytes + (j - kWInstr) * 1024;
    }
  }
  auto issue = [&](int slot, int c) {
    uint8_t* base = &ring[slot * kSlotB];
#pragma unroll
    for (int i = 0; i < kPerWaveMax; ++i)
      if (i < my_count)
        dma16(src[i] + size_t(c) * (is_w[i] ? kRowB : kXChunkK * 2), base + dst[i]);
  };
  // wait until at most `groups` of this wave's chunk groups are outstanding
  // (a wave issues kPerWaveMax or kPerWaveMax - 1 DMAs per chunk)
  auto wait_groups = [&](int groups) {
    const bool full = my_count == kPerWaveMax;
    if (groups == 0) __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (groups == 1 && full) __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(kPerWaveMax) : "memory");
    else if (groups == 1) __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(kPerWaveMax - 1) : "memory");
    else if (full) __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kPerWaveMax) : "memory");
    else __asm__ volatile("s_waitcnt vmcnt(%0)" :: "n"(2 * kPerWaveMax - 2) : "memory");
  };

  // scale rows of the workgroup (contiguous; buffer runs to the array's end)
  {
    const int rows = min(kRows, N - n0);
    const uint32_t bytes = uint32_t(rows) * uint32_t(num_scales) * kSSize;
    const uint32_t avail = uint32_t(N - n0) * uint32_t(num_scales) * kSSize;
    const uint64_t base = reinterpret_cast<uint64_t>(S) + uint64_t(n0) * num_scales * kSSize;
    const i32x4_t rsrc = {int(uint32_t(base)), int(uint32_t(base >> 32) & 0xFFFFu), int(avail),
                          0x00020000};
    const int ninstr = int((bytes + 1023) >> 10);
    for (int j = wave; j < ninstr; j += 8)
      dma16_buf(rsrc, uint32_t(j * 1024 + lane * 16), &sl[j * 1024]);
  }

  const uint32_t magic = opaque_u32(0x64006400u);
  float4_t acc[4][TILES];
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int slot, int c) {
    const uint8_t* wl = &ring[slot * kSlotB];
    const uint8_t* xl = wl + kWBytes;
    float4_t part[4][TILES];
    if constexpr (WBITS == 8) {
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int t = 0; t < TILES; ++t) part[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int f = 0; f < 2; ++f) {
        const int kb = wave * 32 + f * 16 + q4 * 4;          // this lane's 4 k (= bytes)
        op_t bw[TILES];
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          const int row = t * 16 + r16;
          const uint32_t w = *reinterpret_cast<const uint32_t*>(
              wl + row * kRowB + (((kb >> 4) ^ (row & (kPos - 1))) << 4) + (kb & 15));
          bw[t] = Mf::decode(w, magic);
        }
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int row = mt * 16 + r16;
          const int byte = kb * 2;
          const u32x2_t xv = *reinterpret_cast<const u32x2_t*>(
              xl + row * (kXChunkK * 2) + (((byte >> 4) ^ (row & 15)) << 4) + (byte & 15));
          const op_t xa = Mf::prep_x(xv);
#pragma unroll
          for (int t = 0; t < TILES; ++t) part[mt][t] = Mf::mfma(xa, bw[t], part[mt][t]);
        }
      }
    } else {
      // one 16x16x32 block: the lane's 8 k are wave * 32 + q4 * 8 .., i.e.
      // dword q4 of weight chunk `wave` and activation bytes 64 w + 16 q4
      op_t bw[TILES];
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int row = t * 16 + r16;
        const uint32_t w = *reinterpret_cast<const uint32_t*>(
            wl + row * kRowB + ((wave ^ (row & (kPos - 1))) << 4) + (q4 << 2));
        bw[t] = Mf::decode(w, magic);
      }
      const op_t nb = Mf::neg_bias();
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        const int row = mt * 16 + r16;
        const int chunk = wave * 4 + q4;
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(
            xl + row * (kXChunkK * 2) + ((chunk ^ (row & 15)) << 4));
        const op_t xa = Mf::prep_x(xv);
        const float4_t start = Mf::mfma(xa, nb, float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int t = 0; t < TILES; ++t) part[mt][t] = Mf::mfma(xa, bw[t], start);
      }
    }
    const int g = (c * kXChunkK + wave * 32) / group;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const uint8_t* ps = sl + (size_t(t * 16 + r16) * num_scales + g) * kSSize;
      float sc;
      if constexpr (SD == LQ_F32) sc = *reinterpret_cast<const float*>(ps);
      else if constexpr (SD == LQ_F16) sc = float(*reinterpret_cast<const half_t*>(ps));
      else sc = bf16_to_f32(*reinterpret_cast<const uint16_t*>(ps));
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        acc[mt][t] += part[mt][t] * sc;
        // keep the MFMA-result read in this block (see gemv_tile_kernel)
        __asm__ volatile("" : "+v"(acc[mt][t]));
      }
    }
  };

  issue(0, 0);
  if (nchunks > 1) issue(1, 1);
  wait_groups(nchunks > 1 ? 1 : 0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    if (c + 2 < nchunks) issue((c + 2) % kXSlots, c + 2);
    compute(c % kXSlots, c);
    wait_groups(c + 2 < nchunks ? 1 : 0);
    __syncthreads();
  }

  float4_t* red = reinterpret_cast<float4_t*>(ring);
#pragma unroll
  for (int mt = 0; mt < 4; ++mt)
#pragma unroll
    for (int t = 0; t < TILES; ++t) red[((wave * 4 + mt) * TILES + t) * 64 + lane] = acc[mt][t];
  __syncthreads();
  for (int pidx = wave; pidx < 4 * TILES; pidx += 8) {
    const int mt = pidx / TILES, t = pidx % TILES;
    float4_t v = red[(mt * TILES + t) * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < 8; ++w2) v += red[((w2 * 4 + mt) * TILES + t) * 64 + lane];
    const int n = n0 + t * 16 + r16;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = mt * 16 + q4 * 4 + r;
      if constexpr (EPI) {
        const float g = v[r];
        const float up = __shfl_xor(g, 1, 64);
        if ((r16 & 1) == 0 && m < M && n < N)
          store_f32<OD>(O, size_t(m) * (N / 2) + n / 2, g / (1.0f + expf(-g)) * up);
      } else {
        if (m < M && n < N) store_f32<OD>(O, size_t(m) * N + n, v[r]);
      }
    }
  }
}

template <int WAVES, int KSPLIT>
static size_t gemv_lds_bytes(int64_t M, int64_t K, int64_t num_scales, int ssize, int step) {
  return size_t(M) * (K + 8) * 2 +
         ((size_t(16 * WAVES / KSPLIT) * num_scales * ssize + 15) & ~size_t(15)) + WAVES * 64 * 16 +
         size_t((K + step - 1) / step) * 16 * 4;
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


constexpr int kGvWaves = 8;       // waves per workgroup of the LDS GEMV
constexpr int kGvMaxLoads = 32;   // weight loads per lane: 32 x 16 B = 128 VGPRs

template <int WBITS, bool POST, int SD, int OD, int KSPLIT, int MAXJ>
static int launch_gemv_lds_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, hipStream_t st) {
  constexpr int rows = 16 * kGvWaves / KSPLIT;
  const unsigned blocks = unsigned((N + rows - 1) / rows);
  const size_t lds = gemv_lds_bytes<kGvWaves, KSPLIT>(M, K, K / G, sizeof(typename Elem<SD>::T), SkinnyGeom<WBITS>::kStep);
  hipLaunchKernelGGL((gemv_lds_kernel<WBITS, POST, SD, OD, kGvWaves, KSPLIT, MAXJ>), dim3(blocks),
                     dim3(64 * kGvWaves), lds, st, static_cast<const half_t*>(X),
                     static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K), int(K / G), int(G));
  return check_launch();
}

// Split factor for the LDS GEMV: the smallest KSPLIT that keeps each wave
// within kGvMaxLoads weight loads and yields >= 4096 waves (4 per SIMD on
// 256 CUs), else the largest; 0 when the problem does not fit the kernel
// (M > 16, LDS over 64 KB, scale rows not a multiple of 16 bytes).
static int gemv_lds_split(int64_t M, int64_t N, int64_t K, int64_t G, int step, int ssize) {
  if (M > 16) return 0;
  if ((K / G) * ssize % 16 != 0) return 0;
  if (gemv_lds_bytes<kGvWaves, 1>(M, K, K / G, ssize, step) > 64 * 1024) return 0;
  const int64_t nsteps = (K + step - 1) / step;
  for (int ks : {4, 8}) {
    if ((nsteps + ks - 1) / ks > kGvMaxLoads) continue;
    const int64_t rows = 16 * kGvWaves / ks;
    const int64_t waves = (N + rows - 1) / rows * kGvWaves;
    if (waves >= 4096 || ks == 8) return ks;
  }
  return 0;
}

template <int WBITS, bool POST, int SD, int OD, int KSPLIT>
static int launch_gemv_lds_j(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t nsteps = (K + SkinnyGeom<WBITS>::kStep - 1) / SkinnyGeom<WBITS>::kStep;
  const int64_t per_wave = (nsteps + KSPLIT - 1) / KSPLIT;
  if (per_wave <= 4) return launch_gemv_lds_t<WBITS, POST, SD, OD, KSPLIT, 4>(X, W, S, O, M, N, K, G, st);
  if (per_wave <= 8) return launch_gemv_lds_t<WBITS, POST, SD, OD, KSPLIT, 8>(X, W, S, O, M, N, K, G, st);
  if (per_wave <= 16) return launch_gemv_lds_t<WBITS, POST, SD, OD, KSPLIT, 16>(X, W, S, O, M, N, K, G, st);
  return launch_gemv_lds_t<WBITS, POST, SD, OD, KSPLIT, 32>(X, W, S, O, M, N, K, G, st);
}

template <int WBITS, bool POST, int SD, int OD>
static int launch_gemv_lds_p(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, int ks, hipStream_t st) {
  if (ks == 4) return launch_gemv_lds_j<WBITS, POST, SD, OD, 4>(X, W, S, O, M, N, K, G, st);
  return launch_gemv_lds_j<WBITS, POST, SD, OD, 8>(X, W, S, O, M, N, K, G, st);
}


template <int M_, int NSEG, int RW, int SD, int OD, bool EPI = false>
static int launch_gemv_rows_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_rows_kernel<M_, NSEG, RW, SD, OD, EPI>), dim3(blocks), dim3(256), 0, st,
                     static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                     int(N), int(K), int(K / G), int(G));
  return check_launch();
}

template <int M_, int SD, int OD, bool EPI = false>
static int launch_gemv_rows_m(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  if (nseg <= 1) return launch_gemv_rows_t<M_, 1, 4, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  if (nseg <= 2) return launch_gemv_rows_t<M_, 2, 4, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  if (nseg <= 4) return launch_gemv_rows_t<M_, 4, 2, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  return launch_gemv_rows_t<M_, 8, 2, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
}

template <int M_, int NSEG, int RW, int SD, int OD>
static int launch_gemv_diag_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_diag_kernel<M_, NSEG, RW, SD, OD>), dim3(blocks), dim3(256), 0, st,
                     static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                     int(N), int(K), int(K / G), int(G));
  return check_launch();
}

template <int M_, int SD, int OD>
static int launch_gemv_diag_m(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  constexpr int rw2 = M_ <= 2 ? 4 : 2;
  if (nseg <= 1) return launch_gemv_diag_t<M_, 1, rw2 * 2, SD, OD>(X, W, S, O, M, N, K, G, st);
  if (nseg <= 2) return launch_gemv_diag_t<M_, 2, rw2, SD, OD>(X, W, S, O, M, N, K, G, st);
  if (nseg <= 4) return launch_gemv_diag_t<M_, 4, (rw2 > 1 ? rw2 / 2 : 1), SD, OD>(X, W, S, O, M, N, K, G, st);
  return launch_gemv_diag_t<M_, 8, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
}

template <int M_, int NSEG, int RW, int SD, int OD>
static int launch_gemv_seg_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  if (K % 2048)
    hipLaunchKernelGGL((gemv_seg_kernel<M_, NSEG, RW, SD, OD, true>), dim3(blocks), dim3(256), 0, st,
                       static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                       int(N), int(K), int(K / G), int(G));
  else
    hipLaunchKernelGGL((gemv_seg_kernel<M_, NSEG, RW, SD, OD, false>), dim3(blocks), dim3(256), 0, st,
                       static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                       int(N), int(K), int(K / G), int(G));
  return check_launch();
}

template <int M_, int SD, int OD>
static int launch_gemv_seg_m(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  constexpr int rw = M_ <= 2 ? 4 : 2;
  if (nseg == 1) return launch_gemv_seg_t<M_, 1, rw * 2, SD, OD>(X, W, S, O, M, N, K, G, st);
  if (nseg == 2) return launch_gemv_seg_t<M_, 2, rw, SD, OD>(X, W, S, O, M, N, K, G, st);
  if constexpr (M_ <= 2) {
    if (nseg <= 4) return launch_gemv_seg_t<M_, 4, (rw > 2 ? rw / 2 : 1), SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (M_ == 1) return launch_gemv_seg_t<M_, 8, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
  return LQ_ERR_SHAPE;   // excluded by gemv_seg_ok
}

// The segment kernel: int4, M <= 4, G % 128 == 0, 2048 <= K <= 16384
// (K / 2048 rounded up to 1, 2, 4 or 8 segments, the last possibly partial),
// at most 8 (activation row, segment) pairs per lane (more spill registers);
// buffer sizes plus the out-of-range offset within 32 bits.
static bool gemv_seg_ok(int wbits, int64_t M, int64_t N, int64_t K, int64_t G) {
  const int64_t lim = (int64_t(1) << 31) - kSegOob;
  const int64_t nseg = (K + 2047) / 2048;
  const int64_t segs = nseg <= 1 ? 1 : nseg <= 2 ? 2 : nseg <= 4 ? 4 : 8;
  const int64_t mrows = M <= 1 ? 1 : M <= 2 ? 2 : 4;
  return wbits == 4 && M <= 4 && G % 128 == 0 && K % G == 0 && K >= 2048 && K <= 16384 &&
         mrows * segs <= 8 && N * (K / 2) < lim && M * K * 2 < lim && N * (K / G) * 4 < lim;
}

// Tiles per workgroup for the LDS-ring kernel: the smallest count whose grid
// fits one workgroup per CU (256 CUs, so no CU streams the activations
// twice), else 4; then fewer while the workgroup's scale rows exceed their
// LDS area.  0 = the scale rows of even one tile do not fit.
static int gemv_tile_count(int64_t N, int64_t K, int64_t G, int scale_bytes) {
  int tiles = 4;
  for (int t = 1; t <= 4; ++t)
    if ((N + 16 * t - 1) / (16 * t) <= 256) { tiles = t; break; }
  const int64_t row_scale_bytes = (K / G) * scale_bytes;
  while (tiles > 0 && 16 * tiles * row_scale_bytes > kTScaleLds) --tiles;
  return tiles;
}

template <int WBITS, int NSC, int SD, int OD, bool EPI = false>
static void launch_gemv_tile_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                               int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int tiles = gemv_tile_count(N, K, G, SD == LQ_F32 ? 4 : 2);
  const unsigned blocks = unsigned((N + 16 * tiles - 1) / (16 * tiles));
  const bool part = ((WBITS == 4 ? K / 2 : K) % kTChunkB) != 0;
#define LQ_TILE_LAUNCH(T_)                                                                      \
  do {                                                                                          \
    if (part)                                                                                   \
      hipLaunchKernelGGL((gemv_tile_kernel<WBITS, NSC, T_, SD, OD, true, EPI>), dim3(blocks),   \
                         dim3(512), 0, st, static_cast<const half_t*>(X),                       \
                         static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),          \
                         int(K / G), int(G));                                                   \
    else                                                                                        \
      hipLaunchKernelGGL((gemv_tile_kernel<WBITS, NSC, T_, SD, OD, false, EPI>), dim3(blocks),  \
                         dim3(512), 0, st, static_cast<const half_t*>(X),                       \
                         static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),          \
                         int(K / G), int(G));                                                   \
  } while (0)
  switch (tiles) {
    case 1: LQ_TILE_LAUNCH(1); break;
    case 2: LQ_TILE_LAUNCH(2); break;
    case 3: LQ_TILE_LAUNCH(3); break;
    default: LQ_TILE_LAUNCH(4); break;
  }
#undef LQ_TILE_LAUNCH
}

template <int WBITS, int SD, int OD, bool EPI = false>
static int launch_gemv_tile(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t eighth_k = kTBlocks * TileMfma<WBITS>::kSpan;
  const int nsc = G >= eighth_k ? 1 : int(eighth_k / G);
  switch (nsc) {
    case 1: launch_gemv_tile_t<WBITS, 1, SD, OD, EPI>(X, W, S, O, M, N, K, G, st); break;
    case 2: launch_gemv_tile_t<WBITS, 2, SD, OD, EPI>(X, W, S, O, M, N, K, G, st); break;
    default: launch_gemv_tile_t<WBITS, 4, SD, OD, EPI>(X, W, S, O, M, N, K, G, st); break;
  }
  return check_launch();
}

// The LDS-ring tile kernel: 2 <= M <= 16 (int8 also M = 1), rows of at least
// one 512-byte chunk (the last one may be partial), 16-byte multiples,
// every wave k-eighth (128 k int4 / 64 k int8) either inside one group or
// split into 2 or 4 whole groups of at least one MFMA block, and the scale
// array a whole number of dwords whose rows fit the LDS scale area.
static bool gemv_tile_ok(int wbits, int64_t M, int64_t N, int64_t K, int64_t G, int scale_bytes) {
  const int64_t row_bytes = wbits == 4 ? K / 2 : K;
  const int64_t span = wbits == 4 ? 32 : 16;
  const int64_t eighth_k = kTBlocks * span;
  const bool groups_ok = G >= eighth_k ? G % eighth_k == 0
                                       : (G >= span && eighth_k % G == 0);
  // (a partial last chunk only behind >= 4 whole ones: on shorter rows the
  // row / LDS kernels are faster)
  return M >= 1 && M <= 16 && row_bytes >= kTChunkB && row_bytes % 16 == 0 && groups_ok &&
         (row_bytes % kTChunkB == 0 || row_bytes >= 4 * kTChunkB) &&
         N * row_bytes < (int64_t(1) << 31) &&
         (N * (K / G) * scale_bytes) % 4 == 0 && gemv_tile_count(N, K, G, scale_bytes) > 0;
}

// 16 < M <= 64 on the activation-in-LDS ring: K % 256, G % 32, fp16
// activations; T = 1..4 tiles so the grid is at most one workgroup per CU,
// while the workgroup's scale rows fit 16 KB and the array is whole dwords.
static int gemv_tile_xl_count(int wbits, int64_t N, int64_t K, int64_t G, int scale_bytes) {
  int tiles = 4;
  for (int t = 1; t <= 4; ++t)
    if ((N + 16 * t - 1) / (16 * t) <= 256) { tiles = t; break; }
  // int4 rows are 128 bytes per chunk: whole 1 KB DMA instructions need T even
  if (wbits == 4 && (tiles & 1)) ++tiles;
  while (tiles > 0 && 16 * tiles * (K / G) * scale_bytes > xl_scale_bytes(wbits, tiles))
    tiles -= wbits == 4 ? 2 : 1;
  return tiles;
}
static bool gemv_tile_xl_ok(int wbits, int64_t M, int64_t N, int64_t K, int64_t G, int scale_bytes) {
  return M > 16 && M <= 64 && K % kXChunkK == 0 && G % 32 == 0 &&
         (N * (K / G) * scale_bytes) % 4 == 0 && gemv_tile_xl_count(wbits, N, K, G, scale_bytes) > 0;
}
template <int WBITS, int SD, int OD, bool EPI = false>
static int launch_gemv_tile_xl(const void* X, const void* W, const void* S, void* O, int64_t M,
                               int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int tiles = gemv_tile_xl_count(WBITS, N, K, G, SD == LQ_F32 ? 4 : 2);
  const unsigned blocks = unsigned((N + 16 * tiles - 1) / (16 * tiles));
#define LQ_TX(T_)                                                                              \
  hipLaunchKernelGGL((gemv_tile_xl_kernel<WBITS, T_, SD, OD, EPI>), dim3(blocks), dim3(512), 0, st, \
                     static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O,     \
                     int(M), int(N), int(K), int(K / G), int(G))
  if constexpr (WBITS == 8) {
    switch (tiles) {
      case 1: LQ_TX(1); break;
      case 2: LQ_TX(2); break;
      case 3: LQ_TX(3); break;
      default: LQ_TX(4); break;
    }
  } else {
    if (tiles == 2) LQ_TX(2);
    else LQ_TX(4);
  }
#undef LQ_TX
  return check_launch();
}

// The diagonal-MFMA kernel applies to int4, M <= 4, G % 128 == 0, K <= 16384.
// Register budget: the (activation row, segment) pairs a lane holds stay
// within what compiles without spills (at most 4 for M <= 2, 2 for M <= 4).
static bool gemv_diag_ok(int wbits, int64_t M, int64_t K, int64_t G) {
  const int64_t nseg = (K + 2047) / 2048;
  return wbits == 4 && M <= 4 && G % 128 == 0 && K % 128 == 0 && K <= 16384 && K >= 2048 &&
         (M <= 1 || (M <= 2 ? nseg <= 2 : nseg <= 1));
}

// The row-contiguous kernel applies to int4, M <= 2, K % 32 == 0, G % 32 == 0,
// K <= 16384.
static bool gemv_rows_ok(int wbits, int64_t M, int64_t K, int64_t G) {
  return wbits == 4 && M <= 2 && K % 32 == 0 && G % 32 == 0 && K >= 32 &&
         K <= (M == 1 ? 8192 : 2048);
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
  // the LDS-ring tile kernel also serves bf16 scales / outputs (not mixed
  // with fp32, to bound the instantiations)
  constexpr bool kTileDt = !(SD == LQ_F32 && OD == LQ_BF16) && !(SD == LQ_BF16 && OD == LQ_F32);
  if constexpr (kTileDt) {
    // int4 M = 1 keeps the segment / row kernels up to K = 8192 (faster there);
    // longer rows stream better through the LDS ring.  int4 M = 2 also takes
    // the segment kernel for K >= 4096 and N <= 8192 (4096 x 4096: 4.9 against
    // 6.1 us; at N = 11008 or K = 2048 the ring wins).
    const bool seg2 = WBITS == 4 && M == 2 && K >= 4096 && N <= 8192 && gemv_seg_ok(WBITS, M, N, K, G);
    if (!seg2 && (M >= 2 || WBITS == 8 || K > 8192) && gemv_tile_ok(WBITS, M, N, K, G, SD == LQ_F32 ? 4 : 2))
      return launch_gemv_tile<WBITS, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (kTileDt) {
    if (gemv_tile_xl_ok(WBITS, M, N, K, G, SD == LQ_F32 ? 4 : 2))
      return launch_gemv_tile_xl<WBITS, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (WBITS == 4 && (SD == LQ_BF16 || OD == LQ_BF16)) {
    // bf16 scales or output at M = 1: the segment kernel (instantiated for
    // M = 1 only; other M take the LDS / skinny kernels)
    if (M == 1 && gemv_seg_ok(WBITS, M, N, K, G))
      return launch_gemv_seg_m<1, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (WBITS == 4 && SD != LQ_BF16 && OD != LQ_BF16) {
    if (gemv_seg_ok(WBITS, M, N, K, G)) {
      if (M == 1) return launch_gemv_seg_m<1, SD, OD>(X, W, S, O, M, N, K, G, st);
      if (M == 2) return launch_gemv_seg_m<2, SD, OD>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_seg_m<4, SD, OD>(X, W, S, O, M, N, K, G, st);
    }
    if (gemv_diag_ok(WBITS, M, K, G)) {
      if (M == 1) return launch_gemv_diag_m<1, SD, OD>(X, W, S, O, M, N, K, G, st);
      if (M == 2) return launch_gemv_diag_m<2, SD, OD>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_diag_m<4, SD, OD>(X, W, S, O, M, N, K, G, st);
    }
    if (gemv_rows_ok(WBITS, M, K, G)) {
      if (M == 1) return launch_gemv_rows_m<1, SD, OD>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_rows_m<2, SD, OD>(X, W, S, O, M, N, K, G, st);
    }
  }
  const int ks = (SD != LQ_BF16 && OD != LQ_BF16)
                     ? gemv_lds_split(M, N, K, G, SkinnyGeom<WBITS>::kStep, sizeof(typename Elem<SD>::T))
                     : 0;
  if constexpr (SD != LQ_BF16 && OD != LQ_BF16) if (ks) {
    if (G % SkinnyGeom<WBITS>::kStep == 0)
      return launch_gemv_lds_p<WBITS, true, SD, OD>(X, W, S, O, M, N, K, G, ks, st);
    return launch_gemv_lds_p<WBITS, false, SD, OD>(X, W, S, O, M, N, K, G, ks, st);
  }
  if (M <= 16) return launch_skinny_mt<WBITS, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
  if (M <= 32) return launch_skinny_mt<WBITS, 2, SD, OD>(X, W, S, O, M, N, K, G, st);
  return launch_skinny_mt<WBITS, 4, SD, OD>(X, W, S, O, M, N, K, G, st);
}

// Gate|up GEMV with the SiLU * mul epilogue on the row-contiguous kernel
// (int4, M <= 2, G % 32 == 0).  Returns LQ_ERR_SHAPE when it does not apply.
template <int WBITS_ = 4>   // a template so that only the TUs that call it instantiate its kernels
int launch_rows_silu(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  // 16 < M <= 64: the activation-in-LDS kernel with the same epilogue
  if (gemv_tile_xl_ok(4, M, N, K, G, sd == LQ_F32 ? 4 : 2)) {
#define LQ_XS(SD_, OD_) \
    if (sd == SD_ && od == OD_) return launch_gemv_tile_xl<4, SD_, OD_, true>(X, W, S, O, M, N, K, G, st)
    LQ_XS(LQ_F16, LQ_F16);
    LQ_XS(LQ_F16, LQ_F32);
    LQ_XS(LQ_F32, LQ_F16);
    LQ_XS(LQ_F32, LQ_F32);
#undef LQ_XS
  }
  // 2 <= M <= 16: the LDS-ring tile kernel with the same epilogue
  if (M >= 2 && gemv_tile_ok(4, M, N, K, G, sd == LQ_F32 ? 4 : 2)) {
#define LQ_TS(SD_, OD_) \
    if (sd == SD_ && od == OD_) return launch_gemv_tile<4, SD_, OD_, true>(X, W, S, O, M, N, K, G, st)
    LQ_TS(LQ_F16, LQ_F16);
    LQ_TS(LQ_F16, LQ_F32);
    LQ_TS(LQ_F32, LQ_F16);
    LQ_TS(LQ_F32, LQ_F32);
#undef LQ_TS
  }
  if (!gemv_rows_ok(4, M, K, G)) return LQ_ERR_SHAPE;
#define LQ_RS(SD_, OD_)                                                                       \
  if (sd == SD_ && od == OD_)                                                                 \
    return M == 1 ? launch_gemv_rows_m<1, SD_, OD_, true>(X, W, S, O, M, N, K, G, st)        \
                  : launch_gemv_rows_m<2, SD_, OD_, true>(X, W, S, O, M, N, K, G, st)
  LQ_RS(LQ_F16, LQ_F16);
  LQ_RS(LQ_F16, LQ_F32);
  LQ_RS(LQ_F32, LQ_F16);
  LQ_RS(LQ_F32, LQ_F32);
#undef LQ_RS
  return LQ_ERR_SHAPE;
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

}  // namespace lq
