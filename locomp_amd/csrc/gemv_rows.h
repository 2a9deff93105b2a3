// gemv_rows_kernel: row-contiguous int4 decode GEMV (M <= 2, G % 32 or G % 16), with the SiLU * mul epilogue.
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_common.h"

namespace lq {

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
// OCC: workgroups per CU the register budget is sized for (2 for 8 segments).
// XD: activation dtype.  bf16 takes the weights decoded to bf16 128 + q
// (0x4300 | q) and v_dot2_f32_bf16 (exact products, fp32 sums), the bias
// 136 x the activation sum; fp32 takes the nibbles as floats q (byte
// conversions) in fp32 FMAs with the activations as loaded, the bias 8 x
// their sum.  SD / OD = kRT take the scale / output dtypes from sd_rt / od_rt.
// FUSE (decode-step fusions, examples/54_smollm2_inference.py:40-73,
// 164-167): kFuseNorm = X is the hidden state, used as
// rmsnorm(X[m]) * gamma (gamma of X's dtype; every wave forms the row's sum
// of squares from the activations it loads anyway, then rounds each
// normalized activation to X's dtype as a separate norm launch would store
// it); kFuseRes = O = X W^T + R (R of O's dtype, read before the store, so
// R may be O itself: the residual stream updated in place).
// G16: scale groups of 16 k multiples (G % 16 == 0, e.g. G = 16 or 48): each
// half of a lane's 32 k (16-aligned, so inside one group) has its own scale
// and bias correction.
constexpr int kFuseNorm = 1, kFuseRes = 2;

// Element i of an fp32 / fp16 / bf16 array whose dtype `dt` is known only at
// run time, without a branch: two 16-bit loads (the bits, for fp32 both
// halves), converted where the value is used.  (A uniform branch around the
// load makes the compiler wait for every load in flight where the paths
// join, and a conversion next to the load waits for it: either serialized
// the weight loads behind it.)
struct Bits16x2 {
  uint32_t lo, hi;   // each a zero-extended 16-bit load
};
__device__ __forceinline__ Bits16x2 load_bits_sel(const void* a, size_t i, int dt) {
  const bool f32 = dt == LQ_F32;
  const uint16_t* p = static_cast<const uint16_t*>(a) + (f32 ? 2 * i : i);
  return Bits16x2{p[0], p[f32 ? 1 : 0]};
}
__device__ __forceinline__ float bits_to_f32_sel(Bits16x2 b, int dt) {
  const float ff = __uint_as_float(b.lo | (b.hi << 16));
  const float fh = float(__builtin_bit_cast(half_t, uint16_t(b.lo)));
  const float fb = __uint_as_float(b.lo << 16);
  return dt == LQ_F32 ? ff : dt == LQ_F16 ? fh : fb;
}

template <int M_, int NSEG, int RW, int SD, int OD, bool EPI = false, int OCC = 3, int XD = LQ_F16,
          int FUSE = 0, bool G16 = false>
__global__ __launch_bounds__(256, OCC) void gemv_rows_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0, const void* __restrict__ gamma = nullptr, float eps = 0.f,
    const void* R = nullptr) {
  static_assert(!(EPI && (FUSE & kFuseRes)), "the residual add takes the plain store");
  typedef typename Elem<SD == kRT ? LQ_F32 : SD>::T stype;   // (kRT: converted at load)
  constexpr bool kH = XD == LQ_F16;
  constexpr bool kF = XD == LQ_F32;
  constexpr int NP = kF ? 2 : 1;                // u32x4 per 8 activations
  constexpr int NH = G16 ? 2 : 1;               // scales per lane k-range
  typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
  auto dot2 = [](uint32_t a, uint32_t b, float c) {
    if constexpr (kH) return __builtin_amdgcn_fdot2(as_h2(a), as_h2(b), c, false);
    else return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2_t, a), __builtin_bit_cast(bf2_t, b), c, false);
  };
  // load the output pointer now (else its kernel-argument load sits between
  // the final reduction and the store)
  __asm__ volatile("" ::"s"(reinterpret_cast<uint64_t>(O)));
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform (SGPR)
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  const int half_k = K >> 1;

  // 1. activations (k-permuted) for this lane's k-ranges
  u32x4_t xv[M_][NSEG][NP][4];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + lane * 32, K - 32);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const size_t at = size_t(m < M ? m : 0) * K + k0 + e * 8;
        if constexpr (kF) {
          const float* xf = static_cast<const float*>(X) + at;
          xv[m][c][0][e] = *reinterpret_cast<const u32x4_t*>(xf);
          xv[m][c][1][e] = *reinterpret_cast<const u32x4_t*>(xf + 4);
        } else {
          xv[m][c][0][e] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(X) + at);
        }
      }
    }
  // (kFuseNorm) the norm weights for the same k-ranges, loaded with the
  // activations; (kFuseRes) the residual of the row this lane stores
  u32x4_t gv[NSEG][NP][4];
  if constexpr ((FUSE & kFuseNorm) != 0) {
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      const int k0 = min(c * 2048 + lane * 32, K - 32);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (kF) {
          const float* gf = static_cast<const float*>(gamma) + k0 + e * 8;
          gv[c][0][e] = *reinterpret_cast<const u32x4_t*>(gf);
          gv[c][1][e] = *reinterpret_cast<const u32x4_t*>(gf + 4);
        } else {
          gv[c][0][e] = *reinterpret_cast<const u32x4_t*>(static_cast<const uint16_t*>(gamma) + k0 + e * 8);
        }
      }
    }
  }
  Bits16x2 rres[M_];
  if constexpr ((FUSE & kFuseRes) != 0) {
    int row = 0, w2 = 32;   // the row this lane stores (as the final reduction leaves it)
#pragma unroll
    for (int c2 = RW; c2 > 1; c2 >>= 1, w2 >>= 1) row = row * 2 + ((lane & w2) ? 1 : 0);
#pragma unroll
    for (int m = 0; m < M_; ++m)
      rres[m] = load_bits_sel(R, size_t(m < M ? m : 0) * N + min(n0 + row, N - 1),
                              OD == kRT ? od_rt : OD);
  }
  // 2. scales of (row, segment[, half])
  const stype* sp = static_cast<const stype*>(S);
  stype sv[RW][NSEG][NH];
  Bits16x2 svb[RW][NSEG][NH];   // (kRT: the bits, converted at use)
#pragma unroll
  for (int r = 0; r < RW; ++r)
#pragma unroll
    for (int c = 0; c < NSEG; ++c)
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        const int k0 = min(c * 2048 + lane * 32, K - 32) + 16 * h;
        const int n = min(n0 + r, N - 1);
        const size_t si = size_t(n) * num_scales + k0 / group;
        if constexpr (SD == kRT)
          svb[r][c][h] = load_bits_sel(S, si, sd_rt);
        else
          sv[r][c][h] = sp[si];
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

  if constexpr ((FUSE & kFuseNorm) != 0) {
    // rmsnorm of each activation row over all K (a wave's lanes hold every
    // k once: lane k-ranges past K, clamped to the row's end, are left out);
    // after every load has been issued, so only the activations' and norm
    // weights' latency is waited for here
    auto rnd = [](float f) -> uint32_t {   // to X's dtype, as bits
      if constexpr (kF) return __float_as_uint(f);
      else if constexpr (kH) return __builtin_bit_cast(uint16_t, half_t(f));
      else return uint32_t(f32_to_bf16(f));
    };
    // The 4 waves hold the same activations: wave w normalizes slice e = w
    // (8 of each lane's 32 k) and the slices are exchanged through LDS, a
    // quarter of the VALU work per wave (every wave doing all 32 cost the
    // 49152 x 576 LM head 5 us).
    __shared__ float nss[M_][4];
    __shared__ u32x4_t nx[M_][NSEG][4][NP][64];
    // element j (0..7) of slice e of a loaded group as fp32
    auto elem8 = [](const u32x4_t (&v)[NP][4], int e, int j) {
      if constexpr (kF) {
        const u32x4_t q = v[j >> 2][e];
        const int t = j & 3;
        return __uint_as_float(t == 0 ? q.x : t == 1 ? q.y : t == 2 ? q.z : q.w);
      } else {
        const u32x4_t q = v[0][e];
        const int t = j >> 1;
        const uint32_t d = t == 0 ? q.x : t == 1 ? q.y : t == 2 ? q.z : q.w;
        const uint16_t bb = uint16_t((j & 1) ? d >> 16 : d);
        if constexpr (kH) return float(__builtin_bit_cast(half_t, bb));
        else return __uint_as_float(uint32_t(bb) << 16);
      }
    };
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e != wave) continue;   // (uniform: one slice per wave)
#pragma unroll
      for (int m = 0; m < M_; ++m) {
        float ss = 0.f;
#pragma unroll
        for (int c = 0; c < NSEG; ++c) {
          float sc = 0.f;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float v = elem8(xv[m][c], e, j);
            sc = fmaf(v, v, sc);
          }
          ss += c * 2048 + lane * 32 < K ? sc : 0.f;
        }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
        if (lane == 0) nss[m][e] = ss;
      }
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (e != wave) continue;
#pragma unroll
      for (int m = 0; m < M_; ++m) {
        const float rms = rsqrtf((nss[m][0] + nss[m][1] + nss[m][2] + nss[m][3]) / float(K) + eps);
#pragma unroll
        for (int c = 0; c < NSEG; ++c) {
          uint32_t y[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) y[j] = rnd(elem8(xv[m][c], e, j) * rms * elem8(gv[c], e, j));
          if constexpr (kF) {
            nx[m][c][e][0][lane] = u32x4_t{y[0], y[1], y[2], y[3]};
            nx[m][c][e][1][lane] = u32x4_t{y[4], y[5], y[6], y[7]};
          } else {
            nx[m][c][e][0][lane] = u32x4_t{y[0] | (y[1] << 16), y[2] | (y[3] << 16), y[4] | (y[5] << 16),
                                           y[6] | (y[7] << 16)};
          }
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int m = 0; m < M_; ++m)
#pragma unroll
      for (int c = 0; c < NSEG; ++c)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int h = 0; h < NP; ++h) xv[m][c][h][e] = nx[m][c][e][h][lane];
  }
  // 4. permute activations, bias correction per (m, segment)
  const uint32_t ones = kH ? 0x3C003C00u : 0x3F803F80u;   // (1, 1) as fp16 / bf16
  // (G16: dwords e = 0, 1 are the first 16 k, e = 2, 3 the second)
  float corr[M_][NSEG][NH];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int c = 0; c < NSEG; ++c) {
      float sum[NH];
#pragma unroll
      for (int hh = 0; hh < NH; ++hh) sum[hh] = 0.f;
      if constexpr (kF) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const u32x4_t v = xv[m][c][h][e];
            sum[G16 ? e >> 1 : 0] +=
                (__uint_as_float(v.x) + __uint_as_float(v.y)) + (__uint_as_float(v.z) + __uint_as_float(v.w));
          }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float& su = sum[G16 ? e >> 1 : 0];
          xv[m][c][0][e] = xperm8(xv[m][c][0][e]);
          su = dot2(xv[m][c][0][e].x, ones, su);
          su = dot2(xv[m][c][0][e].y, ones, su);
          su = dot2(xv[m][c][0][e].z, ones, su);
          su = dot2(xv[m][c][0][e].w, ones, su);
        }
      }
      const bool valid = (m < M) && (c * 2048 + lane * 32 < K);
#pragma unroll
      for (int hh = 0; hh < NH; ++hh)
        corr[m][c][hh] = valid ? sum[hh] * (kF ? 8.0f : kH ? kInt4Bias : 136.0f) : 0.f;
    }
  const uint32_t magic = opaque_u32(kH ? 0x64006400u : 0x43004300u);

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
        if constexpr (kF) {
          // byte j of lo / hi = nibble 2j / 2j + 1 of the dword = k 8e + 2j (+ 1)
          const uint32_t w = wv[r][c][e];
          const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
          const float q[8] = {float(lo & 0xFFu), float(hi & 0xFFu), float((lo >> 8) & 0xFFu),
                              float((hi >> 8) & 0xFFu), float((lo >> 16) & 0xFFu),
                              float((hi >> 16) & 0xFFu), float(lo >> 24), float(hi >> 24)};
#pragma unroll
          for (int m = 0; m < M_; ++m) {
            const u32x4_t a0 = xv[m][c][0][e], a1 = xv[m][c][1][e];
            float t = q[0] * __uint_as_float(a0.x);
            t = fmaf(q[1], __uint_as_float(a0.y), t);
            t = fmaf(q[2], __uint_as_float(a0.z), t);
            t = fmaf(q[3], __uint_as_float(a0.w), t);
            t = fmaf(q[4], __uint_as_float(a1.x), t);
            t = fmaf(q[5], __uint_as_float(a1.y), t);
            t = fmaf(q[6], __uint_as_float(a1.z), t);
            pe[m][e] = fmaf(q[7], __uint_as_float(a1.w), t);
          }
        } else {
          const u32x4_t b = int4x8_biased_kperm_m(wv[r][c][e], magic);
#pragma unroll
          for (int m = 0; m < M_; ++m) {
            float t = dot2(b.x, xv[m][c][0][e].x, 0.f);
            t = dot2(b.y, xv[m][c][0][e].y, t);
            t = dot2(b.z, xv[m][c][0][e].z, t);
            pe[m][e] = dot2(b.w, xv[m][c][0][e].w, t);
          }
        }
      }
      float sc[NH];
#pragma unroll
      for (int h = 0; h < NH; ++h) {
        if constexpr (SD == kRT) sc[h] = bits_to_f32_sel(svb[r][c][h], sd_rt);
        else if constexpr (SD == LQ_F32) sc[h] = sv[r][c][h];
        else if constexpr (SD == LQ_F16) sc[h] = float(sv[r][c][h]);
        else sc[h] = bf16_to_f32(sv[r][c][h]);
        sc[h] = valid ? sc[h] : 0.f;
      }
#pragma unroll
      for (int m = 0; m < M_; ++m) {
        if constexpr (G16) {
          acc[m][r] += ((pe[m][0] + pe[m][1]) - corr[m][c][0]) * sc[0];
          acc[m][r] += ((pe[m][2] + pe[m][3]) - corr[m][c][1]) * sc[1];
        } else {
          const float part = (pe[m][0] + pe[m][1]) + (pe[m][2] + pe[m][3]);
          acc[m][r] += (part - corr[m][c][0]) * sc[0];
        }
      }
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
    // the remaining full sum: LDS shuffles across the 16-lane rows, then an
    // in-row prefix sum by DPP row shifts, which leaves the sum of each span
    // of 2 width lanes in its last lane
#pragma unroll
    for (; width >= 16; width >>= 1) v[0] += __shfl_xor(v[0], width, 64);
    if (width >= 1) v[0] += dpp_row_shr<1>(v[0]);
    if (width >= 2) v[0] += dpp_row_shr<2>(v[0]);
    if (width >= 4) v[0] += dpp_row_shr<4>(v[0]);
    if (width >= 8) v[0] += dpp_row_shr<8>(v[0]);
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
      if ((lane & lowmask) == lowmask && (row & 1) == 0 && m < M && n0 + row + 1 < N) {
        const float g = v[0];
        store_out<OD>(O, size_t(m) * (N >> 1) + ((n0 + row) >> 1), g / (1.0f + expf(-g)) * other, od_rt);
      }
    } else {
      if ((lane & lowmask) == lowmask && m < M && n0 + row < N) {
        const size_t at = size_t(m) * N + n0 + row;
        float y = v[0];
        if constexpr ((FUSE & kFuseRes) != 0) y += bits_to_f32_sel(rres[m], OD == kRT ? od_rt : OD);
        store_out<OD>(O, at, y, od_rt);
      }
    }
  }
}

}  // namespace lq
