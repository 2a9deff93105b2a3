// Dequant-matmul on fp32 VALU FMAs for scale groups the MFMA kernels do not
// take (G % 32 != 0: G = 8, 16, 24, 40, 48 ... for int4; int8 G % 4 == 0),
// any activation dtype, any M; optionally with the gate|up SiLU * mul
// epilogue.  The reference's kernels accept any G dividing K
// (examples/38_quantized_matmul.py:141-155); their arithmetic is fp32 FMAs
// on w = (q - 8) s (int4) / q s (int8), which this kernel keeps: exact
// integer weights, per-group fp32 sums scaled when the group ends.
//
// Layout: lane l of a wave owns weight row n = 64 b + l (row block b =
// blockIdx.x); all lanes walk the same k, so the activations of a step are
// wave-uniform and come through the scalar data path (scalar loads of
// X[m, k .. k + 8), int8 k + 4; fp32 FMAs, fp16 / bf16 activation pairs
// as loaded in dot2 instructions) and every group boundary is a uniform
// branch.  Each
// lane streams its own row as dwords (8 int4 / 4 int8 weights), prefetched
// a block of 8 dwords ahead.  The 4 waves of a workgroup and blockIdx.y
// (k split over workgroups) take contiguous runs of whole groups (and of
// whole 8-dword blocks where the rows allow 16-byte weight loads); the waves
// are summed through LDS, the splits by a second kernel over fp32 partial
// slices.  MT activation rows per pass (M > MT: further passes over the
// same weights, which then come from L2).
#include "lq_common.h"

namespace lq {

void* stream_workspace(int slot, size_t bytes, hipStream_t st);
int launch_split_reduce(const float* P, void* O, int64_t M, int64_t N, int splits, bool silu,
                        int od, hipStream_t st);

constexpr int kGWaves = 4;

// A run-time-dtype (fp32 / fp16 / bf16) element as its bits, loaded as two
// 16-bit halves without a branch, converted where used.
struct Bits16 {
  uint32_t lo, hi;
};
__device__ __forceinline__ Bits16 load_bits16(const void* a, size_t i, int dt) {
  const bool f32 = dt == LQ_F32;
  const uint16_t* p = static_cast<const uint16_t*>(a) + (f32 ? 2 * i : i);
  return Bits16{p[0], p[f32 ? 1 : 0]};
}
__device__ __forceinline__ float bits16_to_f32(Bits16 b, int dt) {
  const float ff = __uint_as_float(b.lo | (b.hi << 16));
  const float fh = float(__builtin_bit_cast(half_t, uint16_t(b.lo)));
  const float fb = __uint_as_float(b.lo << 16);
  return dt == LQ_F32 ? ff : dt == LQ_F16 ? fh : fb;
}

// One dword of weights -> WPD exact floats (int4: q - 8, low nibble first;
// int8: q).
template <int WBITS>
__device__ __forceinline__ void decode_dword(uint32_t d, float (&w)[8]) {
  if constexpr (WBITS == 4) {
    const uint32_t lo = d & 0x0F0F0F0Fu, hi = (d >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      w[2 * b] = float((lo >> (8 * b)) & 0xFFu) - 8.0f;
      w[2 * b + 1] = float((hi >> (8 * b)) & 0xFFu) - 8.0f;
    }
  } else {
#pragma unroll
    for (int b = 0; b < 4; ++b) w[b] = float(int8_t(uint8_t(d >> (8 * b))));
  }
}

// fp16 / bf16 activations: the decoded weights as pairs of that type
// (exact: |q - 8| <= 8, |q| <= 128), to meet the activation pairs as loaded
// in v_dot2_f32_f16 / v_dot2_f32_bf16 (exact products, fp32 sums).
template <int XD>
__device__ __forceinline__ uint32_t pack_pair(float lo, float hi) {
  if constexpr (XD == LQ_F16)
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(lo, hi));
  else
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}
template <int XD>
__device__ __forceinline__ float dot2(uint32_t x, uint32_t w, float c) {
  typedef __bf16 bf2_t __attribute__((ext_vector_type(2)));
  if constexpr (XD == LQ_F16) return __builtin_amdgcn_fdot2(as_h2(x), as_h2(w), c, false);
  else return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2_t, x), __builtin_bit_cast(bf2_t, w), c, false);
}

// P: fp32 partial slices [gridDim.y][M][N] when gridDim.y > 1, else O.
// unit: dwords per run unit (whole groups; VEC: also whole blocks, and the
// weight rows 16-byte aligned, so each block is two 16-byte loads).
template <int WBITS, int XD, int MT, bool EPI, bool VEC>
__global__ __launch_bounds__(64 * kGWaves) void group_valu_kernel(
    const void* __restrict__ X, const uint32_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, float* __restrict__ P, int M, int N, int K, int num_scales, int group,
    int unit, int sd, int od) {
  constexpr int kWpd = WBITS == 4 ? 8 : 4;              // weights per dword
  constexpr int kDepth = 8;                             // dwords per prefetch block
  constexpr int kR = MT < 2 ? MT : 2;                   // activation rows per scalar batch
  __shared__ float red[kGWaves][MT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = blockIdx.x * 64 + lane;
  const int nr = min(n, N - 1);
  const int row_dw = K / kWpd;                          // dwords per weight row
  const int gdw = group / kWpd;                         // dwords per group
  // this wave's run of whole units
  const int pieces = gridDim.y * kGWaves;
  const int piece = blockIdx.y * kGWaves + wave;
  const int units = row_dw / unit;
  const int d0 = int(int64_t(units) * piece / pieces) * unit;
  const int d1 = int(int64_t(units) * (piece + 1) / pieces) * unit;
  const int g0 = d0 / gdw;
  const uint32_t* wrow = W + size_t(nr) * row_dw;
  const size_t srow = size_t(nr) * num_scales;
  const bool split = gridDim.y > 1;

  for (int mt0 = 0; mt0 < M; mt0 += MT) {
    float acc[MT], part[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = part[i] = 0.f;
    // activation row of pass slot i (rows past M repeat row M - 1; not stored)
    // (32-bit element offsets, M K < 2^31: half the scalar registers)
    uint32_t xrow[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) xrow[i] = uint32_t(min(mt0 + i, M - 1)) * uint32_t(K);
    // A block is kDepth dwords of each lane's row; the next block's weights
    // and the scales of the groups that end in it are loaded while this one
    // is computed (a scale loaded at the group's end would wait for every
    // load before it).  sc[j]: the scale of the group ending with dword j.
    uint32_t cur[kDepth], nxt[kDepth];
    float sc[kDepth], sn[kDepth];
    int pg = g0, pleft = gdw;   // group and dwords left in it at the fetch cursor
    auto fetch = [&](int ds, uint32_t (&wv)[kDepth], float (&sv)[kDepth]) {
      if (ds + kDepth <= row_dw) {
        const uint32_t* p = wrow + ds;
        if constexpr (VEC) {
          const u32x4_t a = *reinterpret_cast<const u32x4_t*>(p);
          const u32x4_t b = *reinterpret_cast<const u32x4_t*>(p + 4);
          wv[0] = a.x; wv[1] = a.y; wv[2] = a.z; wv[3] = a.w;
          wv[4] = b.x; wv[5] = b.y; wv[6] = b.z; wv[7] = b.w;
        } else {
#pragma unroll
          for (int j = 0; j < kDepth; ++j) wv[j] = p[j];
        }
      } else {   // past the row's end: its last dword again (never used)
#pragma unroll
        for (int j = 0; j < kDepth; ++j) wv[j] = wrow[min(ds + j, row_dw - 1)];
      }
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        sv[j] = 0.f;
        if (ds + j < d1 && --pleft == 0) {
          sv[j] = load_f32_rt<kRT>(S, srow + pg, sd);
          ++pg;
          pleft = gdw;
        }
      }
    };
    fetch(d0, cur, sc);
    int left = gdw;                                      // dwords left in the current group
    for (int d = d0; d < d1; d += kDepth) {
      fetch(d + kDepth, nxt, sn);
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        if (d + j >= d1) break;
        float w[8];
        decode_dword<WBITS>(cur[j], w);
        uint32_t wp[4];   // (fp16 / bf16 activations) weight pairs
        if constexpr (XD != LQ_F32) {
#pragma unroll
          for (int e = 0; e < kWpd / 2; ++e) wp[e] = pack_pair<XD>(w[2 * e], w[2 * e + 1]);
        }
        const uint32_t k = uint32_t(d + j) * kWpd;
        // Activation rows in batches of kR scalar loads, double-buffered.
        // Scalar loads return out of order, so a use waits for every one in
        // flight: each batch is waited for before the next goes out, and
        // that one's latency then runs under this one's FMAs.
        // (fp32: kWpd floats per row; fp16 / bf16: kWpd / 2 raw pairs)
        constexpr int kXW = XD == LQ_F32 ? kWpd : kWpd / 2;
        uint32_t xv[2][kR][kXW];
        auto load_row = [&](int i, uint32_t (&v)[kXW]) {
          const uint32_t* p = reinterpret_cast<const uint32_t*>(
              static_cast<const uint8_t*>(X) + size_t(xrow[i] + k) * (XD == LQ_F32 ? 4 : 2));
#pragma unroll
          for (int e = 0; e < kXW; ++e) v[e] = p[e];
        };
#pragma unroll
        for (int r = 0; r < kR; ++r) load_row(r, xv[0][r]);
#pragma unroll
        for (int i0 = 0; i0 < MT; i0 += kR) {
          const int b = (i0 / kR) & 1;
          __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): batch b is in
          if (i0 + kR < MT) {
#pragma unroll
            for (int r = 0; r < kR; ++r) load_row(i0 + kR + r, xv[b ^ 1][r]);
          }
#pragma unroll
          for (int r = 0; r < kR; ++r) {
            float a = part[i0 + r];
#pragma unroll
            for (int e = 0; e < kXW; ++e) {
              if constexpr (XD == LQ_F32) a = fmaf(__uint_as_float(xv[b][r][e]), w[e], a);
              else a = dot2<XD>(xv[b][r][e], wp[e], a);
            }
            part[i0 + r] = a;
          }
        }
        if (--left == 0) {   // a group ends: scale its sums
#pragma unroll
          for (int i = 0; i < MT; ++i) {
            acc[i] = fmaf(sc[j], part[i], acc[i]);
            part[i] = 0.f;
          }
          left = gdw;
        }
      }
#pragma unroll
      for (int j = 0; j < kDepth; ++j) {
        cur[j] = nxt[j];
        sc[j] = sn[j];
      }
    }
    // waves -> LDS -> wave w sums pass slots w, w + 4, ...
#pragma unroll
    for (int i = 0; i < MT; ++i) red[wave][i][lane] = acc[i];
    __syncthreads();
    for (int i = wave; i < MT; i += kGWaves) {
      float v = red[0][i][lane];
#pragma unroll
      for (int w2 = 1; w2 < kGWaves; ++w2) v += red[w2][i][lane];
      const int m = mt0 + i;
      if (split) {
        if (m < M && n < N) P[(size_t(blockIdx.y) * M + m) * N + n] = v;
      } else if constexpr (EPI) {
        // rows 2i (gate) and 2i + 1 (up) sit in lanes l and l ^ 1
        const float up = __shfl_xor(v, 1, 64);
        if ((lane & 1) == 0 && m < M && n < N)
          store_out<kRT>(O, size_t(m) * (N / 2) + n / 2, v / (1.0f + expf(-v)) * up, od);
      } else {
        if (m < M && n < N) store_out<kRT>(O, size_t(m) * N + n, v, od);
      }
    }
    __syncthreads();   // red is rewritten by the next pass
  }
}

// Decode rows (M <= 4): lane l of a wave walks dword l of every 64-dword
// segment of each of the wave's RW weight rows (one coalesced 256-byte load
// per row and segment), so a lane's 8 (int4) / 4 (int8) weights lie in one
// scale group (G % 8 / % 4) and its partial sum is scaled at once; the next
// SB segments' weights, scales and activations load while these compute;
// the lanes are summed at the end (a butterfly per output).
template <int WBITS, int XD, int M_, int RW, int SB, bool EPI>
__global__ __launch_bounds__(256) void group_rows_kernel(
    const void* __restrict__ X, const uint32_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd, int od) {
  constexpr int kWpd = WBITS == 4 ? 8 : 4;
  constexpr int kXW = XD == LQ_F32 ? kWpd : kWpd / 2;   // activation dwords per lane and row
  static_assert(!EPI || RW % 2 == 0, "gate / up pairs within one wave");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n0 = (blockIdx.x * 4 + wave) * RW;
  const int row_dw = K / kWpd;
  const int nseg = (row_dw + 63) / 64;
  const int xb = XD == LQ_F32 ? 4 : 2;

  // SB segments per step (RW x SB weight loads in flight per wave)
  struct Seg {
    uint32_t w[SB][RW];
    Bits16 s[SB][RW];
    uint32_t x[SB][M_][kXW];
  };
  auto fetch = [&](Seg& g, int c0) {
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      // (lanes past the row: its last dword, not used)
      const int d = min((c0 + j) * 64 + lane, row_dw - 1);
      const int gi = int(uint32_t(d) * kWpd / uint32_t(group));
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int n = min(n0 + r, N - 1);
        g.w[j][r] = W[size_t(n) * row_dw + d];
        g.s[j][r] = load_bits16(S, size_t(n) * num_scales + gi, sd);
      }
#pragma unroll
      for (int m = 0; m < M_; ++m) {
        const uint32_t* p = reinterpret_cast<const uint32_t*>(
            static_cast<const uint8_t*>(X) + (size_t(m < M ? m : 0) * K + size_t(d) * kWpd) * xb);
#pragma unroll
        for (int e = 0; e < kXW; ++e) g.x[j][m][e] = p[e];
      }
    }
  };
  float acc[M_][RW];
#pragma unroll
  for (int m = 0; m < M_; ++m)
#pragma unroll
    for (int r = 0; r < RW; ++r) acc[m][r] = 0.f;
  Seg cur, nxt;
  fetch(cur, 0);
  for (int c = 0; c < nseg; c += SB) {
    if (c + SB < nseg) fetch(nxt, c + SB);
#pragma unroll
    for (int j = 0; j < SB; ++j) {
      const bool valid = (c + j) * 64 + lane < row_dw;
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        float w[8];
        decode_dword<WBITS>(cur.w[j][r], w);
        uint32_t wp[4];
        if constexpr (XD != LQ_F32) {
#pragma unroll
          for (int e = 0; e < kWpd / 2; ++e) wp[e] = pack_pair<XD>(w[2 * e], w[2 * e + 1]);
        }
        const float sc = valid ? bits16_to_f32(cur.s[j][r], sd) : 0.f;
#pragma unroll
        for (int m = 0; m < M_; ++m) {
          float a = 0.f;
#pragma unroll
          for (int e = 0; e < kXW; ++e) {
            if constexpr (XD == LQ_F32) a = fmaf(__uint_as_float(cur.x[j][m][e]), w[e], a);
            else a = dot2<XD>(cur.x[j][m][e], wp[e], a);
          }
          acc[m][r] = fmaf(a, sc, acc[m][r]);
        }
      }
    }
    cur = nxt;
  }
#pragma unroll
  for (int m = 0; m < M_; ++m) {
    float v[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      v[r] = acc[m][r];
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) v[r] += __shfl_xor(v[r], off, 64);
    }
    if (lane != 0 || m >= M) continue;
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = n0 + r;
      if constexpr (EPI) {
        if ((r & 1) == 0 && n + 1 < N)
          store_out<kRT>(O, size_t(m) * (N / 2) + n / 2, v[r] / (1.0f + expf(-v[r])) * v[r + 1], od);
      } else {
        if (n < N) store_out<kRT>(O, size_t(m) * N + n, v[r], od);
      }
    }
  }
}

template <int WBITS, int XD, int M_, bool EPI>
static void launch_group_rows_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                                int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  constexpr int kRW = 4;
  constexpr int kSB = 4 / M_;   // (the activations of M_ rows x SB segments in registers)
  hipLaunchKernelGGL((group_rows_kernel<WBITS, XD, M_, kRW, kSB, EPI>),
                     dim3(unsigned((N + 4 * kRW - 1) / (4 * kRW))), dim3(256), 0, st, X,
                     static_cast<const uint32_t*>(W), S, O, int(M), int(N), int(K), int(K / G),
                     int(G), sd, od);
}

template <int WBITS, int XD, bool EPI>
static void launch_group_rows(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  if (M <= 1) launch_group_rows_t<WBITS, XD, 1, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
  else if (M <= 2) launch_group_rows_t<WBITS, XD, 2, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
  else launch_group_rows_t<WBITS, XD, 4, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
}

template <int WBITS, int XD, bool EPI, bool VEC>
static void launch_group_mt(const void* X, const void* W, const void* S, void* O, float* P,
                            int64_t M, int64_t N, int64_t K, int64_t G, int unit, int splits,
                            int sd, int od, hipStream_t st) {
  const dim3 grid(unsigned((N + 63) / 64), unsigned(splits));
#define LQ_GV(MT_)                                                                              \
  hipLaunchKernelGGL((group_valu_kernel<WBITS, XD, MT_, EPI, VEC>), grid, dim3(64 * kGWaves), 0, \
                     st, X, static_cast<const uint32_t*>(W), S, O, P, int(M), int(N), int(K),    \
                     int(K / G), int(G), unit, sd, od)
  if (M <= 1) LQ_GV(1);
  else if (M <= 2) LQ_GV(2);
  else if (M <= 4) LQ_GV(4);
  else if (M <= 8) LQ_GV(8);
  else LQ_GV(16);
#undef LQ_GV
}

// Shapes: G % (weights per dword) == 0, X 4-byte aligned, W 4-byte aligned,
// sizes within 32-bit indexing.  `fixed`: scratch for the k-split partials
// (nullptr: the stream's workspace; without either the kernel runs
// unsplit).  LQ_ERR_SHAPE when it does not apply.
template <int WBITS, bool EPI>
int launch_group_valu(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                      int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st,
                      const FixedScratch* fixed) {
  constexpr int64_t kWpd = WBITS == 4 ? 8 : 4;
  if (G % kWpd != 0 || K % G != 0 || (EPI && N % 2 != 0)) return LQ_ERR_SHAPE;
  const int64_t lim = int64_t(1) << 31;
  if (M * K >= lim || N * K >= lim || M * N >= lim) return LQ_ERR_SHAPE;
  if ((reinterpret_cast<uintptr_t>(X) & 3) || (reinterpret_cast<uintptr_t>(W) & 3))
    return LQ_ERR_SHAPE;
  // k split over workgroups until about two workgroups per CU, each wave
  // keeping at least 4 groups
  if (M <= 4) {   // decode rows: lanes along k
#define LQ_GR(XD_) launch_group_rows<WBITS, XD_, EPI>(X, W, S, O, M, N, K, G, sd, od, st)
    if (xd == LQ_F32) LQ_GR(LQ_F32);
    else if (xd == LQ_F16) LQ_GR(LQ_F16);
    else LQ_GR(LQ_BF16);
#undef LQ_GR
    return check_launch();
  }
  // run units: whole groups, and whole 8-dword blocks when the rows allow
  // 16-byte loads
  const int64_t row_dw = K / kWpd, gdw = G / kWpd;
  int64_t unit = gdw;
  while (unit % 8 != 0) unit += gdw;
  const bool vec = row_dw % unit == 0 && (reinterpret_cast<uintptr_t>(W) & 15) == 0;
  if (!vec) unit = gdw;
  const int64_t blocks = (N + 63) / 64;
  const int64_t units = row_dw / unit;
  // k split over workgroups until about two workgroups per CU, every wave
  // keeping at least 2 units and 16 dwords (more splits measured slower:
  // 4096 x 4096 G = 16, M = 1 11.5 -> 13.6 us at four workgroups per CU)
  int splits = 1;
  while (splits < 16 && blocks * splits < 512 && units >= int64_t(splits) * 4 * kGWaves &&
         row_dw >= int64_t(splits) * 32 * kGWaves)
    splits *= 2;
  float* P = nullptr;
  if (splits > 1) {
    const size_t bytes = size_t(splits) * size_t(M) * size_t(N) * sizeof(float);
    void* ws = fixed ? (bytes <= fixed->bytes ? fixed->p : nullptr)
                     : (bytes <= (size_t(256) << 20) ? stream_workspace(0, bytes, st) : nullptr);
    if (ws == nullptr) splits = 1;
    P = static_cast<float*>(ws);
  }
#define LQ_GX(XD_)                                                                             \
  (vec ? launch_group_mt<WBITS, XD_, EPI, true>(X, W, S, O, P, M, N, K, G, int(unit), splits, sd, od, st) \
       : launch_group_mt<WBITS, XD_, EPI, false>(X, W, S, O, P, M, N, K, G, int(unit), splits, sd, od, st))
  if (xd == LQ_F32) LQ_GX(LQ_F32);
  else if (xd == LQ_F16) LQ_GX(LQ_F16);
  else LQ_GX(LQ_BF16);
#undef LQ_GX
  int rc = check_launch();
  if (rc != LQ_OK || splits == 1) return rc;
  return launch_split_reduce(P, O, M, N, splits, EPI, od, st);
}

template int launch_group_valu<4, false>(const void*, const void*, const void*, void*, int64_t,
                                         int64_t, int64_t, int64_t, int, int, int, hipStream_t,
                                         const FixedScratch*);
template int launch_group_valu<8, false>(const void*, const void*, const void*, void*, int64_t,
                                         int64_t, int64_t, int64_t, int, int, int, hipStream_t,
                                         const FixedScratch*);
template int launch_group_valu<4, true>(const void*, const void*, const void*, void*, int64_t,
                                        int64_t, int64_t, int64_t, int, int, int, hipStream_t,
                                        const FixedScratch*);

}  // namespace lq
