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
//
// The kernels live in gemv_skinny.h, gemv_rows.h, gemv_diag.h, gemv_seg.h
// and gemv_tile.h (MFMA operand traits in gemv_traits.h); this file holds
// their launchers and the kernel choice.
#include "gemv_skinny.h"
#include "gemv_rows.h"
#include "gemv_diag.h"
#include "gemv_seg.h"
#include "gemv_tile.h"

namespace lq {

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


template <int M_, int NSEG, int RW, int SD, int OD, bool EPI = false, int OCC = 3, int XD = LQ_F16>
static int launch_gemv_rows_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st, int sd_rt = 0,
                              int od_rt = 0) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  hipLaunchKernelGGL((gemv_rows_kernel<M_, NSEG, RW, SD, OD, EPI, OCC, XD>), dim3(blocks), dim3(256), 0,
                     st, X, static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K), int(K / G),
                     int(G), sd_rt, od_rt);
  return check_launch();
}

template <int M_, int SD, int OD, bool EPI = false>
static int launch_gemv_rows_m(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  // Small matrices are latency bound: one row per wave (two for the gate / up
  // pairs) spreads them over 4x the workgroups (576 x 576: 2.8 -> 2.5 us; at
  // 4096 x 4096 four rows per wave stay faster).
  constexpr int kSmallRW = EPI ? 2 : 1;
  if (nseg <= 2 && N <= 3072) {
    if (nseg <= 1) return launch_gemv_rows_t<M_, 1, kSmallRW, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
    return launch_gemv_rows_t<M_, 2, kSmallRW, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  }
  if (nseg <= 1) return launch_gemv_rows_t<M_, 1, 4, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  // (two activation rows x 2 segments: 210 VGPRs, sized for 2 workgroups per CU)
  if (nseg <= 2) return launch_gemv_rows_t<M_, 2, 4, SD, OD, EPI, M_ == 2 ? 2 : 3>(X, W, S, O, M, N, K, G, st);
  // M = 1 runs 3 and 6 segments as such instead of padding to 4 / 8 (G = 32:
  // 4096 x 6144 5.7 -> 4.8 us, 11008 x 6144 11.4 -> 9.0, 4096 x 11008
  // 9.9 -> 8.5, 11008 x 11008 21.7 -> 18.4)
  if constexpr (M_ == 1) {
    if (nseg == 3) {
      if (N >= 8192) return launch_gemv_rows_t<M_, 3, 4, SD, OD, EPI, 2>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_rows_t<M_, 3, 2, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
    }
  }
  // (M = 2 takes K <= 4096, two segments: the longer forms are M = 1 only)
  if constexpr (M_ == 1) {
    if (nseg <= 4) return launch_gemv_rows_t<M_, 4, 2, SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
    // 6 segments: 181 VGPRs, sized for 2 workgroups per CU (3 measured slower)
    if (nseg <= 6) return launch_gemv_rows_t<M_, 6, 2, SD, OD, EPI, 2>(X, W, S, O, M, N, K, G, st);
    // 8 segments (K <= 16384): 237 VGPRs, sized for 2 workgroups per CU
    return launch_gemv_rows_t<M_, 8, 2, SD, OD, EPI, 2>(X, W, S, O, M, N, K, G, st);
  }
  return LQ_ERR_SHAPE;
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
  // (the segment counts gemv_diag_ok admits: 2 up to M = 2, 8 at M = 1)
  if constexpr (M_ <= 2) {
    if (nseg <= 2) return launch_gemv_diag_t<M_, 2, rw2, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (M_ == 1) {
    if (nseg <= 4) return launch_gemv_diag_t<M_, 4, (rw2 > 1 ? rw2 / 2 : 1), SD, OD>(X, W, S, O, M, N, K, G, st);
    return launch_gemv_diag_t<M_, 8, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  return LQ_ERR_SHAPE;
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
  if constexpr (M_ == 1) {
    // M = 1 runs 3 and 6 segments as such instead of padding to 4 / 8 (the
    // padded segments' MFMAs and activation registers cost as much as real
    // ones): 4096 x 6144 5.2 -> 4.7 us, 4096 x 11008 9.7 -> 7.3, 8192 x
    // 11008 17.5 -> 11.8.  Two rows per wave from N = 4096 (4 at 3 segments
    // from N = 8192) halve the workgroups, each of which builds the whole
    // activation row (4096 x 14336: 10.1 -> 8.5 us).
    if (nseg == 3) {
      if (N >= 8192) return launch_gemv_seg_t<M_, 3, 4, SD, OD>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_seg_t<M_, 3, 2, SD, OD>(X, W, S, O, M, N, K, G, st);
    }
  }
  if constexpr (M_ <= 2) {
    if (nseg <= 4) return launch_gemv_seg_t<M_, 4, (rw > 2 ? rw / 2 : 1), SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (M_ == 1) {
    if (nseg <= 6) {
      if (N >= 4096) return launch_gemv_seg_t<M_, 6, 2, SD, OD>(X, W, S, O, M, N, K, G, st);
      return launch_gemv_seg_t<M_, 6, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
    }
    if (N >= 4096) return launch_gemv_seg_t<M_, 8, 2, SD, OD>(X, W, S, O, M, N, K, G, st);
    return launch_gemv_seg_t<M_, 8, 1, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  return LQ_ERR_SHAPE;   // excluded by gemv_seg_ok
}

// The segment kernel: int4, M <= 4, G % 128 == 0, 2048 <= K <= 16384
// (K / 2048 rounded up to 1, 2, 4 or 8 segments, at M = 1 also 3 or 6; the
// last possibly partial),
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
  return M >= 1 && M <= 16 && K < (int64_t(1) << 22) && row_bytes >= kTChunkB &&
         row_bytes % 16 == 0 && groups_ok &&
         (row_bytes % kTChunkB == 0 || row_bytes >= 4 * kTChunkB) &&
         N * row_bytes < (int64_t(1) << 31) &&
         (N * (K / G) * scale_bytes) % 4 == 0 && gemv_tile_count(N, K, G, scale_bytes) > 0;
}

// 16 < M <= 64 on the activation-in-LDS ring: K % 256, G % 32, fp16
// activations; T = 1..4 tiles so the grid is at most one workgroup per CU,
// while the workgroup's scale rows fit the LDS the ring leaves (which
// depends on the activation tile count mt) and the array is whole dwords.
static int gemv_tile_xl_count(int wbits, int64_t N, int64_t K, int64_t G, int scale_bytes,
                              int mt) {
  int tiles = 4;
  for (int t = 1; t <= 4; ++t)
    if ((N + 16 * t - 1) / (16 * t) <= 256) { tiles = t; break; }
  // int4 rows are 128 bytes per chunk: whole 1 KB DMA instructions need T even
  if (wbits == 4 && (tiles & 1)) ++tiles;
  while (tiles > 0 && 16 * tiles * (K / G) * scale_bytes > xl_scale_bytes(wbits, tiles, mt))
    tiles -= wbits == 4 ? 2 : 1;
  return tiles;
}
// activation tiles: 1 up to 16 rows (int8 only), 2 up to 32, else 4
static inline int xl_mtiles(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
static bool gemv_tile_xl_ok(int wbits, int64_t M, int64_t N, int64_t K, int64_t G, int scale_bytes) {
  return (M > 16 || wbits == 8) && M >= 1 && M <= 64 && K % kXChunkK == 0 &&
         K < (int64_t(1) << 22) && G % 32 == 0 &&
         (N * (K / G) * scale_bytes) % 4 == 0 &&
         gemv_tile_xl_count(wbits, N, K, G, scale_bytes, xl_mtiles(M)) > 0;
}
template <int WBITS, int SD, int OD, bool EPI, int MT, int XD = LQ_F16>
static void launch_gemv_tile_xl_mt(const void* X, const void* W, const void* S, void* O, int64_t M,
                                   int64_t N, int64_t K, int64_t G, hipStream_t st, int sd_rt = 0,
                                   int od_rt = 0) {
  const int ssz = (SD == kRT ? sd_rt : SD) == LQ_F32 ? 4 : 2;
  const int tiles = gemv_tile_xl_count(WBITS, N, K, G, ssz, MT);
  const unsigned blocks = unsigned((N + 16 * tiles - 1) / (16 * tiles));
#define LQ_TX(T_)                                                                              \
  hipLaunchKernelGGL((gemv_tile_xl_kernel<WBITS, T_, SD, OD, EPI, MT, XD>), dim3(blocks), dim3(512), \
                     0, st, X, static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),   \
                     int(K / G), int(G), sd_rt, od_rt)
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
}
template <int WBITS, int SD, int OD, bool EPI = false>
static int launch_gemv_tile_xl(const void* X, const void* W, const void* S, void* O, int64_t M,
                               int64_t N, int64_t K, int64_t G, hipStream_t st) {
  const int mt = xl_mtiles(M);
  if constexpr (WBITS == 8) {
    if (mt == 1) {
      launch_gemv_tile_xl_mt<WBITS, SD, OD, EPI, 1>(X, W, S, O, M, N, K, G, st);
      return check_launch();
    }
  }
  if (mt <= 2) launch_gemv_tile_xl_mt<WBITS, SD, OD, EPI, 2>(X, W, S, O, M, N, K, G, st);
  else launch_gemv_tile_xl_mt<WBITS, SD, OD, EPI, 4>(X, W, S, O, M, N, K, G, st);
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
         K <= (M == 1 ? 16384 : 4096);
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
  if constexpr (kTileDt && WBITS == 8) {
    // int8, 8 < M <= 16, scale groups of whole 256-k chunks (per channel):
    // the activation-in-LDS kernel with one activation tile (its raw sums
    // span a group; 4096 x 4096 per channel M = 16: 8.9 against 10.7 us).
    // Smaller M or groups take the ring tile kernel below.
    if (M > 8 && G % kXChunkK == 0 && gemv_tile_xl_ok(WBITS, M, N, K, G, SD == LQ_F32 ? 4 : 2))
      return launch_gemv_tile_xl<WBITS, SD, OD>(X, W, S, O, M, N, K, G, st);
  }
  if constexpr (kTileDt) {
    // int4 M = 1 keeps the segment / row kernels up to K = 8192 (faster there);
    // longer rows stream better through the LDS ring.  int4 M = 2 also takes
    // the segment kernel for K >= 4096 (4096 x 4096: 4.7 against 6.0 us,
    // 11008 x 4096: 8.1 against 8.8; at K = 2048, and at M = 3, 4 with
    // N >= 11008, the ring wins).
    const bool seg2 = WBITS == 4 && M == 2 && K >= 4096 && gemv_seg_ok(WBITS, M, N, K, G);
    // int4 M = 1 with K > 8192: the segment kernel at up to 6 segments for
    // any N (4096 x 11008: 7.3 against 11.2 us, 11008 x 11008: 16.3 against
    // 17.2, 14336 x 11008: 19.7 against 20.4), at 7 or 8 segments up to
    // N = 8192 (4096 x 14336: 8.5 against 11.7), the ring beyond
    const bool seg1 = WBITS == 4 && M == 1 && K > 8192 && (N <= 8192 || K <= 6 * 2048) &&
                      gemv_seg_ok(WBITS, M, N, K, G);
    // int4 M = 1 with K > 8192 and groups the segment kernel cannot take
    // (G % 128 != 0): the row kernel at 8 segments (G = 32: 4096 x 11008 10.0
    // against 13.0 us, 11008 x 11008 21.7 against 31.3)
    const bool rows1 = WBITS == 4 && M == 1 && K > 8192 && G % 128 != 0 && gemv_rows_ok(WBITS, M, K, G);
    // int4 M = 2 with G % 128 != 0 and K <= 4096: the row kernel (G = 32:
    // 11008 x 4096 9.0 against 13.0 us, 4096 x 4096 5.0 against 7.1)
    const bool rows2 = WBITS == 4 && M == 2 && G % 128 != 0 && gemv_rows_ok(WBITS, M, K, G);
    // int4 M = 3, 4 with N <= 2048 and 2048 < K <= 4096: the segment kernel
    // (the ring has at most 128 one-tile workgroups there: 1024 x 4096 5.3
    // against 4.5 us, 2048 x 4096 5.4 against 4.5; at K = 2048 or N = 3072
    // the ring wins); fp16 scales / outputs only (its M = 4 instantiation)
    const bool seg34 = WBITS == 4 && SD != LQ_BF16 && OD != LQ_BF16 && (M == 3 || M == 4) &&
                       N <= 2048 && K > 2048 && K <= 4096 && gemv_seg_ok(WBITS, M, N, K, G);
    if (!seg2 && !seg1 && !rows1 && !rows2 && !seg34 && (M >= 2 || WBITS == 8 || K > 8192) &&
        gemv_tile_ok(WBITS, M, N, K, G, SD == LQ_F32 ? 4 : 2))
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
