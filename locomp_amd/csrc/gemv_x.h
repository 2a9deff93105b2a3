// Decode (M <= 16) dequant-matmul for bf16 and fp32 activations: the LDS-ring
// tile kernel of gemv_impl.h instantiated with bf16 MFMAs (TileMfma<WBITS,
// LQ_BF16 / LQ_F32>), scale and output dtypes taken at run time.
#pragma once
#include "gemv_impl.h"

namespace lq {

void* stream_workspace(int slot, size_t bytes, hipStream_t st);

// fp32 activations X [M, K] -> their bf16 parts, P bf16 with row m * mstride
// + pstride * part = part `part` of row m: NPARTS = 3, the exact three-way
// split (the tile kernel's 12 part rows at M <= 4: mstride 1, pstride 4; rows
// of m >= M are not written and not read); NPARTS = 2, the round-to-nearest
// two-way split (rows 2m, 2m + 1: mstride 2, pstride 1).  Thread i takes 8
// consecutive k of one row.
template <int NPARTS>
static __global__ __launch_bounds__(256) void split_f32_parts_kernel(const float* __restrict__ X,
                                                             uint16_t* __restrict__ P, int M,
                                                             int K, int mstride, int pstride) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  const int per_row = K >> 3;
  if (i >= M * per_row) return;
  const int m = i / per_row, k = (i - m * per_row) * 8;
  const u32x4_t a = *reinterpret_cast<const u32x4_t*>(X + size_t(m) * K + k);
  const u32x4_t b = *reinterpret_cast<const u32x4_t*>(X + size_t(m) * K + k + 4);
  const uint32_t x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
  for (int p = 0; p < NPARTS; ++p) {
    uint32_t h[8];
#pragma unroll
    for (int e = 0; e < 8; ++e)
      h[e] = (NPARTS == 3 ? f32_part_bits(x[e], p) : f32_rn2_part_bits(x[e], p)) >> 16;
    const u32x4_t v = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                       h[6] | (h[7] << 16)};
    *reinterpret_cast<u32x4_t*>(P + (size_t(m) * mstride + size_t(pstride) * p) * K + k) = v;
  }
}

template <int WBITS, int XD, int NSC, bool EPI = false>
static void launch_tile_x_nsc(const void* X, const void* W, const void* S, void* O, int64_t M,
                              int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  // fp32 activations hold twice the registers per batch: at most 2 tiles
  // (3 and 4 spill)
  int tiles = gemv_tile_count(N, K, G, sd == LQ_F32 ? 4 : 2);
  if (XD == LQ_F32 && tiles > 2) tiles = 2;
  // (the pre-split parts are bf16 rows: any tile count)
  const unsigned blocks = unsigned((N + 16 * tiles - 1) / (16 * tiles));
  const bool part = ((WBITS == 4 ? K / 2 : K) % kTChunkB) != 0;
#define LQ_TX_LAUNCH(T_)                                                                        \
  do {                                                                                          \
    if (part)                                                                                   \
      hipLaunchKernelGGL((gemv_tile_kernel<WBITS, NSC, T_, kRT, kRT, true, EPI, XD>),           \
                         dim3(blocks), dim3(512), 0, st, X, static_cast<const uint8_t*>(W), S, \
                         O, int(M), int(N), int(K), int(K / G), int(G), sd, od);                \
    else                                                                                        \
      hipLaunchKernelGGL((gemv_tile_kernel<WBITS, NSC, T_, kRT, kRT, false, EPI, XD>),          \
                         dim3(blocks), dim3(512), 0, st, X, static_cast<const uint8_t*>(W), S, \
                         O, int(M), int(N), int(K), int(K / G), int(G), sd, od);                \
  } while (0)
  if constexpr (XD == LQ_F32) {
    if (tiles == 1) LQ_TX_LAUNCH(1);
    else LQ_TX_LAUNCH(2);
  } else {
    switch (tiles) {
      case 1: LQ_TX_LAUNCH(1); break;
      case 2: LQ_TX_LAUNCH(2); break;
      case 3: LQ_TX_LAUNCH(3); break;
      default: LQ_TX_LAUNCH(4); break;
    }
  }
#undef LQ_TX_LAUNCH
}

template <int NSEG, int RW, int XD>
static void launch_seg_x_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                           int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  const unsigned blocks = unsigned((N + 4 * RW - 1) / (4 * RW));
  if (K % 2048)
    hipLaunchKernelGGL((gemv_seg_kernel<1, NSEG, RW, kRT, kRT, true, XD>), dim3(blocks), dim3(256), 0,
                       st, X, static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),
                       int(K / G), int(G), sd, od);
  else
    hipLaunchKernelGGL((gemv_seg_kernel<1, NSEG, RW, kRT, kRT, false, XD>), dim3(blocks), dim3(256), 0,
                       st, X, static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K),
                       int(K / G), int(G), sd, od);
}

// M = 1, int4, G % 128: the 2048-k segment kernel (bf16 up to 8 segments,
// fp32 - three operand sets per segment - up to 2, 3 at N <= 4096);
// LQ_ERR_SHAPE otherwise.
static int launch_seg_x(const void* X, const void* W, const void* S, void* O, int64_t M,
                        int64_t N, int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  if (M != 1 || !gemv_seg_ok(4, 1, N, K, G)) return LQ_ERR_SHAPE;
  if (xd == LQ_BF16) {
    if (nseg == 1) launch_seg_x_t<1, 8, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
    else if (nseg == 2) launch_seg_x_t<2, 4, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
    // 3 and 6 segments as such (not padded to 4 / 8), 2 rows per wave from
    // 3 segments (4096 x 6144 5.8 -> 4.9 us, 4096 x 11008 12.2 -> 7.8,
    // 11008 x 11008 28.5 -> 18.5, 4096 x 14336 12.5 -> 10.6)
    else if (nseg == 3) launch_seg_x_t<3, 2, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
    else if (nseg == 4) launch_seg_x_t<4, 2, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
    else if (nseg <= 6) launch_seg_x_t<6, 2, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
    else launch_seg_x_t<8, 2, LQ_BF16>(X, W, S, O, M, N, K, G, sd, od, st);
  } else {
    if (nseg == 1) launch_seg_x_t<1, 8, LQ_F32>(X, W, S, O, M, N, K, G, sd, od, st);
    else if (nseg == 2) launch_seg_x_t<2, 4, LQ_F32>(X, W, S, O, M, N, K, G, sd, od, st);
    // 3 segments (200 VGPRs at 2 rows per wave) up to N = 4096 (4096 x 6144
    // 9.5 -> 7.3 us against the pre-split ring; at N = 11008 the ring wins,
    // 14.0 against 16.1; 4 segments spill or lose)
    else if (nseg == 3 && N <= 4096) launch_seg_x_t<3, 2, LQ_F32>(X, W, S, O, M, N, K, G, sd, od, st);
    else return LQ_ERR_SHAPE;
  }
  return check_launch();
}

// The row kernel (int4, G % 32) with bf16 (M <= 2) or fp32 (M = 1, K <= 4096)
// activations, scale / output dtypes at run time; segment counts and rows
// per wave as for fp16.
template <int M_, int XD, bool EPI = false>
static int launch_rows_x_m(const void* X, const void* W, const void* S, void* O, int64_t M,
                           int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  const int64_t nseg = (K + 2047) / 2048;
  constexpr int kSmallRW = EPI ? 2 : 1;   // (gate / up pairs stay in one wave)
  if (nseg <= 2 && N <= 3072) {
    if (nseg <= 1) return launch_gemv_rows_t<M_, 1, kSmallRW, kRT, kRT, EPI, 3, XD>(X, W, S, O, M, N, K, G, st, sd, od);
    return launch_gemv_rows_t<M_, 2, kSmallRW, kRT, kRT, EPI, 3, XD>(X, W, S, O, M, N, K, G, st, sd, od);
  }
  if (nseg <= 1) return launch_gemv_rows_t<M_, 1, 4, kRT, kRT, EPI, 3, XD>(X, W, S, O, M, N, K, G, st, sd, od);
  if (nseg <= 2)
    return launch_gemv_rows_t<M_, 2, 4, kRT, kRT, EPI, (M_ == 2 || XD == LQ_F32) ? 2 : 3, XD>(
        X, W, S, O, M, N, K, G, st, sd, od);
  if constexpr (M_ == 1 && XD != LQ_F32) {
    if (nseg == 3) return launch_gemv_rows_t<M_, 3, 2, kRT, kRT, EPI, 3, XD>(X, W, S, O, M, N, K, G, st, sd, od);
    if (nseg == 4) return launch_gemv_rows_t<M_, 4, 2, kRT, kRT, EPI, 3, XD>(X, W, S, O, M, N, K, G, st, sd, od);
    if (nseg <= 6) return launch_gemv_rows_t<M_, 6, 2, kRT, kRT, EPI, 2, XD>(X, W, S, O, M, N, K, G, st, sd, od);
    return launch_gemv_rows_t<M_, 8, 2, kRT, kRT, EPI, 2, XD>(X, W, S, O, M, N, K, G, st, sd, od);
  }
  return LQ_ERR_SHAPE;
}

// The row kernel with bf16 (M <= 2) or fp32 (M = 1, K <= 4096) activations
// (fp16 too, for bf16 scales / outputs: then with kRT dtypes); EPI: the
// gate / up SiLU * mul epilogue, O [M, N / 2].  LQ_ERR_SHAPE where it does
// not apply.
template <bool EPI = false>
static int launch_rows_x(const void* X, const void* W, const void* S, void* O, int64_t M,
                         int64_t N, int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st) {
  // bf16 3 <= M <= 4 on one segment (K <= 2048) where the tile kernel does
  // not apply (short rows: SmolLM2 at batch 4), four activation rows per
  // lane: 576 x 576 4.2 -> 3.9 us against the generic kernel (fp32 lost
  // there, 4.1 -> 4.9, and keeps the generic kernel)
  if (xd == LQ_BF16 && M >= 3 && M <= 4 && K <= 2048 && K % 32 == 0 && G % 32 == 0 && !EPI &&
      !gemv_tile_ok(4, M, N, K, G, sd == LQ_F32 ? 4 : 2))
    return launch_gemv_rows_t<4, 1, 1, kRT, kRT, false, 2, LQ_BF16>(X, W, S, O, M, N, K, G, st, sd, od);
  if (M > (xd == LQ_F32 ? 1 : 2) || !gemv_rows_ok(4, M, K, G) || (xd == LQ_F32 && K > 4096))
    return LQ_ERR_SHAPE;
  if (EPI && N % 2 != 0) return LQ_ERR_SHAPE;
  if (xd == LQ_F32) return launch_rows_x_m<1, LQ_F32, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
  if (xd == LQ_BF16) {
    if (M == 1) return launch_rows_x_m<1, LQ_BF16, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
    return launch_rows_x_m<2, LQ_BF16, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
  }
  if constexpr (EPI) {
    if (M == 1) return launch_rows_x_m<1, LQ_F16, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
    return launch_rows_x_m<2, LQ_F16, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
  }
  return LQ_ERR_SHAPE;
}

// bf16 activations at 16 < M <= 64 (int8 also 8 < M <= 16 with whole-chunk
// groups, as for fp16) on the activation-in-LDS kernel with bf16 MFMAs;
// LQ_ERR_SHAPE where it does not apply.
// bf16 rows on the decode kernels: the LDS-ring tile kernel (M <= 16) or
// the activation-in-LDS kernel (16 < M <= 64).  XD = LQ_BF16 (activations)
// or kXPairs (M bf16 part rows of M / 2 fp32 rows, pairs added at the
// store); EPI: gate/up rows interleaved, silu(gate) * up stored.
// LQ_ERR_SHAPE for shapes those kernels do not take.
template <int WBITS, int XD, bool EPI>
int launch_tile_rows_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                       int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  const int ssz = sd == LQ_F32 ? 4 : 2;
  if (M <= 16) {
    if (!gemv_tile_ok(WBITS, M, N, K, G, ssz)) return LQ_ERR_SHAPE;
    const int64_t eighth_k = kTBlocks * TileMfma<WBITS>::kSpan;
    const int nsc = G >= eighth_k ? 1 : int(eighth_k / G);
    if (nsc == 1) launch_tile_x_nsc<WBITS, XD, 1, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
    else if (nsc == 2) launch_tile_x_nsc<WBITS, XD, 2, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
    else launch_tile_x_nsc<WBITS, XD, 4, EPI>(X, W, S, O, M, N, K, G, sd, od, st);
    return check_launch();
  }
  if (M > 64 || !gemv_tile_xl_ok(WBITS, M, N, K, G, ssz)) return LQ_ERR_SHAPE;
  if (xl_mtiles(M) <= 2)
    launch_gemv_tile_xl_mt<WBITS, kRT, kRT, EPI, 2, XD>(X, W, S, O, M, N, K, G, st, sd, od);
  else
    launch_gemv_tile_xl_mt<WBITS, kRT, kRT, EPI, 4, XD>(X, W, S, O, M, N, K, G, st, sd, od);
  return check_launch();
}

// bf16 activations, 16 < M <= 64.
template <int WBITS>
int launch_tile_xl_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                     int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  if (M <= 16) return LQ_ERR_SHAPE;
  return launch_tile_rows_x<WBITS, LQ_BF16, false>(X, W, S, O, M, N, K, G, sd, od, st);
}

// bf16 activations at M <= 16, fp32 at M <= 4 (three MFMA rows per
// activation row), on the shapes gemv_tile_ok accepts; LQ_ERR_SHAPE otherwise.
// int4 M = 1 with G % 128 takes the segment kernel.  fp32 activations are
// first split into bf16 part rows (split_f32_parts_kernel) in `fixed` or the
// stream's workspace slot 2, so the tile kernel streams bf16 operands; with
// neither available (a capturing stream before any such call) the tile
// kernel splits them itself, at fewer tiles per workgroup.
template <int WBITS>
int launch_skinny_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                    int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st,
                    const FixedScratch* fixed) {
  if (xd != LQ_BF16 && xd != LQ_F32) return LQ_ERR_SHAPE;
  if constexpr (WBITS == 4) {
    const int rc = launch_seg_x(X, W, S, O, M, N, K, G, xd, sd, od, st);
    if (rc != LQ_ERR_SHAPE) return rc;
    // the row kernel for what the segment kernel leaves at M <= 2 (fp32:
    // M = 1, K <= 4096), as for fp16: rows the tile kernel does not take
    // (SmolLM2 576 x 1536 G = 32: 6.8 -> 2.7 us bf16, 7.0 -> 3.7 fp32, on
    // the generic kernel before) and faster than it where it does (4096 x
    // 4096 G = 32: bf16 7.8 -> 5.6, M = 2 7.9 -> 6.9, fp32 9.8 -> 8.2)
    const int rr = launch_rows_x(X, W, S, O, M, N, K, G, xd, sd, od, st);
    if (rr != LQ_ERR_SHAPE) return rr;
  }
  if (xd == LQ_F32 ? M > 4 : M > 16) return LQ_ERR_SHAPE;
  if (!gemv_tile_ok(WBITS, M, N, K, G, sd == LQ_F32 ? 4 : 2)) return LQ_ERR_SHAPE;
  const int64_t eighth_k = kTBlocks * TileMfma<WBITS>::kSpan;
  const int nsc = G >= eighth_k ? 1 : int(eighth_k / G);
#define LQ_NSC(XD_)                                                                         \
  switch (nsc) {                                                                            \
    case 1: launch_tile_x_nsc<WBITS, XD_, 1>(X, W, S, O, M, N, K, G, sd, od, st); break;    \
    case 2: launch_tile_x_nsc<WBITS, XD_, 2>(X, W, S, O, M, N, K, G, sd, od, st); break;    \
    default: launch_tile_x_nsc<WBITS, XD_, 4>(X, W, S, O, M, N, K, G, sd, od, st); break;   \
  }
  void* parts = nullptr;
  // (small matrices: the tile kernel splits the activations itself, one
  // launch instead of two; its smaller tile count costs nothing there)
  if (xd == LQ_F32 && N * K >= (int64_t(1) << 22)) {
    const size_t bytes = size_t(12) * size_t(K) * 2;
    parts = fixed ? (bytes <= fixed->bytes ? fixed->p : nullptr) : stream_workspace(2, bytes, st);
  }
  if (parts) {
    const int threads = int(M * (K / 8));
    hipLaunchKernelGGL(split_f32_parts_kernel<3>, dim3((threads + 255) / 256), dim3(256), 0, st,
                       static_cast<const float*>(X), static_cast<uint16_t*>(parts), int(M), int(K), 1, 4);
    X = parts;
    LQ_NSC(kXPre)
  } else if (xd == LQ_BF16) {
    LQ_NSC(LQ_BF16)
  } else {
    LQ_NSC(LQ_F32)
  }
#undef LQ_NSC
  return check_launch();
}

}  // namespace lq
