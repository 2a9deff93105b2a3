// gemv_tile_kernel (2 <= M <= 16, LDS ring) and gemv_tile_xl_kernel (16 < M <= 64, activations in LDS).
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_traits.h"

namespace lq {

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
// m + 4 part holds part `part` of activation row m; kXPre: the same rows
// read as bf16 from a matrix of parts split beforehand; kXPairs: M bf16 part
// rows, pairs 2i, 2i + 1 added into output row i); SD / OD = kRT take
// the scale / output dtype from sd_rt / od_rt.
template <int WBITS, int NSC, int TILES, int SD, int OD, bool PART, bool EPI = false,
          int XD = LQ_F16>
__global__ __launch_bounds__(512, 1) void gemv_tile_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0) {
  constexpr bool kPre = XD == kXPre;                     // pre-split fp32: bf16 part rows
  constexpr bool kPairs = XD == kXPairs;                 // bf16 part rows 2i, 2i + 1
  typedef TileMfma<WBITS, (kPre || kPairs) ? LQ_BF16 : XD> Mf;
  typedef typename Mf::op_t op_t;
  typedef typename Mf::x_t x_t;
  const float rgroup = 1.0f / float(group);             // for div_rcp (K < 2^22)
  constexpr int kSpan = Mf::kSpan;                      // k per MFMA block
  constexpr int kEighthK = kTBlocks * kSpan;            // k per wave per chunk
  constexpr int kChunkK = kTWaves * kEighthK;
  constexpr int kPerScale = kTBlocks / NSC;             // blocks sharing one scale
  constexpr int kXB = XD == LQ_F32 ? 4 : 2;             // activation element bytes
  constexpr bool kSplit = XD == LQ_F32 || kPre;        // MFMA row m + 4 part
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
  // (pre-split: lane row r16 is row r16 of the part matrix)
  const uint8_t* xrow = static_cast<const uint8_t*>(X) +
                        (size_t(kPre ? r16 : min(xm, M - 1)) * K + wave * kEighthK + q4 * (kSpan / 4)) * kXB;
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
        int g = div_rcp(kbase + sg * kPerScale * kSpan, group, rgroup);
        if constexpr (PART) g = min(g, num_scales - 1);
        sc[t][sg] = load_scale<SD>(sl + (size_t(row) * num_scales + g) * kSSize, sd_rt);
      }
    }
    op_t xa[kTBlocks];
#pragma unroll
    for (int f = 0; f < kTBlocks; ++f) {
      xa[f] = Mf::prep_x(bt.x[f], kPre ? 0 : xpart);
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
      static_assert(!EPI, "three-part fp32 rows take the plain store");
      if (q4 == 0) {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (r < M && n < N) store_out<OD>(O, size_t(r) * N + n, v[r], od_rt);
      }
    } else if constexpr (kPairs) {
#pragma unroll
      for (int r = 0; r < 4; r += 2) {
        const int m = q4 * 4 + r;   // part rows m, m + 1: output row m / 2
        const float y = v[r] + v[r + 1];
        if constexpr (EPI) {
          const float up = __shfl_xor(y, 1, 64);
          if ((r16 & 1) == 0 && m < M && n < N)
            store_out<OD>(O, size_t(m >> 1) * (N / 2) + n / 2, y / (1.0f + expf(-y)) * up, od_rt);
        } else {
          if (m < M && n < N) store_out<OD>(O, size_t(m >> 1) * N + n, y, od_rt);
        }
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
// weight) tiles as one 16x16x32 block: int8 weights converted to fp16
// exactly, summed raw over the chunks of a scale group and scaled when the
// group changes; int4 with the 5-op biased decode, the bias one MFMA per
// activation tile shared by the T weight tiles, scaled every chunk.  The
// group scale (G % 32 == 0) is applied in fp32.  Workgroup b walks the
// chunks starting at chunk b mod (K / 256).
constexpr int kXChunkK = 256;
constexpr int kXSlots = 3;
// LDS of the ring (also the cross-wave sum) and of the scale rows: whatever
// the ring leaves of 160 KB, at most kTScaleLds.
constexpr int xl_ring_bytes(int wbits, int tiles, int mtiles) {
  const int slot = 16 * tiles * kXChunkK * wbits / 8 + 16 * mtiles * kXChunkK * 2;
  const int red = 8 * mtiles * tiles * 1024;
  return kXSlots * slot > red ? kXSlots * slot : red;
}
constexpr int xl_scale_bytes(int wbits, int tiles, int mtiles) {
  const int left = 160 * 1024 - xl_ring_bytes(wbits, tiles, mtiles);
  return (left > kTScaleLds ? kTScaleLds : left) & ~1023;
}

// EPI: gate/up rows interleaved; store silu(gate) * up to O [M, N / 2].
// MT: 16-row activation tiles (2 for M <= 32, else 4).  XD: fp16, bf16 or
// kXPairs (bf16 part rows, M of them; O holds M / 2 rows).
template <int WBITS, int TILES, int SD, int OD, bool EPI = false, int MT = 4, int XD = LQ_F16>
__global__ __launch_bounds__(512, 1) void gemv_tile_xl_kernel(
    const void* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int sd_rt = 0,
    int od_rt = 0) {
  static_assert(XD == LQ_F16 || XD == LQ_BF16 || XD == kXPairs, "fp16 or bf16 activations");
  constexpr bool kH = XD == LQ_F16;
  constexpr bool kPairs = XD == kXPairs;   // bf16 part rows 2i, 2i + 1 of fp32 rows
  typedef TileMfma<WBITS, kH ? LQ_F16 : LQ_BF16> Mf;
  typedef typename Mf::op_t op_t;
  const float rgroup = 1.0f / float(group);             // for div_rcp (K < 2^22)
  constexpr int kRows = 16 * TILES;
  constexpr int kRowB = kXChunkK * WBITS / 8;             // weight bytes per row per chunk
  constexpr int kPos = kRowB / 16;                        // 16-byte positions per weight row
  constexpr int kWBytes = kRows * kRowB;
  constexpr int kXBytes = 16 * MT * kXChunkK * 2;         // 16 MT activation rows, fp16
  constexpr int kSlotB = kWBytes + kXBytes;
  const int kSSize = SD == kRT ? (sd_rt == LQ_F32 ? 4 : 2) : (SD == LQ_F32 ? 4 : 2);
  constexpr int kWInstr = kWBytes / 1024;
  constexpr int kInstr = kWInstr + kXBytes / 1024;
  constexpr int kPerWaveMax = (kInstr + 7) / 8;
  static_assert(kWBytes % 1024 == 0, "whole weight DMA instructions");
  // the cross-wave sum reuses the ring (sized to hold it)
  constexpr int kRingB = xl_ring_bytes(WBITS, TILES, MT);
  static_assert(kRingB >= kXSlots * kSlotB, "ring holds the slots");
  constexpr int kSclB = xl_scale_bytes(WBITS, TILES, MT);
  static_assert(kRingB + kSclB <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) uint8_t ring[kRingB];
  __shared__ __attribute__((aligned(16))) uint8_t sl[kSclB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform (SGPR)
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
      src[i] = reinterpret_cast<const uint8_t*>(static_cast<const uint16_t*>(X) + size_t(m) * K) + (((lane & 31) ^ (row & 15)) << 4);
      dst[i] = kWBytes + (j - kWInstr) * 1024;
    }
  }
  // Step c works on chunk phys(c): workgroup b starts at chunk b mod nchunks,
  // so the workgroups do not all read the same column of their rows at once.
  const int rot = int(blockIdx.x % unsigned(nchunks));
  auto phys = [&](int c) { const int p = c + rot; return p >= nchunks ? p - nchunks : p; };
  auto issue = [&](int slot, int c) {
    uint8_t* base = &ring[slot * kSlotB];
    const int pc = phys(c);
#pragma unroll
    for (int i = 0; i < kPerWaveMax; ++i)
      if (i < my_count)
        dma16(src[i] + size_t(pc) * (is_w[i] ? kRowB : kXChunkK * 2), base + dst[i]);
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

  const uint32_t magic = opaque_u32(Mf::kMagic);
  float4_t acc[MT][TILES];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < TILES; ++t) acc[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};

  // int8: raw sums over the chunks of one scale group, scaled into acc when
  // the group changes (per-channel scales: once, after the last chunk).
  float4_t raw[MT][TILES];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < TILES; ++t) raw[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};
  auto add_scaled = [&](const float4_t (&part)[MT][TILES], int g) {
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const uint8_t* ps = sl + (size_t(t * 16 + r16) * num_scales + g) * kSSize;
      float sc;
      if constexpr (SD == kRT) sc = load_scale<kRT>(ps, sd_rt);
      else if constexpr (SD == LQ_F32) sc = *reinterpret_cast<const float*>(ps);
      else if constexpr (SD == LQ_F16) sc = float(*reinterpret_cast<const half_t*>(ps));
      else sc = bf16_to_f32(*reinterpret_cast<const uint16_t*>(ps));
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        acc[mt][t] += part[mt][t] * sc;
        // keep the MFMA-result read in this block (see gemv_tile_kernel)
        __asm__ volatile("" : "+v"(acc[mt][t]));
      }
    }
  };

  // int8: a group of G % 256 == 0 spans cpg whole chunks (and the chunk walk
  // wraps at a group boundary, K % G == 0); other groups are scaled every
  // chunk.  `left` counts the chunks to the end of the current group.
  const int cpg = group % kXChunkK == 0 ? group / kXChunkK : 1;
  int left = cpg - rot % cpg;
  auto compute = [&](int slot, int c) {
    const uint8_t* wl = &ring[slot * kSlotB];
    const uint8_t* xl = wl + kWBytes;
    const int pc = phys(c);
    if constexpr (WBITS == 8) {
      // one 16x16x32 block: the lane's 8 k are wave * 32 + q4 * 8 ..: bytes
      // 8 q4 of weight position 2 wave + q4 / 2, activation position 4 wave + q4;
      // the int8 weights are converted to fp16 (bf16 activations: bf16)
      // exactly.
      u32x4_t bw[TILES];
#pragma unroll
      for (int t = 0; t < TILES; ++t) {
        const int row = t * 16 + r16;
        const u32x2_t w = *reinterpret_cast<const u32x2_t*>(
            wl + row * kRowB + (((2 * wave + (q4 >> 1)) ^ (row & (kPos - 1))) << 4) + ((q4 & 1) << 3));
        if constexpr (kH) {
          half2_t lo[2], hi[2];
          int8x4_to_h2(w.x, lo);
          int8x4_to_h2(w.y, hi);
          bw[t] = u32x4_t{as_u32(lo[0]), as_u32(lo[1]), as_u32(hi[0]), as_u32(hi[1])};
        } else {
          const u32x2_t a = int8x4_to_bf16(w.x), b = int8x4_to_bf16(w.y);
          bw[t] = u32x4_t{a.x, a.y, b.x, b.y};
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + r16;
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(
            xl + row * (kXChunkK * 2) + (((4 * wave + q4) ^ (row & 15)) << 4));
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          if constexpr (kH)
            raw[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                __builtin_bit_cast(h8, xv), __builtin_bit_cast(h8, bw[t]), raw[mt][t], 0, 0, 0);
          else
            raw[mt][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                __builtin_bit_cast(bf8_t, xv), __builtin_bit_cast(bf8_t, bw[t]), raw[mt][t], 0, 0, 0);
        }
      }
      if (--left == 0 || c + 1 == nchunks) {
        left = cpg;
        add_scaled(raw, div_rcp(pc * kXChunkK + wave * 32, group, rgroup));
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int t = 0; t < TILES; ++t) raw[mt][t] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
    } else {
      // one 16x16x32 block: the lane's 8 k are wave * 32 + q4 * 8 .., i.e.
      // dword q4 of weight chunk `wave` and activation bytes 64 w + 16 q4
      float4_t part[MT][TILES];
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
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 16 + r16;
        const int chunk = wave * 4 + q4;
        const u32x4_t xv = *reinterpret_cast<const u32x4_t*>(
            xl + row * (kXChunkK * 2) + ((chunk ^ (row & 15)) << 4));
        const op_t xa = Mf::prep_x(xv);
        const float4_t start = Mf::mfma(xa, nb, float4_t{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int t = 0; t < TILES; ++t) part[mt][t] = Mf::mfma(xa, bw[t], start);
      }
      add_scaled(part, div_rcp(pc * kXChunkK + wave * 32, group, rgroup));
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
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int t = 0; t < TILES; ++t) red[((wave * MT + mt) * TILES + t) * 64 + lane] = acc[mt][t];
  __syncthreads();
  for (int pidx = wave; pidx < MT * TILES; pidx += 8) {
    const int mt = pidx / TILES, t = pidx % TILES;
    float4_t v = red[(mt * TILES + t) * 64 + lane];
#pragma unroll
    for (int w2 = 1; w2 < 8; ++w2) v += red[((w2 * MT + mt) * TILES + t) * 64 + lane];
    const int n = n0 + t * 16 + r16;
#pragma unroll
    for (int r = 0; r < 4; r += kPairs ? 2 : 1) {
      const int m = mt * 16 + q4 * 4 + r;
      // pairs: part rows m, m + 1 -> output row m / 2
      const float y = kPairs ? v[r] + v[(r + 1) & 3] : v[r];
      const int mo = kPairs ? m >> 1 : m;
      if constexpr (EPI) {
        const float up = __shfl_xor(y, 1, 64);
        if ((r16 & 1) == 0 && m < M && n < N)
          store_out<OD>(O, size_t(mo) * (N / 2) + n / 2, y / (1.0f + expf(-y)) * up, od_rt);
      } else {
        if (m < M && n < N) store_out<OD>(O, size_t(mo) * N + n, y, od_rt);
      }
    }
  }
}

}  // namespace lq
