// Prefill-shaped dequant-matmul for gfx950: O[M, N] = X[M, K] @ deq(W)^T with
// fp16 activations, int4 or int8 group-wise weights, fp16 MFMA and fp32
// accumulation.
//
// The reference has no GEMM for this path; it would run one matvec launch per
// activation row (locomp examples/38_quantized_matmul.py:154).  Values follow
// the same definition: w = (q - 8) * s[n, k / G] (int4), q * s (int8).
//
// Tiling (default GemmCfg<4, 2, 4, 4>: 512 lanes, BM x BN = 256 x 128, BK = 64):
//   * Waves form a 4 x 2 grid; each owns 64 x 64 outputs: 4 x 4 tiles of
//     v_mfma_f32_16x16x32_f16 (fp32 accumulators in VGPRs), which reads 16 KB
//     of LDS fragments per wave per k-step (32 x 128 waves read 20 KB).
//   * Activations: each k-step's 256 x 64 fp16 tile is copied global -> LDS by
//     the gfx950 direct-to-LDS load (global_load_lds_dwordx4): no VGPRs, 128 B
//     of one row per 8 lanes, XOR-swizzled chunk order chosen through the
//     source addresses.  A 3-slot ring keeps steps ks + 1 and ks + 2 in flight.
//   * Weights: the 128 x 32-byte (int4) or 128 x 64-byte (int8) tile of step
//     ks + 3 (int4) / ks + 2 (int8) is loaded into registers during step ks,
//     and each tile is dequantised during the step before its use to exact
//     fp16 (q - 8) times the fp16 scale (one rounding; int8: the exact q) and
//     written to an XOR-swizzled LDS tile (2 stages) that every wave reads as
//     the B operand.
//   * One barrier per step, in its middle: the MFMA operand fragments of each
//     32-k half are read from LDS while the other half's MFMAs run (the next
//     step's first half right after the barrier).  The loop's loads are
//     inline asm with hand-placed s_waitcnt (the compiler would drain vmcnt
//     before every LDS read after an LDS-DMA); MFMAs use the VGPR-destination
//     form (build flag), which keeps the accumulators from being copied
//     between VGPRs and AGPRs.
//   * XCD-aware order: consecutive workgroups are dealt round-robin to the 8
//     XCDs, so each XCD is given a block of tiles that share activation and
//     weight rows in its L2 (cfg 5a: 4 x 8 tiles, 1 MB of X rows and 2 MB of
//     packed weights).
#include <algorithm>
#include <mutex>
#include <type_traits>
#include <vector>

#include "lq_common.h"


namespace lq {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf8_t __attribute__((ext_vector_type(8)));

constexpr int kBK = 64;

// Tile configuration: WM x WN waves, each owning (16 TM) x (16 TN) outputs.
// OCC_ = workgroups per CU the register budget is sized for.
template <int WM_, int WN_, int TM_, int TN_, int OCC_ = 1>
struct GemmCfg {
  static constexpr int WM = WM_, WN = WN_, TM = TM_, TN = TN_, kOcc = OCC_;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int BM = WM * TM * 16;
  static constexpr int BN = WN * TN * 16;
};

// Weight bytes of one k-step row (64 k): 32 (int4) or 64 (int8); bytes per
// loader thread; k covered by one loader thread.
template <class C, int WBITS>
struct GemmB {
  static constexpr int kRowBytes = 64 * WBITS / 8;
  static constexpr int kBytes = C::BN * kRowBytes / C::kThreads;
  static constexpr int kPerRow = kRowBytes / kBytes;
  static constexpr int kSpanK = kBytes * 8 / WBITS;
  static_assert(kBytes == 8 || kBytes == 16, "64- or 128-bit weight loads");
};

// LDS element offset (halves) of 16-byte chunk c (of 8 per row) of weight
// row n, XOR-swizzled so the 16 rows one ds_read_b128 touches spread over banks.
__device__ __forceinline__ int b_lds_off(int n, int c) { return n * kBK + ((c ^ (n & 7)) << 3); }

// ------------------------------------------------------ explicit loads --
// The main loop's global loads are issued with inline asm so that the
// compiler's wait analysis (which treats an LDS-DMA as a write to all of LDS
// and would drain vmcnt before every LDS read) stays out of the loop; every
// wait is placed by hand and names the registers it guards, so no consumer
// can be scheduled before it.  M0 is used by nothing else in this kernel.
// (lds_addr, dma16 and the gload_* helpers live in lq_common.h.)

// A (activation) tile in LDS: BM rows x 64 k fp16 = 128 B per row, 16-byte
// chunk c of row m stored at chunk position c ^ (m & 7).
__device__ __forceinline__ int a_lds_off(int m, int c) { return m * kBK + ((c ^ (m & 7)) << 3); }

constexpr int kAStages = 3;   // activation ring: steps ks, ks + 1, ks + 2
constexpr int kGemmScaleFloats = 8192;   // int8 post-scale: BN x (K / G) fp32 scales
constexpr int kBStages = 2;

// XCD-aware tile order: workgroup b runs on XCD b % 8.  When the tile grid
// splits into 8 equal blocks of gm x gn tiles, XCD x takes block x, with gm
// chosen to minimise the bytes one k-step of the block reads (gm tiles of
// `a_bytes` activation bytes per k + gn tiles of `b_bytes` weight bytes per
// k): the XCD's L2 then holds the activation rows and weight rows its tiles
// share.  Otherwise XCD x takes the contiguous slice [x per, (x + 1) per) of
// the row-major tile list.  Returns the tile's row and column indices.
__device__ __forceinline__ void xcd_tile(int b, int tiles_m, int tiles_n, int a_bytes, int b_bytes,
                                         int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int t = b, gm = 0;
  if (total % 8 == 0) {
    const int per = total >> 3;
    int best = 1 << 30;
    for (int d = 1; d <= tiles_m && d <= per; ++d) {
      if (tiles_m % d || per % d || tiles_n % (per / d)) continue;
      const int cost = d * a_bytes + (per / d) * b_bytes;
      if (cost < best) { best = cost; gm = d; }
    }
    if (gm == 0) t = (b & 7) * per + (b >> 3);
  }
  if (gm > 0) {
    const int gn = (total >> 3) / gm, gcols = tiles_n / gn;
    const int xcd = b & 7, local = b >> 3;
    tm = (xcd / gcols) * gm + local % gm;
    tn = (xcd % gcols) * gn + local / gm;
  } else {
    tm = t / tiles_n;
    tn = t % tiles_n;
  }
}

// EPI: gate/up rows interleaved (2i, 2i + 1); store silu(gate) * up to
// O [M, N / 2] (columns n and n + 1 sit in lanes r16 and r16 ^ 1).
// XD: activation dtype, fp16 (fp16 MFMA) or bf16 (bf16 MFMA; B holds the
// exact integers q - 8 / q as bf16 and the scales are applied in fp32, like
// int8).  XD = kXPairs: bf16 part rows of fp32 activations, the two parts of
// row i at rows 2i and 2i + 1 (M counts part rows); the epilogue adds each
// pair (rows 4 q + r and 4 q + r + 1 sit in one lane) and stores O [M / 2, N]
// (EPI: [M / 2, N / 2]).  SD / OD = kRT take the scale / output dtype from
// sd_rt / od_rt.
template <class C, int WBITS, int SD, int OD, bool EPI = false, int XD = LQ_F16>
__global__ __launch_bounds__(C::kThreads, C::kOcc) void gemm_w4_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int group, int tiles_m, int tiles_n,
    int kspan, int sd_rt = 0, int od_rt = 0) {
  constexpr int TM = C::TM, TN = C::TN, BM = C::BM, BN = C::BN;
  static_assert(BM % (8 * C::kWaves) == 0, "A DMA: whole 1 KB instructions per wave");
  constexpr bool kParts = XD == kXPairs;
  constexpr bool kBf = XD == LQ_BF16 || kParts;
  typedef typename Elem<SD == kRT ? LQ_F32 : SD>::T stype;
  __shared__ __attribute__((aligned(16))) half_t As[kAStages][BM * kBK];
  __shared__ __attribute__((aligned(16))) half_t Bs[kBStages][BN * kBK];
  // int8 (and bf16 activations): B holds the exact integers and the group
  // scales are applied to fp32 partial sums (a pre-scaled fp16 weight would
  // round |q s| up to 2.5 to 11 bits, too coarse at K = 4096; bf16 keeps 8);
  // the tile's scale rows live here.
  constexpr bool kPost = WBITS == 8 || kBf;
  __shared__ float Ssh[kPost ? kGemmScaleFloats : 1];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // wave-uniform (an SGPR): addresses derived from it stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15;
  const int q4 = lane >> 4;
  const int wm = wave / C::WN;
  const int wn = wave % C::WN;

  int m0, n0;
  xcd_tile(blockIdx.x, tiles_m, tiles_n, BM * 2, BN * WBITS / 8, m0, n0);
  m0 *= BM;
  n0 *= BN;
  const int row_bytes = WBITS == 4 ? (K >> 1) : K;
  // split-K: workgroup row blockIdx.y covers k in [kbeg, min(kbeg + kspan, K))
  // (kspan a whole number of 64-k steps) and writes its fp32 partial sums to
  // slice blockIdx.y of O
  const int kbeg = blockIdx.y * kspan;
  kspan = min(kspan, K - kbeg);                // the last split may be shorter
  const size_t obase = size_t(blockIdx.y) * (kParts ? M / 2 : M) * N;
  const int wrow0 = wm * TM * 16;              // first tile row this wave multiplies

  // A DMA: wave w copies rows [w * kDmaRows, (w + 1) * kDmaRows) of the tile
  // (128 B per row): instruction i writes LDS bytes [i KB, i KB + 1 KB) of that
  // slice, lane L at +16 L, i.e. row (8 i + L / 8), chunk position L % 8,
  // holding logical chunk (L % 8) ^ (row & 7).  Eight lanes cover one row.
  constexpr int kDmaRows = BM / C::kWaves;
  constexpr int kADma = kDmaRows / 8;
  // (buffer loads: a per-lane 32-bit byte offset fixed for the whole loop,
  // the step's k in the scalar offset; rows past M re-read row M - 1)
  const int drow0 = wave * kDmaRows;
  const i32x4_t xrsrc = {int(uint32_t(reinterpret_cast<uint64_t>(X))),
                         int(uint32_t(reinterpret_cast<uint64_t>(X) >> 32) & 0xFFFFu),
                         int(uint32_t(M) * uint32_t(K) * 2u), 0x00020000};
  uint32_t adma_off[kADma];
#pragma unroll
  for (int i = 0; i < kADma; ++i) {
    const int row = drow0 + 8 * i + (lane >> 3);
    const int m = min(m0 + row, M - 1);
    const int c = (lane & 7) ^ (row & 7);
    adma_off[i] = (uint32_t(m) * uint32_t(K) + uint32_t(kbeg + c * 8)) * 2u;
  }
  const uint32_t as_base = lds_addr(&As[0][0]) + uint32_t(drow0 * kBK * 2);   // (scalar)
  auto dma_a = [&](int stage, int k0) {
#pragma unroll
    for (int i = 0; i < kADma; ++i)
      dma16_so(xrsrc, adma_off[i], uint32_t(k0) * 2u,
               as_base + uint32_t(stage * BM * kBK * 2 + 8 * i * kBK * 2));
  };

  // B loader: Bg::kBytes weight bytes (Bg::kSpanK k) of one weight row
  typedef GemmB<C, WBITS> Bg;
  constexpr int kPerRow = Bg::kPerRow;
  const int b_n = tid / kPerRow;
  const int b_part = tid % kPerRow;
  const int bn = min(n0 + b_n, N - 1);
  const uint8_t* wrow = W + size_t(bn) * row_bytes + (WBITS == 4 ? (kbeg >> 1) : kbeg) + b_part * Bg::kBytes;
  const stype* sp = static_cast<const stype*>(S) + size_t(bn) * num_scales;
  constexpr int kBWords = Bg::kBytes / 4;
  // Packed weights rotate through kBSets register sets, loaded kBSets steps
  // ahead.  Three (int4): during step ks the loads of B(ks + 3) fill one,
  // B(ks + 1) is dequantised from another, and the third holds B(ks + 2),
  // which the step's middle wait covers.  Two (int8, whose post-scale
  // accumulators leave no registers for a third): B(ks + 2) fills one and is
  // waited for at the end of the step.  A set is never copied while its loads
  // are in flight.
  constexpr int kBSets = kPost ? 2 : 3;
  struct BRegs {
    u32x4_t b;      // 16-byte loads
    u32x2_t b2;     // 8-byte loads
    uint32_t s;     // raw scale bits, converted when the tile is dequantised
  };
  auto load_b = [&](BRegs& r, int k0) {
    const int kb = WBITS == 4 ? (k0 >> 1) : k0;          // byte offset of k0 in the row
    if constexpr (kBWords == 4) r.b = gload_b128(wrow + kb);
    else r.b2 = gload_b64(wrow + kb);
    if constexpr (!kPost) {
      const stype* ps = sp + (kbeg + k0 + b_part * Bg::kSpanK) / group;
      if constexpr (sizeof(stype) == 2) r.s = gload_u16(ps);
      else r.s = gload_b32(ps);
    }
  };
  // Placed right after the wait that covers a set's loads: names its registers
  // there, so no read of them is scheduled before the wait.
  auto tie_b = [&](BRegs& r) {
    if constexpr (kBWords == 4) __asm__ volatile("" : "+v"(r.b));
    else __asm__ volatile("" : "+v"(r.b2));
    if constexpr (!kPost) __asm__ volatile("" : "+v"(r.s));
  };
  auto store_b = [&](const BRegs& r, int stage) {
    float bs;
    if constexpr (SD == LQ_F32) bs = __uint_as_float(r.s);
    else if constexpr (SD == LQ_F16) bs = float(__builtin_bit_cast(half_t, uint16_t(r.s)));
    else bs = bf16_to_f32(uint16_t(r.s));
    uint32_t bq[4];   // first kBWords used
    if constexpr (kBWords == 4) {
      bq[0] = r.b.x; bq[1] = r.b.y; bq[2] = r.b.z; bq[3] = r.b.w;
    } else {
      bq[0] = r.b2.x; bq[1] = r.b2.y; bq[2] = 0u; bq[3] = 0u;
    }
    const half_t hs = half_t(bs);
    const half2_t s2 = {hs, hs};
    half_t* dst = Bs[stage];
    const uint32_t magic = opaque_u32(0x64006400u);
    if constexpr (kBf) {
      // exact integers as bf16: an integer of at most 8 significant bits is
      // exact as a float, whose high half is then its bf16 pattern
      (void)s2;
      auto pack = [](float lo, float hi) {
        return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
      };
      if constexpr (WBITS == 4) {
#pragma unroll
        for (int i = 0; i < kBWords; ++i) {
          const uint32_t e = bq[i] & 0x0F0F0F0Fu, o = (bq[i] >> 4) & 0x0F0F0F0Fu;
          float f[8];
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            f[2 * b] = float((e >> (8 * b)) & 0xFFu) - 8.0f;       // k = 2 b
            f[2 * b + 1] = float((o >> (8 * b)) & 0xFFu) - 8.0f;   // k = 2 b + 1
          }
          u32x4_t v;
          v.x = pack(f[0], f[1]);
          v.y = pack(f[2], f[3]);
          v.z = pack(f[4], f[5]);
          v.w = pack(f[6], f[7]);
          *reinterpret_cast<u32x4_t*>(dst + b_lds_off(b_n, b_part * kBWords + i)) = v;
        }
      } else {
#pragma unroll
        for (int i = 0; i < kBWords / 2; ++i) {
          float f[8];
#pragma unroll
          for (int b = 0; b < 8; ++b) {
            const uint32_t u = bq[2 * i + (b >> 2)] ^ 0x80808080u;
            f[b] = float((u >> (8 * (b & 3))) & 0xFFu) - 128.0f;
          }
          u32x4_t v;
          v.x = pack(f[0], f[1]);
          v.y = pack(f[2], f[3]);
          v.z = pack(f[4], f[5]);
          v.w = pack(f[6], f[7]);
          *reinterpret_cast<u32x4_t*>(dst + b_lds_off(b_n, b_part * (kBWords / 2) + i)) = v;
        }
      }
    } else if constexpr (WBITS == 4) {
      // one dword = 8 k = one 16-byte LDS chunk
#pragma unroll
      for (int i = 0; i < kBWords; ++i) {
        half2_t h[4];
        int4x8_to_h2(bq[i], h, magic);
        u32x4_t v;
        v.x = as_u32(h[0] * s2);
        v.y = as_u32(h[1] * s2);
        v.z = as_u32(h[2] * s2);
        v.w = as_u32(h[3] * s2);
        *reinterpret_cast<u32x4_t*>(dst + b_lds_off(b_n, b_part * kBWords + i)) = v;
      }
    } else {
      // two dwords = 8 k = one 16-byte LDS chunk of exact integers
      (void)s2;
#pragma unroll
      for (int i = 0; i < kBWords / 2; ++i) {
        half2_t h[4];
        int8x4_to_h2(bq[2 * i], h);
        int8x4_to_h2(bq[2 * i + 1], h + 2);
        u32x4_t v;
        v.x = as_u32(h[0]);
        v.y = as_u32(h[1]);
        v.z = as_u32(h[2]);
        v.w = as_u32(h[3]);
        *reinterpret_cast<u32x4_t*>(dst + b_lds_off(b_n, b_part * (kBWords / 2) + i)) = v;
      }
    }
  };

  float4_t acc[TM][TN];
  float4_t part[kPost ? TM : 1][kPost ? TN : 1];   // int8: this group's unscaled sums
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (kPost) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) part[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
    // stage the tile's scale rows (fp32) before any hand-counted load
    // (the groups this split touches: g0 .. g0 + ns - 1; a group may start
    // in an earlier split or end in a later one)
    const int g0 = kbeg / group, ns = (kbeg + kspan - 1) / group - g0 + 1;
    for (int idx = tid; idx < BN * ns; idx += C::kThreads) {
      const int row = idx / ns;
      const int n = min(n0 + row, N - 1);
      Ssh[idx] = load_f32_rt<SD>(S, size_t(n) * num_scales + g0 + (idx - row * ns), sd_rt);
    }
  }

  const int ksteps = kspan / kBK;
  // prologue: A(0), A(1) by DMA; B(0) dequantised into LDS; B(1) (and B(2))
  // in their register sets
  BRegs r0, r1, r2;
  dma_a(0, 0);
  dma_a(1, min(1, ksteps - 1) * kBK);
  load_b(r0, 0);
  load_b(r1, min(1, ksteps - 1) * kBK);
  if constexpr (kBSets == 3) load_b(r2, min(2, ksteps - 1) * kBK);
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  tie_b(r0);
  tie_b(r1);
  if constexpr (kBSets == 3) tie_b(r2);
  store_b(r0, 0);
  __syncthreads();

  // MFMA operand fragments of one 32-k half step (kk): lane (r16, q4) holds
  // k = 8 q4 .. 8 q4 + 7 of that half.  The reads of the next half are issued
  // before the MFMAs of the current one, so LDS reads overlap the matrix
  // cores instead of alternating with them.
  auto read_frags = [&](int a_st, int b_st, int kk, h8 (&fa)[TM], h8 (&fb)[TN]) {
    const half_t* as_l = As[a_st];
    const half_t* bs_l = Bs[b_st];
#pragma unroll
    for (int j = 0; j < TN; ++j)
      fb[j] = *reinterpret_cast<const h8*>(bs_l + b_lds_off((wn * TN + j) * 16 + r16, kk * 4 + q4));
#pragma unroll
    for (int i = 0; i < TM; ++i)
      fa[i] = *reinterpret_cast<const h8*>(as_l + a_lds_off(wrow0 + i * 16 + r16, kk * 4 + q4));
  };
  // acc += part * s[n, g]; part = 0, for the group holding split-relative k
  // `kin` (the first k of the half that ends it)
  const bool half_groups = group % kBK != 0;
  auto post_scale = [&](int kin) {
    const int ns = (kbeg + kspan - 1) / group - kbeg / group + 1;
    const int g = (kbeg + kin) / group - kbeg / group;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const float sj = Ssh[((wn * TN + j) * 16 + r16) * ns + g];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        acc[i][j] += part[i][j] * sj;
        part[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};
        // keep the MFMA-result read in this block (see the decode GEMV)
        __asm__ volatile("" : "+v"(acc[i][j]), "+v"(part[i][j]));
      }
    }
  };
  auto mfmas = [&](const h8 (&fa)[TM], const h8 (&fb)[TN]) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (kBf)
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
              __builtin_bit_cast(bf8_t, fa[i]), __builtin_bit_cast(bf8_t, fb[j]), part[i][j], 0, 0, 0);
        else if constexpr (kPost)
          part[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], part[i][j], 0, 0, 0);
        else
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
  };
  // loads this thread issues per step besides the A DMA: weights (+ scale)
  constexpr int kBLoads = kPost ? 1 : 2;

  h8 fa0[TM], fb0[TN], fa1[TM], fb1[TN];
  read_frags(0, 0, 0, fa0, fb0);
  int a_stage = 0;
  // rl: receives B(ks + kBSets); rs: holds B(ks + 1), dequantised now; rt
  // (three sets): holds B(ks + 2), covered by this step's middle wait.
  auto step = [&](int ks, BRegs& rl, const BRegs& rs, BRegs& rt) {
    const int b_stage = ks & 1;
    const int a_next = a_stage == 2 ? 0 : a_stage + 1;
    const int a_next2 = a_stage == 0 ? 2 : a_stage - 1;   // (a_stage + 2) % 3
    // Issue B(ks + kBSets) then A(ks + 2) (branch-free: past the end they
    // re-read the last step and land in buffers no one reads).  A stage
    // (ks + 2) % 3 and B stage (ks + 1) % 2 were last read in step ks - 1,
    // before its middle barrier.
    load_b(rl, min(ks + kBSets, ksteps - 1) * kBK);
    dma_a(a_next2, min(ks + 2, ksteps - 1) * kBK);
    // The scheduling barriers keep each half's fragment reads ahead of the
    // other half's MFMAs (the scheduler would otherwise sink them to their use).
    read_frags(a_stage, b_stage, 1, fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    mfmas(fa0, fb0);
    store_b(rs, b_stage ^ 1);                  // dequantise B(ks + 1)
    __builtin_amdgcn_sched_barrier(0);
    // Only this step's loads may remain: A(ks + 1) (and with three sets
    // B(ks + 2)) landed, and after the barrier B(ks + 1) is in LDS for every
    // wave: the next step's first half can be read.
    __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kBLoads + kADma) : "memory");
    if constexpr (kBSets == 3) tie_b(rt);
    __syncthreads();
    read_frags(a_next, b_stage ^ 1, 0, fa0, fb0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPost) {
      // groups of an odd number of 32-k halves (G % 64 == 32) may end after
      // the first half: fold its sums before the second half's MFMAs
      if (half_groups && (kbeg + ks * kBK + kBK / 2) % group == 0) post_scale(ks * kBK);
    }
    mfmas(fa1, fb1);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (kPost) {
      // a group (or this split's share of one) ends with this step
      if ((kbeg + (ks + 1) * kBK) % group == 0 || ks + 1 == ksteps) post_scale(ks * kBK + kBK / 2);
    }
    if constexpr (kBSets == 2) {
      __asm__ volatile("s_waitcnt vmcnt(%0)" ::"n"(kADma) : "memory");   // B(ks + 2) landed
      tie_b(rl);
    }
    a_stage = a_next;
  };
  if constexpr (kBSets == 3) {
    for (int ks = 0; ks < ksteps; ks += 3) {
      step(ks, r0, r1, r2);
      if (ks + 1 < ksteps) step(ks + 1, r1, r2, r0);
      if (ks + 2 < ksteps) step(ks + 2, r2, r0, r1);
    }
  } else {
    for (int ks = 0; ks < ksteps; ks += 2) {
      step(ks, r0, r1, r2);
      if (ks + 1 < ksteps) step(ks + 1, r1, r0, r2);
    }
  }

  // The last steps' A copies (clamped repeats) are still in flight: drain
  // them before the workgroup's LDS can be handed to another workgroup.
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  tie_b(r0);
  tie_b(r1);
  if constexpr (kBSets == 3) tie_b(r2);
  // Epilogue: lane holds rows 4 * (lane / 16) + r, column lane % 16 of each tile.
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wrow0 + i * 16 + q4 * 4 + r;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int n = n0 + (wn * TN + j) * 16 + r16;
        if constexpr (kParts) {
          // hi part + lo part (M even: row m + 1 < M with m)
          if ((r & 1) != 0) continue;
          const float y = acc[i][j][r] + acc[i][j][(r + 1) & 3];
          if constexpr (EPI) {
            const float up = __shfl_xor(y, 1, 64);
            if ((r16 & 1) == 0 && m < M && n < N)
              store_out<OD>(O, size_t(m >> 1) * (N / 2) + n / 2, y / (1.0f + expf(-y)) * up, od_rt);
          } else {
            if (m < M && n < N) store_out<OD>(O, obase + size_t(m >> 1) * N + n, y, od_rt);
          }
        } else if constexpr (EPI) {
          const float g = acc[i][j][r];
          const float up = __shfl_xor(g, 1, 64);
          if ((r16 & 1) == 0 && m < M && n < N)
            store_out<OD>(O, size_t(m) * (N / 2) + n / 2, g / (1.0f + expf(-g)) * up, od_rt);
        } else {
          if (m < M && n < N) store_out<OD>(O, obase + size_t(m) * N + n, acc[i][j][r], od_rt);
        }
      }
    }
  }
}

// ------------------------------------------------- pair-split int4 GEMM --
// Prefill with int4 weights and fp16 activations on 128 x 256 output tiles
// (cfg 5a: 16 x 16 tiles, one per CU).  Against the 256 x 128 kernel above it
// moves a third fewer bytes from L2 per k (the int4 weight tile is the cheap
// operand, so the tile is made wide in N) and about half the LDS bytes:
//   * Waves (cb = w & 3, p = w >> 2): wave w owns output columns cb*64..+64 of
//     the tile and all 128 rows (8 x 4 tiles of v_mfma_f32_16x16x32_f16, fp32
//     accumulators in VGPRs), and of every 128-k unit only the 64-k stage p.
//     The two waves of a column block (one SIMD each, if the hardware deals
//     waves to SIMDs in turn) therefore split K, and add their sums through
//     LDS once at the end.
//   * Weights never pass through LDS: each wave loads its own packed bytes
//     (lane (r16, q4) of column tile j: the 8 bytes of k = 16 q4 .. 16 q4 + 15
//     of its stage, one 8-byte load) two units ahead into registers and
//     dequantises them to exact fp16 (q - 8) * s just before its MFMAs.  Every
//     weight of the tile is decoded once per workgroup.  The MFMA's k order
//     inside the stage is permuted to match: block t of lane (r16, q4) holds
//     k = 16 q4 + 8 t + i, i.e. 16-byte activation chunk 2 q4 + t of the row.
//   * Activations: each unit's 128 x 128 fp16 tile is copied global -> LDS by
//     direct-to-LDS buffer loads (XOR-swizzled chunks, as above) into a ring of
//     four units (128 KB), three units ahead.  One barrier per unit.
//   * Every wait is a hand-placed vmcnt that is exact under in-order
//     completion: per unit each wave issues 4 weight loads, 4 scale loads and
//     4 activation copies, in that order.
// Needs K % 128 == 0 and a power-of-two group G >= 16 dividing K (a lane's 16
// k then share one scale); the buffer sizes of X, W and the scales below 4 GB.
constexpr int kPBM = 128, kPBN = 256, kPUnit = 128, kPLds = 160 * 1024;

__device__ __forceinline__ u32x2_t bload_b64(i32x4_t rsrc, uint32_t voff, uint32_t soff) {
  u32x2_t v;
  __asm__ volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rsrc), "s"(soff) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t bload_u16(i32x4_t rsrc, uint32_t voff) {
  uint32_t v;
  __asm__ volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t bload_b32(i32x4_t rsrc, uint32_t voff) {
  uint32_t v;
  __asm__ volatile("buffer_load_dword %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t bload_u16_so(i32x4_t rsrc, uint32_t voff, uint32_t soff) {
  uint32_t v;
  __asm__ volatile("buffer_load_ushort %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rsrc), "s"(soff) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t bload_b32_so(i32x4_t rsrc, uint32_t voff, uint32_t soff) {
  uint32_t v;
  __asm__ volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(v) : "v"(voff), "s"(rsrc), "s"(soff) : "memory");
  return v;
}
__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4_t{int(uint32_t(a)), int(uint32_t(a >> 32) & 0xFFFFu), int(bytes), 0x00020000};
}

// Scheduling pattern for one row tile's 4 MFMAs and the work meant to run
// under them: DS LDS reads after the first MFMA, VALU VALU ops after each.
template <int DS, int VALU>
__device__ __forceinline__ void interleave_mfma4() {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
    if constexpr (DS > 0)
      if (j == 0) __builtin_amdgcn_sched_group_barrier(0x100, DS, 0);   // LDS read
    __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);   // VALU
  }
}

template <int SD, int OD, bool EPI, int SLOTS>
__global__ __launch_bounds__(512, 1) void gemm_w4p_kernel(
    const half_t* __restrict__ X, const uint8_t* __restrict__ W, const void* __restrict__ S,
    void* __restrict__ O, int M, int N, int K, int num_scales, int lg_group, int tiles_m,
    int tiles_n) {
  // SLOTS units of activations (32 KB each), then the tile's scale rows; the
  // first 128 KB take the final reduction.
  __shared__ __attribute__((aligned(16))) uint8_t lds[kPLds];
  half_t (*As)[kPBM * kBK] = reinterpret_cast<half_t (*)[kPBM * kBK]>(lds);
  uint8_t* Ss = lds + SLOTS * 32768;
  constexpr int kDA = SLOTS - 1;                 // activation copies run kDA units ahead
  typedef typename Elem<SD>::T stype;
  constexpr uint32_t kEs = sizeof(stype);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cb = wave & 3, p = wave >> 2;
  const int r16 = lane & 15, q4 = lane >> 4;
  int m0, n0;
  xcd_tile(blockIdx.x, tiles_m, tiles_n, kPBM * 2, kPBN / 2, m0, n0);
  m0 *= kPBM;
  n0 *= kPBN;
  const int units = K / kPUnit;
  const uint32_t row_bytes = uint32_t(K) >> 1;

  // A copies: wave w writes rows (w & 3) * 32 .. + 32 of stage p of a unit,
  // 8 rows (1 KB) per instruction; lane L of instruction i: row 8 i + L / 8,
  // chunk position L % 8 holding logical chunk (L % 8) ^ (row & 7).  Rows past
  // M re-read row M - 1.
  const i32x4_t xrsrc = buffer_rsrc(X, uint32_t(M) * uint32_t(K) * 2u);
  const int arow = cb * 32 + (lane >> 3);        // row of copy 0; copy i adds 8 i
  // LDS position x of a row holds logical chunk 2 (y & 3) + (y >> 2), y =
  // x ^ (row & 7): the fragment of lane (r16, q4), block t (logical chunk
  // 2 q4 + t) then sits at position (q4 + 4 t) ^ (row & 7), the positions of
  // the 256 x 128 kernel's reads, which measured free of bank conflicts.
  const int apos = (lane & 7) ^ (arow & 7);      // (row & 7: the same for every copy i)
  const uint32_t achunk = uint32_t((2 * (apos & 3) + (apos >> 2)) * 16);
  const uint32_t aoff0 = uint32_t(min(m0 + arow, M - 1)) * uint32_t(K) * 2u + achunk;
  const uint32_t as_base = lds_addr(&As[0][0]) + uint32_t((p * kPBM * kBK + cb * 32 * kBK) * 2);

  // Weight and scale rows of this lane's four column tiles (rows past N
  // re-read row N - 1).
  const i32x4_t wrsrc = buffer_rsrc(W, uint32_t(N) * row_bytes);
  const uint32_t srow_bytes = uint32_t(num_scales) * kEs;
  const i32x4_t srsrc = buffer_rsrc(S, uint32_t(N) * srow_bytes);
  const int nb = n0 + cb * 64 + r16;             // row of column tile 0
  const uint32_t bv0 = uint32_t(min(nb, N - 1)) * row_bytes + uint32_t(q4 * 8);

  struct PSet {
    u32x2_t b[4];     // packed weights: .x block t = 0, .y block t = 1
  };
  auto tie = [&](PSet& r) {
#pragma unroll
    for (int j = 0; j < 4; ++j) __asm__ volatile("" : "+v"(r.b[j]));
  };
  // The tile's scale rows are one contiguous block of 256 x num_scales
  // entries; it is copied to LDS once (16 bytes per lane; rows past N read as
  // 0), before every other load.
  {
    const uint32_t sbytes = uint32_t(kPBN) * srow_bytes;
    const uint32_t sbase = uint32_t(n0) * srow_bytes;
    const uint32_t ss_lds = lds_addr(&Ss[0]) + uint32_t(wave * 1024);
    for (uint32_t o = 0; o < sbytes; o += 8192u)
      dma16_so(srsrc, sbase + o + uint32_t(tid * 16), 0u, ss_lds + o);
  }
  const int srow0 = cb * 64 + r16;               // tile-local scale row of column tile 0

  float4_t acc[8][4];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = float4_t{0.f, 0.f, 0.f, 0.f};

  const uint32_t magic = opaque_u32(0x64006400u);
  // exact fp16 (q - 8) * s of block t of column tile j
  // scale of column tile j for unit u, as fp16
  auto scale = [&](int j, int u) {
    const int g = (u * kPUnit + p * 64 + q4 * 16) >> lg_group;
    const stype v = *reinterpret_cast<const stype*>(&Ss[((srow0 + j * 16) * num_scales + g) * int(kEs)]);
    if constexpr (SD == LQ_F16) return v;
    else if constexpr (SD == LQ_F32) return half_t(v);
    else return half_t(bf16_to_f32(v));
  };
  // exact fp16 (q - 8) * s of weights 2 e, 2 e + 1 of block t of column
  // tile j: one half2 (4 VALU ops)
  auto decode_pair = [&](const PSet& r, int j, int t, int e, half_t hs) {
    const uint32_t w = t == 0 ? r.b[j].x : r.b[j].y;
    const half2_t s2 = {hs, hs};
    return as_u32(int4_pair_to_h2(w, e, magic) * s2);
  };
  auto read_a = [&](const half_t* a, int i, int t) {
    const int m = i * 16 + r16;
    return *reinterpret_cast<const h8*>(a + m * kBK + (((q4 + 4 * t) ^ (m & 7)) << 3));
  };
  // The main loop, for a tile whose rows and columns all exist (FULL: every
  // row offset is a scalar step from the lane's first) or one at the matrix
  // edge (rows clamped lane by lane).
  auto main_loop = [&](auto full_tag) {
    constexpr bool FULL = decltype(full_tag)::value;
    // copy i (8 rows, 1 KB) of this wave's share of unit ud's activations
    auto dma = [&](int ud, int i) {
      const uint32_t kd = uint32_t(min(ud, units - 1) * kPUnit + p * 64) * 2u;
      const uint32_t slot = as_base + uint32_t((ud % SLOTS) * 2 * kPBM * kBK * 2 + i * 8 * kBK * 2);
      if constexpr (FULL)
        dma16_so(xrsrc, aoff0, kd + uint32_t(i * 8) * uint32_t(K) * 2u, slot);
      else
        dma16_so(xrsrc, uint32_t(min(m0 + arow + 8 * i, M - 1)) * uint32_t(K) * 2u + achunk, kd, slot);
    };
    auto bload = [&](PSet& r, int u, int j) {
      const uint32_t kb = uint32_t(min(u, units - 1) * 64 + p * 32);
      if constexpr (FULL) r.b[j] = bload_b64(wrsrc, bv0, kb + uint32_t(j * 16) * row_bytes);
      else r.b[j] = bload_b64(wrsrc, uint32_t(min(nb + 16 * j, N - 1)) * row_bytes + uint32_t(q4 * 8), kb);
    };
    u32x4_t fb[4];
    h8 fa[8];
    u32x4_t fc[4];
    // Block t = 0 of unit u (after the barrier that makes its copy visible):
    // under row tile i, its t = 1 fragment, two pairs of the t = 1 weights of
    // column tile i / 2, and (i < 4) one activation copy of unit u + kDA, whose
    // slot (that of unit u - 1) no wave reads any more.
    auto block0 = [&](int u, const PSet& cur) __attribute__((always_inline)) {
      const half_t* a = As[(u % SLOTS) * 2 + p];
      half_t hs[4];
#pragma unroll
      for (int i = 0; i < 8; ++i) fa[i] = read_a(a, i, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) hs[j] = scale(j, u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], __builtin_bit_cast(h8, fb[j]),
                                                             acc[i][j], 0, 0, 0);
        fa[i] = read_a(a, i, 1);
        const int jj = i >> 1, e0 = (i & 1) * 2;
        fc[jj][e0] = decode_pair(cur, jj, 1, e0, hs[jj]);
        fc[jj][e0 + 1] = decode_pair(cur, jj, 1, e0 + 1, hs[jj]);
        interleave_mfma4<1, 2>();
        if (i < 4) dma(u + kDA, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // Block t = 1 of unit u: under row tile i, two pairs of unit u + 1's t = 0
    // weights of column tile i / 2 and (i < 4) one weight load of unit u + 2
    // into `fut` (unit u's set).
    auto block1 = [&](int u, const PSet& nxt, PSet& fut) __attribute__((always_inline)) {
      half_t hs[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) hs[j] = scale(j, u + 1 < units ? u + 1 : u);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(fa[i], __builtin_bit_cast(h8, fc[j]),
                                                             acc[i][j], 0, 0, 0);
        const int jj = i >> 1, e0 = (i & 1) * 2;
        fb[jj][e0] = decode_pair(nxt, jj, 0, e0, hs[jj]);
        fb[jj][e0 + 1] = decode_pair(nxt, jj, 0, e0 + 1, hs[jj]);
        interleave_mfma4<0, 2>();
        if (i < 4) bload(fut, u + 2, i);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    // The two waves of a column block run half a unit apart, so that one of
    // them is always in the pure-MFMA block t = 1 while the other reads its
    // fragments and issues copies (started together after each barrier, both
    // stall on the same LDS reads).  Waves p = 0 run barrier u, block 0 and
    // block 1 of unit u; waves p = 1 run block 0 of unit u, barrier u + 1,
    // block 1 of unit u (after barrier 0 at the start; the last unit has no
    // barrier).  Both read unit u's fragments only after barrier u and are
    // done with unit u - 1's before barrier u + 1.  Each wave counts its own
    // loads, issued as B0 B1 D0 D1 [D2] (prologue), then D(u + kDA) B(u + 2)
    // per unit (D: 4 copies, B: 4 weight loads); every wait is exact under
    // in-order completion:
    //  * before barrier u, the copy D(u) has landed.  p = 0 (after unit
    //    u - 1): kDA = 3: 8 / 12 / 16 / 20 loads after it at u = 0 / 1 / 2 /
    //    later; kDA = 2: 4 / 8 / 12.  p = 1 (after block 0 of unit u - 1,
    //    before barrier u): kDA = 3: 8 (u = 0, 1), 12 (u = 2), 16; kDA = 2: 4
    //    (u = 0, 1), 8;
    //  * before block 1 of unit u, the weights B(u + 1): after them only the
    //    copy D(u + kDA) (4).
    auto top_wait = [&](int u) __attribute__((always_inline)) {
      if (p == 0) {
        if constexpr (kDA == 3) {
          if (u == 0) __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else if (u == 1) __asm__ volatile("s_waitcnt vmcnt(12)" ::: "memory");
          else if (u == 2) __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory");
          else __asm__ volatile("s_waitcnt vmcnt(20)" ::: "memory");
        } else {
          if (u == 0) __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory");
          else if (u == 1) __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else __asm__ volatile("s_waitcnt vmcnt(12)" ::: "memory");
        }
      } else {
        if constexpr (kDA == 3) {
          if (u <= 1) __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
          else if (u == 2) __asm__ volatile("s_waitcnt vmcnt(12)" ::: "memory");
          else __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory");
        } else {
          if (u <= 1) __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory");
          else __asm__ volatile("s_waitcnt vmcnt(8)" ::: "memory");
        }
      }
    };
    auto unit = [&](int u, PSet& cur, PSet& nxt) __attribute__((always_inline)) {
      if (p == 0) {
        top_wait(u);
        __syncthreads();
      }
      block0(u, cur);
      if (p == 1 && u + 1 < units) {
        top_wait(u + 1);
        __syncthreads();
      }
      __asm__ volatile("s_waitcnt vmcnt(4)" ::: "memory");
      tie(nxt);
      block1(u, nxt, cur);
    };
    PSet r0, r1;
#pragma unroll
    for (int j = 0; j < 4; ++j) bload(r0, 0, j);
#pragma unroll
    for (int j = 0; j < 4; ++j) bload(r1, 1, j);
#pragma unroll
    for (int d = 0; d < kDA; ++d)
#pragma unroll
      for (int i = 0; i < 4; ++i) dma(d, i);
    // the scale copy and the weights of unit 0 have landed (after them: B1
    // and the kDA prologue copies); the barrier makes every wave's scales
    // visible
    if constexpr (kDA == 3) __asm__ volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else __asm__ volatile("s_waitcnt vmcnt(12)" ::: "memory");
    tie(r0);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const half_t h = scale(j, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) fb[j][e] = decode_pair(r0, j, 0, e, h);
    }
    if (p == 1) {   // barrier 0
      top_wait(0);
      __syncthreads();
    }
    for (int u = 0; u < units; u += 2) {
      unit(u, r0, r1);
      if (u + 1 < units) unit(u + 1, r1, r0);
    }
    // Drain the copies and loads past the end before LDS is reused.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    tie(r0);
    tie(r1);
  };
  if (m0 + kPBM <= M && n0 + cb * 64 + 64 <= N) main_loop(std::true_type{});
  else main_loop(std::false_type{});
  __syncthreads();

  // The two K halves: waves p = 1 hand their sums to waves p = 0 through LDS
  // (32 KB per wave, lane-contiguous 16-byte slots), which add them.
  float4_t* red = reinterpret_cast<float4_t*>(lds);
  if (p == 1) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) red[(cb * 32 + i * 4 + j) * 64 + lane] = acc[i][j];
  }
  __syncthreads();
  if (p == 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] += red[(cb * 32 + i * 4 + j) * 64 + lane];
  }
  // Lane holds rows 4 q4 + r of column r16 of each 16 x 16 tile.  EPI: the
  // gate / up pair (columns 2c, 2c + 1) sits in lanes r16, r16 ^ 1.
  auto value = [&](int i, int j, int r) {
    if constexpr (EPI) {
      const float g = acc[i][j][r];
      const float up = __shfl_xor(g, 1, 64);
      return g / (1.0f + expf(-g)) * up;
    } else {
      return acc[i][j][r];
    }
  };
  constexpr int kOutCols = EPI ? kPBN / 2 : kPBN;
  constexpr int kOutEs = OD == LQ_F32 ? 4 : 2;
  const int out_n = EPI ? N / 2 : N;
  const int on0 = EPI ? n0 / 2 : n0;
  // Whole tiles with 16-byte aligned output rows are staged in LDS row by row
  // (the first kPBM x kOutCols x kOutEs bytes) and stored by all 8 waves in
  // 16-byte pieces; other tiles store element by element.
  const bool staged = m0 + kPBM <= M && on0 + kOutCols <= out_n &&
                      (uint32_t(out_n) * kOutEs) % 16u == 0 &&
                      (reinterpret_cast<uintptr_t>(O) & 15u) == 0;
  if (staged) {
    __syncthreads();   // every wave is done with the partial sums in LDS
    if (p == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float v = value(i, j, r);
            const int m = i * 16 + q4 * 4 + r;
            const int n = cb * 64 + j * 16 + r16;
            if (!EPI || (r16 & 1) == 0)
              store_out<OD>(lds, size_t(m) * kOutCols + (EPI ? n / 2 : n), v, 0);
          }
    }
    __syncthreads();
    constexpr int kRowPieces = kOutCols * kOutEs / 16;
    for (int idx = tid; idx < kPBM * kRowPieces; idx += 512) {
      const int m = idx / kRowPieces, c = idx - m * kRowPieces;
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(lds + size_t(idx) * 16);
      *reinterpret_cast<u32x4_t*>(static_cast<uint8_t*>(O) +
                                  (size_t(m0 + m) * out_n + on0) * kOutEs + size_t(c) * 16) = v;
    }
    return;
  }
  if (p == 1) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + i * 16 + q4 * 4 + r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int n = n0 + cb * 64 + j * 16 + r16;
        const float v = value(i, j, r);
        if constexpr (EPI) {
          if ((r16 & 1) == 0 && m < M && n < N) store_out<OD>(O, size_t(m) * (N / 2) + n / 2, v, 0);
        } else {
          if (m < M && n < N) store_out<OD>(O, size_t(m) * N + n, v, 0);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Activation ring units for a tile whose scale rows take `sbytes` of LDS:
// four (32 KB of scales) or three (64 KB); 0 = the scales do not fit.
static int pair_slots(int64_t sbytes) {
  return sbytes <= kPLds - 4 * 32768 ? 4 : sbytes <= kPLds - 3 * 32768 ? 3 : 0;
}

template <int SD, int OD, bool EPI>
static int launch_gemm_pair(const void* X, const void* W, const void* S, void* O, int64_t M,
                            int64_t N, int64_t K, int64_t G, hipStream_t st) {
  int lg = 0;
  while ((int64_t(1) << lg) < G) ++lg;
  const int tiles_m = int((M + kPBM - 1) / kPBM);
  const int tiles_n = int((N + kPBN - 1) / kPBN);
  const int64_t es = SD == LQ_F32 ? 4 : 2;
  const dim3 grid(unsigned(tiles_m * tiles_n)), block(512);
  if (pair_slots(kPBN * (K / G) * es) == 4)
    hipLaunchKernelGGL((gemm_w4p_kernel<SD, OD, EPI, 4>), grid, block, 0, st,
                       static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                       int(N), int(K), int(K / G), lg, tiles_m, tiles_n);
  else
    hipLaunchKernelGGL((gemm_w4p_kernel<SD, OD, EPI, 3>), grid, block, 0, st,
                       static_cast<const half_t*>(X), static_cast<const uint8_t*>(W), S, O, int(M),
                       int(N), int(K), int(K / G), lg, tiles_m, tiles_n);
  return check_launch();
}

// Whether the pair-split kernel takes this int4 / fp16-activation shape: its
// layout limits (K % 128, power-of-two G >= 16, the tile's scale rows within
// 64 KB of LDS, buffers below 4 GB) and enough 128 x 256 tiles to give every
// CU one.
static bool pair_applies(int64_t M, int64_t N, int64_t K, int64_t G, int sd) {
  if (K % kPUnit != 0 || G < 16 || (G & (G - 1)) != 0 || K % G != 0) return false;
  const int64_t es = sd == LQ_F32 ? 4 : 2;
  if (pair_slots(kPBN * (K / G) * es) == 0) return false;
  const int64_t lim = int64_t(1) << 32;
  if (M * K * 2 >= lim || N * (K / 2) >= lim || (N + kPBN) * (K / G) * es >= lim) return false;
  return ((M + kPBM - 1) / kPBM) * ((N + kPBN - 1) / kPBN) >= 256;
}

#ifndef LQ_GEMM_CFG
#define LQ_GEMM_CFG 4, 2, 4, 4
#endif
typedef GemmCfg<LQ_GEMM_CFG> GemmDefault;   // default: 256 x 128 tile, 4 x 2 waves of 64 x 64

// k per split: the 64-k steps dealt in equal runs, the last run possibly
// shorter (the kernel clamps it to K)
static int64_t split_span(int64_t K, int splits) {
  return (K / kBK + splits - 1) / splits * kBK;
}

template <class C, int WBITS, int SD, int OD, bool EPI = false, int XD = LQ_F16>
static int launch_gemm_cfg(const void* X, const void* W, const void* S, void* O, int64_t M,
                           int64_t N, int64_t K, int64_t G, int splits, hipStream_t st,
                           int sd_rt = 0, int od_rt = 0) {
  const int tiles_m = int((M + C::BM - 1) / C::BM);
  const int tiles_n = int((N + C::BN - 1) / C::BN);
  hipLaunchKernelGGL((gemm_w4_kernel<C, WBITS, SD, OD, EPI, XD>), dim3(unsigned(tiles_m * tiles_n), unsigned(splits)),
                     dim3(C::kThreads), 0, st, static_cast<const half_t*>(X),
                     static_cast<const uint8_t*>(W), S, O, int(M), int(N), int(K), int(K / G),
                     int(G), tiles_m, tiles_n, int(split_span(K, splits)), sd_rt, od_rt);
  return check_launch();
}

typedef GemmCfg<4, 2, 2, 4> GemmSmall;     // 128 x 128 tile, 8 waves of 32 x 64

// ------------------------------------------------------------- split-K --
// Fewer output tiles than CUs (M < 1024 at N = 4096): the k range is split
// over up to 8 workgroups per tile, each writing fp32 partial sums to a
// workspace slice [s][M][N]; split_reduce_kernel adds the slices in order and
// converts.  The workspace is cached per (device, stream) and only grows; a
// buffer is never freed while the process runs (a captured graph may still
// name it), and a call on a capturing stream that would need a larger one
// runs unsplit instead.  Calls on one stream are ordered; different streams
// have different workspaces.  Slot 0 holds split-K partials, slot 1 the
// staged matvec of the SiLU * mul fallback (which may itself split K).
constexpr size_t kSplitWsMax = size_t(256) << 20;

struct SplitWs {
  int dev;
  hipStream_t st;
  int slot;
  void* p;
  size_t bytes;
};
static std::mutex g_ws_mu;
static std::vector<SplitWs> g_ws;
static std::vector<SplitWs> g_ws_old;   // superseded by a larger buffer (a graph may name them)

void* stream_workspace(int slot, size_t bytes, hipStream_t st) {
  int dev = 0;
  if (bytes > kSplitWsMax || hipGetDevice(&dev) != hipSuccess) return nullptr;
  std::lock_guard<std::mutex> lock(g_ws_mu);
  for (SplitWs& w : g_ws)
    if (w.dev == dev && w.st == st && w.slot == slot && w.bytes >= bytes) return w.p;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return nullptr;
  size_t sz = size_t(1) << 20;
  while (sz < bytes) sz <<= 1;
  void* p = nullptr;
  if (hipMalloc(&p, sz) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  for (SplitWs& w : g_ws)
    if (w.dev == dev && w.st == st && w.slot == slot) {   // grown: the old buffer stays allocated
      g_ws_old.push_back(w);
      w.p = p;
      w.bytes = sz;
      return p;
    }
  g_ws.push_back(SplitWs{dev, st, slot, p, sz});
  return p;
}

// Frees the workspaces kept for `st` on the current device (all streams of
// the device if `all`), after waiting for the device to be idle.  A graph
// captured earlier that names one must not be replayed afterwards.
int release_workspaces(hipStream_t st, bool all) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  std::lock_guard<std::mutex> lock(g_ws_mu);
  bool any = false;
  for (const auto* v : {&g_ws, &g_ws_old})
    for (const SplitWs& w : *v) any = any || (w.dev == dev && (all || w.st == st));
  if (!any) return LQ_OK;
  e = hipDeviceSynchronize();
  if (e != hipSuccess) return int(e);
  for (auto* v : {&g_ws, &g_ws_old}) {
    std::vector<SplitWs> keep;
    for (const SplitWs& w : *v) {
      if (w.dev == dev && (all || w.st == st)) {
        e = hipFree(w.p);
        if (e != hipSuccess) return int(e);
      } else {
        keep.push_back(w);
      }
    }
    v->swap(keep);
  }
  return LQ_OK;
}
static void* split_workspace(size_t bytes, hipStream_t st) { return stream_workspace(0, bytes, st); }

// Fixed split-K scratch for callers that cannot allocate (the _noalloc entry
// point): one array per device, held by the loaded code object until the
// process ends.  Host code must use the per-device address from
// hipGetSymbolAddress, never `scratch` itself (in host code that name is a
// host-side stand-in, not a device address).  Every call on a device shares
// the device's array: calls that overlap on one device race.  The split-K
// kernels write every element of the slices they read back, so nothing has to
// be cleared between calls.
static __device__ __align__(256) uint8_t scratch[kStaticScratchBytes];

int static_scratch(void** ptr) {
  constexpr int kMaxDev = 64;
  static std::mutex mu;
  static void* addr[kMaxDev] = {};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return int(e);
  if (dev < 0 || dev >= kMaxDev) return LQ_ERR_SCRATCH;
  std::lock_guard<std::mutex> lock(mu);
  if (addr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      (void)hipGetLastError();
      return e != hipSuccess ? int(e) : LQ_ERR_SCRATCH;
    }
    addr[dev] = p;
  }
  *ptr = addr[dev];
  return LQ_OK;
}

template <int OD>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ P,
                                                           void* __restrict__ O, size_t mn,
                                                           int splits, int od_rt = 0) {
  const size_t i = (size_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= mn) return;
  if (i + 4 <= mn && (mn & 3) == 0) {
    float4_t a = *reinterpret_cast<const float4_t*>(P + i);
    for (int s = 1; s < splits; ++s) a += *reinterpret_cast<const float4_t*>(P + size_t(s) * mn + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) store_out<OD>(O, i + e, a[e], od_rt);
  } else {
    for (size_t e = i; e < i + 4 && e < mn; ++e) {
      float a = P[e];
      for (int s = 1; s < splits; ++s) a += P[size_t(s) * mn + e];
      store_out<OD>(O, e, a, od_rt);
    }
  }
}

// int8 stages the scale rows of every group a split touches in kGemmScaleFloats
// of LDS (128 rows): the fewest splits (dividing the 64-k steps) that keep a
// split's groups within that; 0 = none does.  int4 needs no staging.
template <int WBITS, bool POST = WBITS == 8>
static int min_splits(int64_t K, int64_t G) {
  if (!POST) return 1;
  static_assert(GemmDefault::BN == 128 && GemmSmall::BN == 128, "scale staging sized for 128 rows");
  const int64_t ksteps = K / kBK;
  for (int64_t s = 1; s <= ksteps && s <= 64; ++s) {
    if (ksteps % s != 0) continue;
    const int64_t span = K / s;
    int64_t most = 0;   // groups the widest split touches
    for (int64_t i = 0; i < s; ++i)
      most = std::max(most, ((i + 1) * span - 1) / G - (i * span) / G + 1);
    if (most <= kGemmScaleFloats / 128) return int(s);
  }
  return 0;
}

// EPI form of the reduction: O [M, N / 2] = silu(sum of column 2i) * sum of
// column 2i + 1.
template <int OD>
__global__ __launch_bounds__(256) void split_reduce_silu_kernel(const float* __restrict__ P,
                                                                void* __restrict__ O, int64_t M,
                                                                int64_t N, int splits,
                                                                int od_rt = 0) {
  const int64_t half = N / 2;
  const int64_t e = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (e >= M * half) return;
  const int64_t m = e / half, i = e - m * half;
  const size_t mn = size_t(M) * size_t(N);
  const size_t at = size_t(m) * N + 2 * i;
  float g = P[at], u = P[at + 1];
  for (int s = 1; s < splits; ++s) {
    g += P[size_t(s) * mn + at];
    u += P[size_t(s) * mn + at + 1];
  }
  store_out<OD>(O, size_t(e), g / (1.0f + expf(-g)) * u, od_rt);
}

// Number of k splits for `tiles` output tiles: the largest of 8, 6, 4, 3, 2
// that keeps tiles x splits <= 256 (one workgroup per CU), deals the 64-k
// steps into runs of >= 4 (equal runs; the last one may be shorter, as
// split_span, when the runs are >= 8), keeps the scale groups any split touches within the staging
// LDS when `post` (int8 / bf16 post-scales), and is at least `need`.
// Uneven runs let step counts without a divisor use every CU (1 x 4096 x
// 11008 tiles: 172 steps, 4 even splits -> 8).
static int choose_splits(int64_t tiles, int64_t K, int64_t G, int need, bool post) {
  const int64_t ksteps = K / kBK;
  for (int s : {8, 6, 4, 3, 2}) {
    if (s < need || tiles * s > 256) continue;
    const int64_t run = (ksteps + s - 1) / s;
    if (run < 4 || ksteps - (s - 1) * run < 4) continue;
    // uneven runs only on long rows (9 steps as 5 + 4: 1024 x 1536 x 576
    // 12.6 -> 18.4 us against unsplit)
    if (ksteps % s != 0 && run < 8) continue;
    if (post) {
      const int64_t span = run * kBK;
      int64_t most = 0;
      for (int64_t i = 0; i < s; ++i)
        most = std::max(most, (std::min((i + 1) * span, K) - 1) / G - (i * span) / G + 1);
      if (most > kGemmScaleFloats / 128) continue;
    }
    return s;
  }
  return need;
}

template <class C, int WBITS, int SD, int OD, bool EPI = false, int XD = LQ_F16>
static int launch_gemm_split(const void* X, const void* W, const void* S, void* O, int64_t M,
                             int64_t N, int64_t K, int64_t G, int splits, hipStream_t st,
                             const FixedScratch* fixed, int sd_rt = 0, int od_rt = 0) {
  // (part rows: the reduction sees the summed rows)
  const size_t mn = size_t(XD == kXPairs ? M / 2 : M) * size_t(N);
  const size_t ws_bytes = mn * sizeof(float) * size_t(splits);
  void* ws;
  if (fixed != nullptr) {   // caller-provided scratch: never allocate
    if (ws_bytes > fixed->bytes) return LQ_ERR_SCRATCH;
    ws = fixed->p;
  } else {
    ws = ws_bytes <= kSplitWsMax ? split_workspace(ws_bytes, st) : nullptr;
    if (ws == nullptr) return LQ_ERR_SHAPE;
  }
  int rc = launch_gemm_cfg<C, WBITS, SD, LQ_F32, false, XD>(X, W, S, ws, M, N, K, G, splits, st,
                                                           sd_rt);
  if (rc != LQ_OK) return rc;
  if constexpr (EPI)
    hipLaunchKernelGGL((split_reduce_silu_kernel<OD>), dim3(unsigned((mn / 2 + 255) / 256)), dim3(256),
                       0, st, static_cast<const float*>(ws), O, int64_t(mn / size_t(N)), N, splits,
                       od_rt);
  else
    hipLaunchKernelGGL((split_reduce_kernel<OD>), dim3(unsigned((mn + 1023) / 1024)), dim3(256), 0, st,
                       static_cast<const float*>(ws), O, mn, splits, od_rt);
  return check_launch();
}

// LQ_ERR_SHAPE: no configuration applies (the caller takes another kernel).
template <int WBITS, int SD, int OD, bool EPI = false, int XD = LQ_F16>
static int launch_gemm_t(const void* X, const void* W, const void* S, void* O, int64_t M,
                         int64_t N, int64_t K, int64_t G, hipStream_t st,
                         const FixedScratch* fixed = nullptr, int sd_rt = 0, int od_rt = 0) {
  if constexpr (WBITS == 4 && XD == LQ_F16 && SD != kRT && OD != kRT) {
    if (pair_applies(M, N, K, G, SD))
      return launch_gemm_pair<SD, OD, EPI>(X, W, S, O, M, N, K, G, st);
  }
  const int need = min_splits<WBITS, WBITS == 8 || XD != LQ_F16>(K, G);
  if (need == 0) return LQ_ERR_SHAPE;
  // 256-row tiles only when they alone give every CU (256) a tile; below that
  // (M <= 1024 at N = 4096) 128 x 128 tiles finish sooner, split over k when
  // they too leave CUs idle.
  const int64_t big_tiles = ((M + GemmDefault::BM - 1) / GemmDefault::BM) *
                            ((N + GemmDefault::BN - 1) / GemmDefault::BN);
  if (big_tiles >= 256) {
    if (need == 1)
      return launch_gemm_cfg<GemmDefault, WBITS, SD, OD, EPI, XD>(X, W, S, O, M, N, K, G, 1, st,
                                                                 sd_rt, od_rt);
    return launch_gemm_split<GemmDefault, WBITS, SD, OD, EPI, XD>(X, W, S, O, M, N, K, G, need, st,
                                                                  fixed, sd_rt, od_rt);
  }
  // Half the CUs or more with 256-row tiles: those tiles with k split in two
  // beat twice as many 128-row tiles (M = 1024 at N = 4096: 62.7 -> 56.9 us).
  if (big_tiles >= 128 && need <= 2 && (K / kBK) % 2 == 0 && K / kBK >= 8) {
    const int rc = launch_gemm_split<GemmDefault, WBITS, SD, OD, EPI, XD>(X, W, S, O, M, N, K, G, 2,
                                                                          st, fixed, sd_rt, od_rt);
    // no workspace, or the caller's fixed scratch too small (nothing was
    // launched): the split is optional when need == 1, so go on unsplit
    if ((rc != LQ_ERR_SHAPE && rc != LQ_ERR_SCRATCH) || need > 1) return rc;
  }
  const int64_t tiles = ((M + GemmSmall::BM - 1) / GemmSmall::BM) *
                        ((N + GemmSmall::BN - 1) / GemmSmall::BN);
  const int splits = choose_splits(tiles, K, G, need, WBITS == 8 || XD != LQ_F16);
  if (splits > 1) {
    const int rc = launch_gemm_split<GemmSmall, WBITS, SD, OD, EPI, XD>(X, W, S, O, M, N, K, G,
                                                                        splits, st, fixed, sd_rt, od_rt);
    if ((rc != LQ_ERR_SHAPE && rc != LQ_ERR_SCRATCH) || need > 1) return rc;
  }
  return launch_gemm_cfg<GemmSmall, WBITS, SD, OD, EPI, XD>(X, W, S, O, M, N, K, G, 1, st, sd_rt,
                                                           od_rt);
}

template <int WBITS>
int launch_gemm(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                int64_t K, int64_t G, int sd, int od, hipStream_t st, const FixedScratch* fixed) {
#define LQ_GM(SD_, OD_) \
  if (sd == SD_ && od == OD_) return launch_gemm_t<WBITS, SD_, OD_>(X, W, S, O, M, N, K, G, st, fixed)
  LQ_GM(LQ_F16, LQ_F16);
  LQ_GM(LQ_F16, LQ_F32);
  LQ_GM(LQ_F16, LQ_BF16);
  LQ_GM(LQ_F32, LQ_F16);
  LQ_GM(LQ_F32, LQ_F32);
  LQ_GM(LQ_F32, LQ_BF16);
  LQ_GM(LQ_BF16, LQ_F16);
  LQ_GM(LQ_BF16, LQ_F32);
  LQ_GM(LQ_BF16, LQ_BF16);
#undef LQ_GM
  return LQ_ERR_DTYPE;
}

// Decode-sized M (16 < M <= 64) on the split-K GEMM, for the callers whose
// shapes it serves faster than the decode kernels (few 128-column tiles, long
// rows): only when the k split applies (>= 2 splits and their workspace or
// the caller's fixed scratch at hand); LQ_ERR_SHAPE otherwise, so the caller
// takes its decode kernel instead of an unsplit GEMM of a few tiles.
template <int WBITS>
int launch_gemm_split_only(const void* X, const void* W, const void* S, void* O, int64_t M,
                           int64_t N, int64_t K, int64_t G, int sd, int od, hipStream_t st,
                           const FixedScratch* fixed) {
  const int need = min_splits<WBITS>(K, G);
  if (need == 0 || K % kBK != 0) return LQ_ERR_SHAPE;
  const int64_t tiles = ((M + GemmSmall::BM - 1) / GemmSmall::BM) *
                        ((N + GemmSmall::BN - 1) / GemmSmall::BN);
  const int splits = choose_splits(tiles, K, G, need, WBITS == 8);
  if (splits < 2) return LQ_ERR_SHAPE;
  int rc = LQ_ERR_DTYPE;
#define LQ_GSO(SD_, OD_)                                                                  \
  if (sd == SD_ && od == OD_)                                                             \
    rc = launch_gemm_split<GemmSmall, WBITS, SD_, OD_>(X, W, S, O, M, N, K, G, splits, st, fixed)
  LQ_GSO(LQ_F16, LQ_F16);
  LQ_GSO(LQ_F16, LQ_F32);
  LQ_GSO(LQ_F16, LQ_BF16);
  LQ_GSO(LQ_F32, LQ_F16);
  LQ_GSO(LQ_F32, LQ_F32);
  LQ_GSO(LQ_F32, LQ_BF16);
  LQ_GSO(LQ_BF16, LQ_F16);
  LQ_GSO(LQ_BF16, LQ_F32);
  LQ_GSO(LQ_BF16, LQ_BF16);
#undef LQ_GSO
  // (no launch happened for a workspace that is missing or too small)
  return rc == LQ_ERR_SCRATCH ? LQ_ERR_SHAPE : rc;
}
template int launch_gemm_split_only<4>(const void*, const void*, const void*, void*, int64_t,
                                       int64_t, int64_t, int64_t, int, int, hipStream_t,
                                       const FixedScratch*);
template int launch_gemm_split_only<8>(const void*, const void*, const void*, void*, int64_t,
                                       int64_t, int64_t, int64_t, int, int, hipStream_t,
                                       const FixedScratch*);

// O [M, N] (od) = the sum of `splits` fp32 partial slices P [splits][M][N]
// (silu: O [M, N / 2] = silu(sum[:, 2i]) * sum[:, 2i + 1]).
int launch_split_reduce(const float* P, void* O, int64_t M, int64_t N, int splits, bool silu,
                        int od, hipStream_t st) {
  const size_t mn = size_t(M) * size_t(N);
  if (silu)
    hipLaunchKernelGGL((split_reduce_silu_kernel<kRT>), dim3(unsigned((mn / 2 + 255) / 256)), dim3(256),
                       0, st, P, O, M, N, splits, od);
  else
    hipLaunchKernelGGL((split_reduce_kernel<kRT>), dim3(unsigned((mn + 1023) / 1024)), dim3(256), 0, st,
                       P, O, mn, splits, od);
  return check_launch();
}

// O [M, N / 2] = silu(P[:, 2i]) * P[:, 2i + 1] for an fp32 matvec result P.
int launch_silu_pairs(const float* P, void* O, int64_t M, int64_t N, int od, hipStream_t st) {
  const unsigned blocks = unsigned((M * (N / 2) + 255) / 256);
  if (od == LQ_F16)
    hipLaunchKernelGGL((split_reduce_silu_kernel<LQ_F16>), dim3(blocks), dim3(256), 0, st, P, O, M, N, 1);
  else if (od == LQ_F32)
    hipLaunchKernelGGL((split_reduce_silu_kernel<LQ_F32>), dim3(blocks), dim3(256), 0, st, P, O, M, N, 1);
  else
    hipLaunchKernelGGL((split_reduce_silu_kernel<LQ_BF16>), dim3(blocks), dim3(256), 0, st, P, O, M, N, 1);
  return check_launch();
}

// Gate|up prefill with the SiLU * mul epilogue (int4, N = 2 I interleaved rows).
int launch_gemm_silu(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                     int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  if (G % 32 != 0) return LQ_ERR_SHAPE;
#define LQ_GS(SD_, OD_) \
  if (sd == SD_ && od == OD_) return launch_gemm_t<4, SD_, OD_, true>(X, W, S, O, M, N, K, G, st)
  LQ_GS(LQ_F16, LQ_F16);
  LQ_GS(LQ_F16, LQ_F32);
  LQ_GS(LQ_F32, LQ_F16);
  LQ_GS(LQ_F32, LQ_F32);
#undef LQ_GS
  return LQ_ERR_SHAPE;
}

// bf16 activations: bf16 MFMAs on exact integer weights, fp32 group scales
// (groups of whole 64-k steps); scale / output dtypes at run time.
template <int WBITS>
int launch_gemm_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                  int64_t K, int64_t G, int xd, int sd, int od, hipStream_t st,
                  const FixedScratch* fixed) {
  if (xd != LQ_BF16 || G % (kBK / 2) != 0) return LQ_ERR_SHAPE;
  return launch_gemm_t<WBITS, kRT, kRT, false, LQ_BF16>(X, W, S, O, M, N, K, G, st, fixed, sd, od);
}
// fp32 activations as bf16 part rows P [2 M, K] (rows 2i, 2i + 1 = the two
// parts of row i): the bf16 GEMM on 2 M rows with the pair sum in its
// epilogue, O [M, N] (od; EPI: gate/up rows interleaved, O [M, N / 2]).
// M2 = 2 M.
template <int WBITS, bool EPI>
int launch_gemm_pairs(const void* P, const void* W, const void* S, void* O, int64_t M2, int64_t N,
                      int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  if (M2 % 2 != 0 || G % (kBK / 2) != 0 || K % kBK != 0) return LQ_ERR_SHAPE;
  return launch_gemm_t<WBITS, kRT, kRT, EPI, kXPairs>(P, W, S, O, M2, N, K, G, st, nullptr, sd, od);
}
template int launch_gemm_pairs<4, false>(const void*, const void*, const void*, void*, int64_t,
                                         int64_t, int64_t, int64_t, int, int, hipStream_t);
template int launch_gemm_pairs<8, false>(const void*, const void*, const void*, void*, int64_t,
                                         int64_t, int64_t, int64_t, int, int, hipStream_t);
template int launch_gemm_pairs<4, true>(const void*, const void*, const void*, void*, int64_t,
                                        int64_t, int64_t, int64_t, int, int, hipStream_t);

// Gate|up prefill with bf16 activations and the SiLU * mul epilogue (int4,
// N = 2 I interleaved rows; scale / output dtypes at run time).
int launch_gemm_silu_x(const void* X, const void* W, const void* S, void* O, int64_t M, int64_t N,
                       int64_t K, int64_t G, int sd, int od, hipStream_t st) {
  if (G % (kBK / 2) != 0 || K % kBK != 0) return LQ_ERR_SHAPE;
  return launch_gemm_t<4, kRT, kRT, true, LQ_BF16>(X, W, S, O, M, N, K, G, st, nullptr, sd, od);
}

template int launch_gemm_x<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, int, hipStream_t, const FixedScratch*);
template int launch_gemm_x<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                              int64_t, int64_t, int, int, int, hipStream_t, const FixedScratch*);

template int launch_gemm<4>(const void*, const void*, const void*, void*, int64_t, int64_t,
                            int64_t, int64_t, int, int, hipStream_t, const FixedScratch*);
template int launch_gemm<8>(const void*, const void*, const void*, void*, int64_t, int64_t,
                            int64_t, int64_t, int, int, hipStream_t, const FixedScratch*);

}  // namespace lq
