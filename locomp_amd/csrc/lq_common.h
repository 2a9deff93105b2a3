// Shared device helpers for the gfx950 int4/int8 weight-only kernels.
//
// Weight formats (identical to locomp's examples 38 and 52):
//   int4: uint8 [N, K/2]; byte j of row n holds k = 2j in the low nibble and
//         k = 2j + 1 in the high nibble; w = (q - 8) * s[n, k / G].
//   int8: int8 [N, K];  w = q * s[n, k / G].
//   scales: [N, K/G] row-major (fp32 or fp16); G = K is per-output-channel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/locomp_amd.h"

namespace lq {

typedef _Float16 half_t;
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- dtypes --

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
  return __uint_as_float(uint32_t(b) << 16);
}

// Round-to-nearest-even fp32 -> bf16 (NaN stays a quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}

// Materialises an fp32 value in a register.  The reference rounds the
// dequantised product to fp32 and then to the output dtype; without this the
// compiler may fold fmul + fptrunc into one mixed-precision FMA (a single
// rounding straight to fp16), which is not bit-identical.
__device__ __forceinline__ float round_f32(float v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}

template <int DT> struct Elem;
template <> struct Elem<LQ_F32>  { typedef float    T; };
template <> struct Elem<LQ_F16>  { typedef half_t   T; };
template <> struct Elem<LQ_BF16> { typedef uint16_t T; };

template <int DT>
__device__ __forceinline__ float load_f32(const void* p, size_t i) {
  if constexpr (DT == LQ_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == LQ_F16) return float(static_cast<const half_t*>(p)[i]);
  else return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void store_f32(void* p, size_t i, float v) {
  if constexpr (DT == LQ_F32) static_cast<float*>(p)[i] = v;
  else if constexpr (DT == LQ_F16) static_cast<half_t*>(p)[i] = half_t(v);
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

// Scale / output dtype given at run time (the kernel's sd / od arguments):
// the instantiations for bf16 and fp32 activations use it to bound their
// number.
constexpr int kRT = -1;
// Activation code of the decode tile kernel for fp32 activations split
// beforehand into their three exact bf16 parts: a bf16 matrix of 12 rows,
// row m + 4 part = part `part` of activation row m (M <= 4).
constexpr int kXPre = 100;
// Activation code of the decode kernels and the prefill GEMM for fp32
// activations split beforehand into two round-to-nearest bf16 parts, rows
// 2i (hi) and 2i + 1 (lo) of a bf16 matrix of 2 M rows (the kernels' M):
// the MFMA output rows 4q + r and 4q + r + 1 sit in one lane, so the store
// adds each pair and writes output row i.
constexpr int kXPairs = 101;
template <int SD>
__device__ __forceinline__ int scale_size(int sd_rt) {
  const int sd = SD == kRT ? sd_rt : SD;
  return sd == LQ_F32 ? 4 : 2;
}
template <int SD>
__device__ __forceinline__ float load_scale(const uint8_t* p, int sd_rt) {
  const int sd = SD == kRT ? sd_rt : SD;
  if (sd == LQ_F32) return *reinterpret_cast<const float*>(p);
  if (sd == LQ_F16) return float(*reinterpret_cast<const half_t*>(p));
  return bf16_to_f32(*reinterpret_cast<const uint16_t*>(p));
}
template <int OD>
__device__ __forceinline__ void store_out(void* O, size_t i, float v, int od_rt) {
  if constexpr (OD != kRT) {
    store_f32<OD>(O, i, v);
  } else {
    if (od_rt == LQ_F32) store_f32<LQ_F32>(O, i, v);
    else if (od_rt == LQ_F16) store_f32<LQ_F16>(O, i, v);
    else store_f32<LQ_BF16>(O, i, v);
  }
}

// Element i of a scale array of dtype SD (kRT: sd_rt), as fp32.
template <int SD>
__device__ __forceinline__ float load_f32_rt(const void* p, size_t i, int sd_rt) {
  const int sd = SD == kRT ? sd_rt : SD;
  if (sd == LQ_F32) return static_cast<const float*>(p)[i];
  if (sd == LQ_F16) return float(static_cast<const half_t*>(p)[i]);
  return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// ------------------------------------------------------ bit-level unpack --

__device__ __forceinline__ uint32_t as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }
__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }

// One packed int4 dword (8 weights, k0..k7 in order) -> four half2 holding
// (q - 8) for (k0,k1), (k2,k3), (k4,k5), (k6,k7), exactly.
// Byte p is replicated into bytes 0 and 2 (v_perm_b32), masked to its low
// nibble at bits 3:0 and its high nibble at bits 23:20, and OR-ed with
// 0x6400 (1024.0h) in each half.  The low half is then 1024 + q_even and the
// high half 1024 + 16 * q_odd, both exact in fp16.  One packed FMA
// h * (1, 1/16) + (-1032, -72) maps both to q - 8 exactly (the products are
// exact and the sum is representable, so the single rounding is exact).
// `magic` = 0x64006400 (an opaque register value lets the mask and the OR
// issue as one v_and_or_b32; with two literal constants they take two ops).
__device__ __forceinline__ half2_t int4_pair_to_h2(uint32_t w, int p, uint32_t magic) {
  const half2_t mul = {half_t(1.0f), half_t(0.0625f)};
  const half2_t add = {half_t(-1032.0f), half_t(-72.0f)};
  const uint32_t sel = 0x00000000u | uint32_t(p) | (uint32_t(p) << 16);
  const uint32_t u = __builtin_amdgcn_perm(w, w, sel);
  const uint32_t t = (u & 0x00F0000Fu) | magic;
  return __builtin_elementwise_fma(as_h2(t), mul, add);
}

__device__ __forceinline__ void int4x8_to_h2(uint32_t w, half2_t out[4], uint32_t magic) {
#pragma unroll
  for (int p = 0; p < 4; ++p) out[p] = int4_pair_to_h2(w, p, magic);
}
__device__ __forceinline__ void int4x8_to_h2(uint32_t w, half2_t out[4]) {
  int4x8_to_h2(w, out, 0x64006400u);
}

// Two int8 weights (bytes 2p, 2p+1 of w) -> half2 exact: (b ^ 0x80) in the
// low mantissa byte of 1024.0h gives 1024 + b + 128; subtract 1152.
__device__ __forceinline__ void int8x4_to_h2(uint32_t w, half2_t out[2]) {
  const half2_t off = {half_t(1152.0f), half_t(1152.0f)};
  const uint32_t x = w ^ 0x80808080u;
  // v_perm_b32 byte selectors: 0..3 pick from the 2nd operand (x), 4..7 from
  // the 1st (0x64646464).  lo = bytes {b0', 0x64, b1', 0x64} (LSB first).
  const uint32_t lo = __builtin_amdgcn_perm(0x64646464u, x, 0x04010400u);
  const uint32_t hi = __builtin_amdgcn_perm(0x64646464u, x, 0x04030402u);
  out[0] = as_h2(lo) - off;
  out[1] = as_h2(hi) - off;
}


// ------------------------------------ biased, k-permuted unpack (MFMA B) --
// For MFMA consumers the order of k inside an 8-wide group is free as long as
// the A operand uses the same order.  These helpers emit, for one group of 8
// weights k0..k7, the four half2 (k0,k4), (k1,k5), (k2,k6), (k3,k7) *biased*:
// each half is the fp16 value BIAS + q exactly, with BIAS = 1032 for int4
// (1024 + q, q = 0..15, stands for q - 8) and 1152 for int8 (1024 + (b ^ 0x80)
// stands for b).  Callers subtract BIAS * sum(x) once per k-range instead of
// once per weight.  xperm8 applies the same permutation to 8 activations.

// (x & mask) | orv.  Written in C (not inline asm) so the compiler's hazard
// tracking sees the VALU write when the result feeds an MFMA; `orv` should be
// an opaque_u32 value so the pair is selected as one v_and_or_b32 (mask in an
// SGPR, orv in a VGPR) rather than v_and + v_or with two literals.
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t mask, uint32_t orv) {
  return (x & mask) | orv;
}

// a / d for 0 <= a < 2^22 and d >= 1, given rd = 1.0f / d.  The float
// product is within 0.75 of a / d (two roundings of at most 2^-24 relative
// each, a / d < 2^22), so its truncation is off by at most one, and the
// remainder test corrects that.  A few VALU ops instead of the integer
// division sequence.
__device__ __forceinline__ int div_rcp(int a, int d, float rd) {
  int q = int(float(a) * rd);
  const int r = a - q * d;
  q += r >= d ? 1 : 0;
  q -= r < 0 ? 1 : 0;
  return q;
}

// v of the lane N below in the same 16-lane row (DPP row_shr:N), 0 for the
// row's first N lanes.
template <int N>
__device__ __forceinline__ float dpp_row_shr(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                               0x110 + N, 0xF, 0xF, true));
}

// A value the optimiser cannot constant-fold (held in a VGPR).
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  __asm__ volatile("" : "+v"(v));
  return v;
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

// Part `part` (0 hi, 1 lo) of the two-way bf16 split of fp32 x with round to
// nearest even: hi = RN(x), lo = RN(x - hi) (x - hi is exact in fp32), as the
// bf16 bit pattern in the high half of the returned dword.  |x - hi - lo| <=
// 2^-16 |x|; at |x| >= 2^127 hi is truncated instead (RN could round to inf).
__device__ __forceinline__ uint32_t f32_rn2_part_bits(uint32_t x, int part) {
  const uint32_t rn = (x + 0x7FFFu + ((x >> 16) & 1u)) & 0xFFFF0000u;
  const uint32_t hi = (x & 0x7F000000u) == 0x7F000000u ? x & 0xFFFF0000u : rn;
  if (part == 0) return hi;
  const uint32_t r = __float_as_uint(__uint_as_float(x) - __uint_as_float(hi));
  return (r + 0x7FFFu + ((r >> 16) & 1u)) & 0xFFFF0000u;
}

constexpr float kInt4Bias = 1032.0f;
constexpr float kInt8Bias = 1152.0f;

// int4: one dword = 8 weights.  (w >> 4i) & 0x000F000F puts nibble i of byte 0
// (k = i) in bits 3:0 and nibble i of byte 2 (k = i + 4) in bits 19:16.
__device__ __forceinline__ u32x4_t int4x8_biased_kperm(uint32_t w) {
  const uint32_t magic = opaque_u32(0x64006400u);
  u32x4_t r;
  r.x = and_or(w, 0x000F000Fu, magic);         // (k0, k4)
  r.y = and_or(w >> 4, 0x000F000Fu, magic);    // (k1, k5)
  r.z = and_or(w >> 8, 0x000F000Fu, magic);    // (k2, k6)
  r.w = and_or(w >> 12, 0x000F000Fu, magic);   // (k3, k7)
  return r;
}

// The same with the OR mask as an argument (0x43004300 gives bf16 128 + q).
__device__ __forceinline__ u32x4_t int4x8_biased_kperm_m(uint32_t w, uint32_t magic) {
  u32x4_t r;
  r.x = and_or(w, 0x000F000Fu, magic);
  r.y = and_or(w >> 4, 0x000F000Fu, magic);
  r.z = and_or(w >> 8, 0x000F000Fu, magic);
  r.w = and_or(w >> 12, 0x000F000Fu, magic);
  return r;
}

// int8: two dwords = 8 weights.  Pair i takes byte i of each dword; the xor
// flips the sign bit (b + 128) and writes the 0x64 exponent byte at once.
__device__ __forceinline__ u32x4_t int8x8_biased_kperm(uint32_t w0, uint32_t w1) {
  u32x4_t r;
  r.x = __builtin_amdgcn_perm(w1, w0, 0x0C040C00u) ^ 0x64806480u;
  r.y = __builtin_amdgcn_perm(w1, w0, 0x0C050C01u) ^ 0x64806480u;
  r.z = __builtin_amdgcn_perm(w1, w0, 0x0C060C02u) ^ 0x64806480u;
  r.w = __builtin_amdgcn_perm(w1, w0, 0x0C070C03u) ^ 0x64806480u;
  return r;
}

// 8 fp16 activations x0..x7 (4 dwords) -> (x0,x4), (x1,x5), (x2,x6), (x3,x7).
__device__ __forceinline__ u32x4_t xperm8(u32x4_t d) {
  u32x4_t r;
  r.x = __builtin_amdgcn_perm(d.z, d.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(d.z, d.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(d.w, d.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(d.w, d.y, 0x07060302u);
  return r;
}

// ---------------------------------------------------------------- launch --

// Device memory a caller lends the split-K prefill instead of the per-stream
// workspace (which allocates): p holds `bytes` bytes.
struct FixedScratch {
  void* p;
  size_t bytes;
};
// Size of the fixed split-K scratch array behind the _noalloc entry point:
// enough for the splits chosen at M <= 512 x N <= 4096 (and M <= 128 x
// N <= 16384); larger splits are rejected with LQ_ERR_SCRATCH.
constexpr size_t kStaticScratchBytes = size_t(32) << 20;
// Per-device address of that array (looked up once per device).
int static_scratch(void** ptr);

__host__ __forceinline__ int check_launch() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? LQ_OK : int(e);
}

// ------------------------------------------------------ explicit loads --
// Global loads issued with inline asm, for kernels that place every vmcnt
// wait by hand (the compiler does not count asm loads, and it treats an
// LDS-DMA as a write to all of LDS).  A register written by one of these
// must not be read before an asm wait that names it.  dma16 uses M0.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// 16 bytes per lane from global memory to LDS (lane L -> lds + 16 L).
__device__ __forceinline__ void dma16(const void* g, const void* lds) {
  const uint32_t a = __builtin_amdgcn_readfirstlane(lds_addr(lds));
  __asm__ volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                   :: "v"(g), "s"(a) : "memory", "m0");
}
// 16 bytes per lane from a raw buffer (byte offset voff + soff, soff
// wave-uniform) to LDS (lane L -> lds + 16 L); bytes past the buffer read as 0.
// (lds: the LDS byte address, wave-uniform)
__device__ __forceinline__ void dma16_so(i32x4_t rsrc, uint32_t voff, uint32_t soff,
                                         uint32_t lds) {
  const uint32_t a = __builtin_amdgcn_readfirstlane(lds);
  __asm__ volatile("s_mov_b32 m0, %3\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                   :: "v"(voff), "s"(rsrc), "s"(soff), "s"(a) : "memory", "m0");
}
__device__ __forceinline__ u32x4_t gload_b128(const void* g) {
  u32x4_t v;
  __asm__ volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(v) : "v"(g) : "memory");
  return v;
}
__device__ __forceinline__ u32x2_t gload_b64(const void* g) {
  u32x2_t v;
  __asm__ volatile("global_load_dwordx2 %0, %1, off nt" : "=v"(v) : "v"(g) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t gload_u16(const void* g) {
  uint32_t v;
  __asm__ volatile("global_load_ushort %0, %1, off" : "=v"(v) : "v"(g) : "memory");
  return v;
}
__device__ __forceinline__ uint32_t gload_b32(const void* g) {
  uint32_t v;
  __asm__ volatile("global_load_dword %0, %1, off" : "=v"(v) : "v"(g) : "memory");
  return v;
}

__device__ __forceinline__ u32x4_t gload_b128_cached(const void* g) {
  u32x4_t v;
  __asm__ volatile("global_load_dwordx4 %0, %1, off" : "=v"(v) : "v"(g) : "memory");
  return v;
}
}  // namespace lq
