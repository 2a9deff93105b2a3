// MFMA operand traits (TileMfma) by weight bits and activation dtype.
// Part of the decode GEMV kernels; see gemv_impl.h for the kernel choice.
#pragma once
#include "gemv_common.h"

namespace lq {

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
// int8 -> four bf16 q, k order kept (exact: at most 8 significant bits, so
// the float's low half is 0).
__device__ __forceinline__ u32x2_t int8x4_to_bf16(uint32_t w) {
  const float f0 = float(int8_t(w)), f1 = float(int8_t(w >> 8));
  const float f2 = float(int8_t(w >> 16)), f3 = float(int8_t(w >> 24));
  u32x2_t r;
  r.x = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
  r.y = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
  return r;
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
  // the same for part `part` of the two-way round-to-nearest split
  __device__ static op_t prep_x2(const x_t& x, int part) {
    uint32_t b[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] = f32_rn2_part_bits(x[i], part);
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

}  // namespace lq
