// The per-element arithmetic of the SiLU-and-mul producer, shared by the producer kernels and the
// one-launch SiLU-mul linear (whose quantizing waves compute the same bf16 stage), so both give
// the same bits. Every function turns off contraction of multiply-adds in its own body: each
// product and sum rounds, except the explicit fused multiply-adds. exp is exp_f32 below:
// Cody-Waite reduction by ln 2 (Cody and Waite, "Software Manual for the Elementary Functions",
// 1980; ln 2 split into a 16-bit head and a tail) and the degree-7 Taylor polynomial of e^r on
// |r| <= ln2 / 2 by Horner, the reduction and each Horner step one fused multiply-add, then an
// exact scaling by 2^n. Rounding to bf16 is round to nearest even with NaN -> 0x7FC0 | sign.
#pragma once
#include "w4a8_internal.h"

namespace w4a8 {
namespace prod {

constexpr float kLog2e = 0x1.715476p+0f;         // fl32(log2 e)
constexpr float kLn2Hi = 0x1.62e4p-1f;            // 16 significant bits: n * kLn2Hi is exact
constexpr float kLn2Lo = 0x1.7f7d1cp-20f;         // ln 2 - kLn2Hi, rounded to fp32
constexpr float kExpHi = 0x1.62e43p+6f;           // 88.7228394: above, e^y overflows fp32
constexpr float kExpLo = -0x1.9fe368p+6f;         // fl32(-150 ln 2): below, e^y rounds to +0
static_assert(kExpHi < 89.0f && kExpLo > -104.0f, "exp_f32's clamp must bracket its range");

// e^y for y in [kExpLo, kExpHi] as described above; above kExpHi it is +inf and below kExpLo +0.
// Branch-free: y is first clamped to [-104, 89], where the same steps already give +inf at and
// above kExpHi (n = 128 and e^r > 1) and +0 below kExpLo (p * 2^-150 < 2^-150 rounds to zero).
// Over all non-NaN inputs this equals the branching form bit for bit (checked on the CPU with the
// same operations). A NaN input gives a finite value (the clamp returns a bound): silu8, the only
// caller, sends every group holding a NaN down its dividing path, where x / d is x's NaN for any
// d, as the exp that kept the NaN gave.
__device__ __forceinline__ float exp_f32(float y) {
#pragma clang fp contract(off)
  // the clamp as one v_med3_f32: fminf(fmaxf()) would first canonicalize y, one more operation
  // per element; for every non-NaN y both are the same clamp
  y = __builtin_amdgcn_fmed3f(y, -104.0f, 89.0f);
  const float n = rintf(y * kLog2e);
  const float r = __builtin_fmaf(-n, kLn2Lo, __builtin_fmaf(-n, kLn2Hi, y));
  float p = 0x1.a01a02p-13f;                      // 1/k!, k = 7 .. 2, rounded to fp32
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

// silu of 8 values, x / (1 + exp_f32(-x)) with the IEEE quotient. Where every value of the group
// has |x| <= 44 (1 <= d <= 2^64: the reciprocal is a normal number, nothing is infinite or NaN)
// the quotient comes from the hardware reciprocal and one Markstein correction, y = rcp(d),
// q = x y, the residual formed negated, r = fma(d, q, -x), then fma(-r, y, q): four operations
// instead of the division's ten (the same value as q + (x - d q) y, and -0 for x = -0 with no
// sign fix). Any other group (rare) divides. Markstein's
// correction is proven correctly rounded only from a correctly rounded reciprocal, and v_rcp_f32
// is within 1 ulp, so the unrounded quotient is checked on the GPU instead, against the IEEE
// quotient for every bf16 x on both paths (w4a8_silu_f32; the SiLU-and-mul and gated-norm tests
// also run every bf16 gate through the producers themselves).
__device__ __forceinline__ void silu8(const float (&x)[8], float (&s)[8]) {
#pragma clang fp contract(off)
  float d[8];
  bool wide = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    d[j] = 1.0f + exp_f32(-x[j]);
    const float y = __builtin_amdgcn_rcpf(d[j]);
    const float q = x[j] * y;
    const float r = __builtin_fmaf(d[j], q, -x[j]);
    s[j] = __builtin_fmaf(-r, y, q);
    wide |= !(__builtin_fabsf(x[j]) <= 44.0f);
  }
  if (__builtin_expect(wide, 0)) {
#pragma unroll
    for (int j = 0; j < 8; ++j) s[j] = x[j] / d[j];
  }
}

// Round to bf16 with the hardware convert (v_cvt_pk_bf16_f32, round to nearest even, the same
// bits as f32_to_bf16 for every non-NaN input, subnormals included); a NaN keeps its payload.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t cvt_bf16x2(float lo, float hi) {
#pragma clang fp contract(off)
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
// for an intermediate whose NaNs only ever reach the canonicalizing pack below
__device__ __forceinline__ float bf16_round_hw(float x) { return (float)(__bf16)x; }

__device__ __forceinline__ void unpack8(const uint4 v, float (&f)[8]) {
#pragma clang fp contract(off)
  f[0] = __uint_as_float(v.x << 16); f[1] = __uint_as_float(v.x & 0xFFFF0000u);
  f[2] = __uint_as_float(v.y << 16); f[3] = __uint_as_float(v.y & 0xFFFF0000u);
  f[4] = __uint_as_float(v.z << 16); f[5] = __uint_as_float(v.z & 0xFFFF0000u);
  f[6] = __uint_as_float(v.w << 16); f[7] = __uint_as_float(v.w & 0xFFFF0000u);
}

// software rounding, NaN -> 0x7FC0 | sign
__device__ __forceinline__ uint4 pack8_sw(const float (&f)[8]) {
#pragma clang fp contract(off)
  return make_uint4(f32_to_bf16(f[0]) | (f32_to_bf16(f[1]) << 16),
                    f32_to_bf16(f[2]) | (f32_to_bf16(f[3]) << 16),
                    f32_to_bf16(f[4]) | (f32_to_bf16(f[5]) << 16),
                    f32_to_bf16(f[6]) | (f32_to_bf16(f[7]) << 16));
}

// pack8 with the hardware convert: two values per operation. A group holding a NaN (rare) takes
// the software rounding, whose NaNs are canonical (0x7FC0 | sign).
__device__ __forceinline__ uint4 pack8_hw(const float (&f)[8]) {
#pragma clang fp contract(off)
  bool nan = false;
#pragma unroll
  for (int j = 0; j < 8; ++j) nan |= f[j] != f[j];
  if (__builtin_expect(nan, 0)) return pack8_sw(f);
  return make_uint4(cvt_bf16x2(f[0], f[1]), cvt_bf16x2(f[2], f[3]), cvt_bf16x2(f[4], f[5]),
                    cvt_bf16x2(f[6], f[7]));
}

// SiLU-and-mul of one 8-element group: bf16(bf16(silu(gate)) * up).
__device__ __forceinline__ uint4 silu_mul_group(const uint4 gv, const uint4 uv) {
#pragma clang fp contract(off)
  float a[8], b[8], sg[8], p[8];
  unpack8(gv, a);
  unpack8(uv, b);
  silu8(a, sg);
#pragma unroll
  for (int j = 0; j < 8; ++j) p[j] = bf16_round_hw(sg[j]) * b[j];
  return pack8_hw(p);
}

}  // namespace prod
}  // namespace w4a8
