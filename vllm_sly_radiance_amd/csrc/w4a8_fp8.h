// Per-token e4m3 quantization of bf16 rows held in registers, shared by the quantizer and the
// fused producers. Semantics: s = max(amax(|x|) * fl32(1/448), 1/(448*512)) (a NaN in the row
// propagates to s); q = e4m3_rne(clamp(x / s, -448, 448)) with the IEEE fp32 quotient x / s. One
// workgroup per row (of 256 threads; of 512 or 1024 where few rows leave each row's chain as the
// latency); the amax runs on the bf16 bit patterns (|x| bits = x & 0x7FFF), which is exact,
// orders like the magnitudes and ranks NaN above inf. Codes come
// from the hardware e4m3 converter (v_cvt_pk_fp8_f32, round to nearest even) on clamped inputs;
// rows whose scale is not finite take a per-element path that maps NaN quotients to 0x7F.
//
// Rows with a finite scale divide by Markstein's correction (P. Markstein, "Computation of
// elementary functions on the IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1), 1990):
// y = 1/s once per row (IEEE division), then per element q0 = x*y, the residual formed negated,
// r = fma(s, q0, -x), and q = fma(-r, y, q0): three operations instead of a full division (the
// same value as q0 + (x - s q0) y, round to nearest being symmetric, and -0 for x = -0 with no
// sign fix, where fma(x - s q0, y, q0) would give +0). Over every
// finite row amax and every bf16 x with |x| <= amax (both signs, 1.07e9 pairs) the result equals
// the IEEE quotient except for quotients below 2^-12, where both round to the same signed zero in
// e4m3 (tests/fp_identities.c, run by tests/test_fp_identities_cpu.py, makes that exhaustive
// check).
#pragma once
#include "w4a8_internal.h"

namespace w4a8 {
namespace fp8 {

constexpr int kThreads = 256;
constexpr float kInv448 = 1.0f / 448.0f;            // fl32(1/448), folded at compile time
constexpr float kMinScale = 1.0f / (448.0f * 512.0f);

// Cross-lane exchange for xor butterflies, in registers (no LDS round trip per step).
//  * lane ^ 32 and lane ^ 16: v_permlane32_swap / v_permlane16_swap with both operands v leave
//    each lane holding its own value in one result and its partner's in the other, so the step
//    combines the pair (a sum is exact in either operand order, as a + b == b + a);
//  * lane ^ 8, 4, 2, 1: DPP moves within rows of 16 lanes: quad_perm [1,0,3,2] (^1),
//    [2,3,0,1] (^2); half-row mirror then quad_perm [3,2,1,0] (^4); row mirror then half-row
//    mirror (^8).
// Every lane of the wave must be active where these run (a read from an inactive lane returns 0
// or a stale value): callers pass a neutral value from lanes that hold nothing instead of
// branching around the call.
template <int Ctrl>
__device__ __forceinline__ uint32_t dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, Ctrl, 0xF, 0xF, false);
}

// The value lane (l ^ O) holds, O in {1, 2, 4, 8}.
template <int O>
__device__ __forceinline__ uint32_t xor_lane(uint32_t v) {
  static_assert(O == 1 || O == 2 || O == 4 || O == 8, "within a row of 16 lanes");
  if constexpr (O == 1) return dpp<0xB1>(v);
  else if constexpr (O == 2) return dpp<0x4E>(v);
  else if constexpr (O == 4) return dpp<0x1B>(dpp<0x141>(v));
  else return dpp<0x141>(dpp<0x140>(v));
}

// {own, partner} for partner lane l ^ 32 (Half = 32) or l ^ 16 (Half = 16), in some order.
template <int Half>
__device__ __forceinline__ uint2 swap_pair(uint32_t v) {
  static_assert(Half == 16 || Half == 32, "lane halves");
  if constexpr (Half == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return make_uint2(r[0], r[1]);
  } else {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return make_uint2(r[0], r[1]);
  }
}

// Wave-wide max by an xor butterfly (every lane gets it).
__device__ __forceinline__ uint32_t wave_max(uint32_t v) {
  uint2 p = swap_pair<32>(v);
  v = max(p.x, p.y);
  p = swap_pair<16>(v);
  v = max(p.x, p.y);
  v = max(v, xor_lane<8>(v));
  v = max(v, xor_lane<4>(v));
  v = max(v, xor_lane<2>(v));
  return max(v, xor_lane<1>(v));
}

// Wave-wide sum in the fixed xor-butterfly order 32, 16, 8, 4, 2, 1: at each step every lane
// adds its value and lane (l ^ o)'s, so every lane ends with the same, reproducible sum.
__device__ __forceinline__ float wave_sum_xor(float v) {
  uint2 p = swap_pair<32>(__float_as_uint(v));
  v = __uint_as_float(p.x) + __uint_as_float(p.y);
  p = swap_pair<16>(__float_as_uint(v));
  v = __uint_as_float(p.x) + __uint_as_float(p.y);
  v = v + __uint_as_float(xor_lane<8>(__float_as_uint(v)));
  v = v + __uint_as_float(xor_lane<4>(__float_as_uint(v)));
  v = v + __uint_as_float(xor_lane<2>(__float_as_uint(v)));
  return v + __uint_as_float(xor_lane<1>(__float_as_uint(v)));
}

// Row-wide max over a workgroup of T threads (all threads get the result).
template <int T>
__device__ __forceinline__ uint32_t block_max_t(uint32_t v) {
  static_assert(T % 64 == 0 && T >= 64 && T <= 1024, "threads");
  __shared__ uint32_t red[T / 64];
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t m = red[0];
#pragma unroll
  for (int i = 1; i < T / 64; ++i) m = max(m, red[i]);
  return m;
}

__device__ __forceinline__ uint32_t block_max(uint32_t v) { return block_max_t<kThreads>(v); }

__device__ __forceinline__ uint32_t abs_bits_max8(const uint4 v) {
  uint32_t m = max(v.x & 0x7FFFu, (v.x >> 16) & 0x7FFFu);
  m = max(m, max(v.y & 0x7FFFu, (v.y >> 16) & 0x7FFFu));
  m = max(m, max(v.z & 0x7FFFu, (v.z >> 16) & 0x7FFFu));
  return max(m, max(v.w & 0x7FFFu, (v.w >> 16) & 0x7FFFu));
}

__device__ __forceinline__ float clamp448(float v) {
  v = v > 448.0f ? 448.0f : v;                       // comparisons keep NaN
  return v < -448.0f ? -448.0f : v;
}

// clamp448 for a quotient that cannot be NaN: one v_med3_f32 instead of two compare-and-selects.
// With a finite row scale every element of the row is finite (a NaN or inf would have made the
// row's amax, and so its scale, non-finite), and so is every quotient.
__device__ __forceinline__ float clamp448_finite(float v) {
  return __builtin_amdgcn_fmed3f(v, -448.0f, 448.0f);
}

__device__ __forceinline__ float lo_bf16(uint32_t d) { return __uint_as_float(d << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t d) { return __uint_as_float(d & 0xFFFF0000u); }

// four quotients -> four e4m3 bytes (little-endian order: first value in byte 0)
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

__device__ __forceinline__ uint32_t code1(float v) {
  if (v != v) return 0x7Fu;
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v, v, 0, false) & 0xFFu;
}

__device__ __forceinline__ uint32_t pack4_any(float a, float b, float c, float d) {
  return code1(a) | (code1(b) << 8) | (code1(c) << 16) | (code1(d) << 24);
}

// x / s for a finite s > 0 and y = 1/s (Markstein's correction; see the file header)
__device__ __forceinline__ float div_rcp(float x, float s, float y) {
  const float q0 = x * y;
  const float r = __builtin_fmaf(s, q0, -x);
  return __builtin_fmaf(-r, y, q0);
}

__device__ __forceinline__ uint32_t quant_dword(uint32_t d0, uint32_t d1, float s, float y) {
  const float a = clamp448_finite(div_rcp(lo_bf16(d0), s, y));
  const float b = clamp448_finite(div_rcp(hi_bf16(d0), s, y));
  const float c = clamp448_finite(div_rcp(lo_bf16(d1), s, y));
  const float d = clamp448_finite(div_rcp(hi_bf16(d1), s, y));
  return pack4(a, b, c, d);
}

// non-finite s: IEEE division per element, NaN quotients to the canonical code
__device__ __forceinline__ uint32_t quant_dword_any(uint32_t d0, uint32_t d1, float s) {
  const float a = clamp448(lo_bf16(d0) / s), b = clamp448(hi_bf16(d0) / s);
  const float c = clamp448(lo_bf16(d1) / s), d = clamp448(hi_bf16(d1) / s);
  return pack4_any(a, b, c, d);
}

// 8 bf16 values (one 16-byte group) -> 8 e4m3 codes, finite s with y = 1/s
__device__ __forceinline__ uint2 quant8(const uint4 v, float s, float y) {
  return make_uint2(quant_dword(v.x, v.y, s, y), quant_dword(v.z, v.w, s, y));
}

__device__ __forceinline__ uint2 quant8_any(const uint4 v, float s) {
  return make_uint2(quant_dword_any(v.x, v.y, s), quant_dword_any(v.z, v.w, s));
}

__device__ __forceinline__ float row_scale(uint32_t amax_bits) {
  const float s = __uint_as_float(amax_bits << 16) * kInv448;
  return s < kMinScale ? kMinScale : s;               // NaN stays NaN
}

__device__ __forceinline__ bool finite(float s) {
  return (__float_as_uint(s) & 0x7F800000u) != 0x7F800000u;
}

// 8 bf16 values -> 8 e4m3 codes for any s; y = 1/s (used only when s is finite)
__device__ __forceinline__ uint2 quant8_any_scale(const uint4 v, float s, float y) {
  return finite(s) ? quant8(v, s, y) : quant8_any(v, s);
}

}  // namespace fp8
}  // namespace w4a8
