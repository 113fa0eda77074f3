// Dynamic per-token bf16 -> fp8 e4m3fn activation quantizer for gfx950.
//
// Semantics are those of the reference's pure-torch quantizer _traced_quant
// (sly/mxfp4/radiance_mxfp4.py:392-396), evaluated in fp32 exactly as torch's CPU kernels do:
//   s = max(amax(|x|) * fl32(1/448), 1/(448*512))      NaN in the row propagates to s
//   q = e4m3_rne(clamp(x / s, -448, 448))               the IEEE fp32 quotient
// One workgroup per token: 4 wave64 at large M, where many rows share each CU; 8 or 16 at
// M <= 256, where each row's load-reduce-store chain is the latency (16 waves hold K <= 8192 at
// one 16-byte chunk per thread; 8 waves measured faster at K = 8704, three chunks per thread
// against two: M = 8 2.73 against 2.88 us, against 3.04 us with 4 waves on MI355X). Each thread
// keeps its 16-byte chunks in registers across the amax reduction, so the row is read from HBM
// once. The amax runs on the bf16 bit patterns
// (|x| bits = x & 0x7FFF): integer max is exact, orders like the magnitudes and ranks NaN above
// inf, which gives torch's NaN propagation for free. Wave64 butterfly, then LDS across waves.
// Codes come from the hardware e4m3 converter (v_cvt_pk_fp8_f32, round to nearest even); inputs
// are clamped first, so it never saturates. Rows whose scale is not finite (a NaN or inf in the
// row) take a per-element path that maps every NaN quotient to the canonical code 0x7F.
#include "w4a8_fp8.h"

namespace w4a8 {
namespace {

using namespace fp8;

// Vector path: 16-byte aligned rows, K % 8 == 0, K <= 8 * T * CPT.
template <int CPT, int T>
__global__ __launch_bounds__(T) void quant_rows_vec(const uint16_t* __restrict__ x, long ldx,
                                                   uint8_t* __restrict__ q, float* __restrict__ s,
                                                   int K) {
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const int nch = K >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)row * ldx);
  uint4 v[CPT];
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = tid + i * T;
    v[i] = c < nch ? xr[c] : make_uint4(0, 0, 0, 0);
    am = max(am, abs_bits_max8(v[i]));
  }
  const float sc = row_scale(block_max_t<T>(am));
  if (tid == 0) s[row] = sc;
  uint2* qr = reinterpret_cast<uint2*>(q + (size_t)row * K);
  if (finite(sc)) {
    const float rcp = 1.0f / sc;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * T;
      if (c < nch) qr[c] = quant8(v[i], sc, rcp);
    }
  } else {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + i * T;
      if (c < nch) qr[c] = quant8_any(v[i], sc);
    }
  }
}

// General path: any K, any alignment; reads the row twice (the second pass hits L2).
__global__ __launch_bounds__(kThreads) void quant_rows_any(const uint16_t* __restrict__ x,
                                                          long ldx, uint8_t* __restrict__ q,
                                                          float* __restrict__ s, int K) {
  const int row = blockIdx.x;
  const uint16_t* xr = x + (size_t)row * ldx;
  uint32_t am = 0;
  for (int k = threadIdx.x; k < K; k += kThreads) am = max(am, (uint32_t)(xr[k] & 0x7FFFu));
  const float sc = row_scale(block_max(am));
  if (threadIdx.x == 0) s[row] = sc;
  uint8_t* qr = q + (size_t)row * K;
  for (int k = threadIdx.x; k < K; k += kThreads)
    qr[k] = (uint8_t)code1(clamp448(__uint_as_float((uint32_t)xr[k] << 16) / sc));
}

}  // namespace

hipError_t launch_quant(const uint16_t* x, long ldx, uint8_t* q, float* s, int M, int K,
                        hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const dim3 grid(M), block(kThreads);
  const bool vec = K % 8 == 0 && ldx % 8 == 0 && ((uintptr_t)x % 16) == 0 &&
                   ((uintptr_t)q % 8) == 0;
  const int nch = ceil_div(K, 8);
#define W4A8_QV(C, T) \
  hipLaunchKernelGGL((quant_rows_vec<C, T>), grid, dim3(T), 0, stream, x, ldx, q, s, K)
  if (vec && M <= 256 && nch <= 1024) W4A8_QV(1, 1024);
  else if (vec && M <= 256 && nch <= 1536) W4A8_QV(3, 512);
  else if (vec && M <= 256 && nch <= 2048) W4A8_QV(2, 1024);
  else {
    const int need = ceil_div(nch, kThreads);
    if (vec && need <= 1) W4A8_QV(1, kThreads);
    else if (vec && need <= 2) W4A8_QV(2, kThreads);
    else if (vec && need <= 3) W4A8_QV(3, kThreads);
    else if (vec && need <= 4) W4A8_QV(4, kThreads);
    else if (vec && need <= 5) W4A8_QV(5, kThreads);
    else if (vec && need <= 6) W4A8_QV(6, kThreads);
    else if (vec && need <= 8) W4A8_QV(8, kThreads);
    else if (vec && need <= 10) W4A8_QV(10, kThreads);
    else if (vec && need <= 12) W4A8_QV(12, kThreads);
    else if (vec && need <= 16) W4A8_QV(16, kThreads);
    else hipLaunchKernelGGL(quant_rows_any, grid, block, 0, stream, x, ldx, q, s, K);
  }
#undef W4A8_QV
  return hipGetLastError();
}

}  // namespace w4a8
