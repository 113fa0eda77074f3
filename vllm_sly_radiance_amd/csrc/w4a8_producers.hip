// Fused fp8 activation producers for gfx950: the norm / activation in front of a W4A8 GEMM and the
// per-token e4m3 quantization in one pass, so the GEMM's (q, scale) input never exists in bf16.
//
// Counterparts of the reference's radiance_add_rms_quant, radiance_silu_mul_quant and
// radiance_gdn_norm_quant (sly/mxfp4/radiance_mxfp4_fp8.hip:1834-2156; ops and call sites in
// sly/mxfp4/radiance_fused_norm.py:132-304). One workgroup per row (256 threads; 1024 for silu
// and gdn at up to 128 rows); thread t owns the row's 8-element groups t, t + T, ..., read once as
// 16-byte vectors and kept in registers through the reductions. With few rows and registered
// scratch, silu splits each row over one-wave workgroups instead (below). The quantization tail
// is the one of the plain quantizer (w4a8_fp8.h), applied to the bf16-rounded producer output, so
// each op equals "producer -> bf16 -> quant".
//
// Every floating-point step is fixed so that the results are reproducible bit for bit on a CPU:
//  * no contracted multiply-add (the pragma below): each product and sum rounds, except the
//    explicit fused multiply-adds of exp_f32 and of the quantizer's division (w4a8_fp8.h, whose
//    codes equal those of the IEEE quotient);
//  * sums of squares run in a fixed order: a thread adds its groups' squares element by element,
//    a wave combines by an xor butterfly (32, 16, 8, 4, 2, 1) and the four waves add in order; a
//    gdn head (16 groups) combines by a 16-lane xor butterfly (8, 4, 2, 1);
//  * 1/sqrt is a correctly rounded square root and a correctly rounded division;
//  * exp is exp_f32 below: Cody-Waite reduction by ln 2 (Cody and Waite, "Software Manual for the
//    Elementary Functions", 1980; ln 2 split into a 16-bit head and a tail) and the degree-7
//    Taylor polynomial of e^r on |r| <= ln2 / 2 by Horner, the reduction and each Horner step one
//    fused multiply-add, then an exact scaling by 2^n;
//  * silu's division is the IEEE quotient (silu8: the reciprocal with one Markstein correction
//    where that equals it, else the division);
//  * rounding to bf16 is round to nearest even with NaN -> 0x7FC0 | sign (the hardware convert,
//    with the software rounding for a group that holds a NaN).
#pragma clang fp contract(off)

#include "w4a8_fp8.h"
#include "w4a8_silu.h"

namespace w4a8 {
namespace {

using namespace fp8;
using namespace prod;

// Row sum over the workgroup in the fixed order (every thread gets the result).
__device__ __forceinline__ float block_sum_fixed(float v) {
  __shared__ float red[kThreads / 64];
  v = wave_sum_xor(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; ++w) t = t + red[w];
  return t;
}

// Row max over a T-thread workgroup (every thread gets the result); max is exact in any order.
template <int T>
__device__ __forceinline__ uint32_t block_max_t(uint32_t v) {
  __shared__ uint32_t red[T / 64];
  v = wave_max(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  uint32_t m = red[0];
#pragma unroll
  for (int w = 1; w < T / 64; ++w) m = max(m, red[w]);
  return m;
}

// Groups tid, tid + T, ... of one row (of two rows, interleaved) into registers, zeros past the
// row's nv groups. The loads go through a buffer resource that ends at the row, so they need no
// branch (past the end the hardware returns zeros without an access), and callers load everything
// a row needs before they use any of it: every load is then in flight at once. A load behind a
// branch, a store or a reduction waits for the previous one's round trip.
__device__ __forceinline__ uint4 load_group(const __amdgpu_buffer_rsrc_t r, int g) {
  const v4i t = __builtin_amdgcn_raw_buffer_load_b128(r, g * 16, 0, 0);
  return make_uint4(t[0], t[1], t[2], t[3]);
}

template <int G, int T>
__device__ __forceinline__ void load_groups(const uint4* a, int nv, uint4 (&av)[G]) {
  const auto ra = __builtin_amdgcn_make_buffer_rsrc((void*)a, 0, nv * 16, kBufferWord3);
#pragma unroll
  for (int i = 0; i < G; ++i) av[i] = load_group(ra, threadIdx.x + i * T);
}

template <int G, int T>
__device__ __forceinline__ void load_groups(const uint4* a, int nv, uint4 (&av)[G],
                                            uint4 (&bv)[G], const uint4* b) {
  const auto ra = __builtin_amdgcn_make_buffer_rsrc((void*)a, 0, nv * 16, kBufferWord3);
  const auto rb = __builtin_amdgcn_make_buffer_rsrc((void*)b, 0, nv * 16, kBufferWord3);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    av[i] = load_group(ra, threadIdx.x + i * T);
    bv[i] = load_group(rb, threadIdx.x + i * T);
  }
}

// Byte offset of 8-element group g of row `row` in q (nv groups per row): row-major, or the
// fragment-tiled layout the tile GEMM reads (16-token blocks of 16 x K bytes; in block b, k-tile t,
// half h, lane l's 16 bytes at ((b KT + t) 2 + h) 1024 + 16 l hold token 16 b + l % 16, k-bytes
// 128 t + 16 (4 h + l / 16)). Group g is the low or high 8 bytes of 16-byte chunk g / 2.
__device__ __forceinline__ size_t q_offset(int row, int g, int nv, bool tiled) {
  if (!tiled) return ((size_t)row * nv + g) * 8;
  const int t = g >> 4, h = (g >> 3) & 1, l = (row & 15) + 16 * ((g >> 1) & 3);
  return (((size_t)(row >> 4) * (nv >> 4) + t) * 2 + h) * 1024 + 16 * l + 8 * (g & 1);
}

// The quantization tail: bf16 groups nb[] (group g = tid + i T) of this row -> scale[row], q row.
template <int G, int T>
__device__ __forceinline__ void quant_tail(const uint4 (&nb)[G], int nv, uint8_t* __restrict__ q,
                                           float* __restrict__ scale, int row, bool tiled) {
  const int tid = threadIdx.x;
  uint32_t am = 0;
#pragma unroll
  for (int i = 0; i < G; ++i)
    if (tid + i * T < nv) am = max(am, abs_bits_max8(nb[i]));
  const float sc = row_scale(block_max_t<T>(am));
  const float rcp = 1.0f / sc;
  if (tid == 0) scale[row] = sc;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + i * T;
    if (g < nv)
      *reinterpret_cast<uint2*>(q + q_offset(row, g, nv, tiled)) =
          quant8_any_scale(nb[i], sc, rcp);
  }
}

// Gemma RMSNorm with residual: v = y + res (fp32); res_out = bf16(v);
// n = bf16((v * (1 / sqrt(sum(v^2) / K + eps))) * (w + 1)). Rounds with selects: at decode sizes
// a row's four waves are alone on their CU.
template <int G>
__global__ __launch_bounds__(kThreads) void add_rms_quant(
    const uint4* __restrict__ y, const uint4* __restrict__ res, const uint4* __restrict__ w,
    uint8_t* __restrict__ q, float* __restrict__ scale, uint4* __restrict__ res_out, int K,
    float eps, int tiled) {
  const int row = blockIdx.x, tid = threadIdx.x, nv = K >> 3;
  y += (size_t)row * nv;
  res += (size_t)row * nv;
  res_out += (size_t)row * nv;
  float v[G][8];
  float part = 0.0f;
  // the weight groups are requested with the row and last, as they are used after its reduction
  uint4 yv[G], rv[G], wv[G];
  load_groups<G, kThreads>(y, nv, yv, rv, res);
  load_groups<G, kThreads>(w, nv, wv);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + i * kThreads;
    if (g < nv) {
      float a[8], b[8];
      unpack8(yv[i], a);
      unpack8(rv[i], b);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[i][j] = a[j] + b[j];
        part = part + v[i][j] * v[i][j];
      }
      res_out[g] = pack8_hw(v[i]);
    }
  }
  const float inv = 1.0f / sqrtf(block_sum_fixed(part) / (float)K + eps);
  uint4 nb[G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + i * kThreads;
    if (g < nv) {
      float wf[8], n[8];
      unpack8(wv[i], wf);
#pragma unroll
      for (int j = 0; j < 8; ++j) n[j] = (v[i][j] * inv) * (wf[j] + 1.0f);
      nb[i] = pack8_hw(n);
    }
  }
  quant_tail<G, kThreads>(nb, nv, q, scale, row, tiled);
}

// SiLU-and-mul: gate_up [M, 2N] -> bf16(bf16(silu(gate)) * up). T threads per row: the only
// reduction is the amax, so any T gives the same bits; short rows of work (small M) take 1024.
// One workgroup per row. With `out` set the bf16 stage is written there ([M, N]) and nothing is
// quantized (the w4a8_silu_mul entry point); otherwise the row is quantized into q and scale.
template <int G, int T>
__global__ __launch_bounds__(T) void silu_mul_quant(const uint4* __restrict__ gu,
                                                    uint8_t* __restrict__ q,
                                                    float* __restrict__ scale,
                                                    uint4* __restrict__ out, int N, int tiled) {
  const int row = blockIdx.x, tid = threadIdx.x, nv = N >> 3;
  const uint4* gate = gu + (size_t)row * 2 * nv;
  const uint4* up = gate + nv;
  uint4 gv[G], uv[G], nb[G];
  load_groups<G, T>(gate, nv, gv, uv, up);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int g = tid + i * T;
    if (g < nv) nb[i] = silu_mul_group(gv[i], uv[i]);
  }
  if (out) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const int g = tid + i * T;
      if (g < nv) out[(size_t)row * nv + g] = nb[i];
    }
    return;
  }
  quant_tail<G, T>(nb, nv, q, scale, row, tiled);
}

// One 8-element group of the per-head gated RMSNorm from its loaded x, z and weight groups. All 16
// lanes of a head call it together. It runs on every lane of a wave that holds part of the row: a
// group past the row holds zeros (the result is finite and never stored), and with no branch per
// group the compiler cannot sink a group's z load behind x's round trip.
__device__ __forceinline__ uint4 gdn_group(const uint4 xv, const uint4 zv, const uint4 wv,
                                           float eps) {
  float v[8];
  unpack8(xv, v);
  float part = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) part = part + v[j] * v[j];
  part = part + __uint_as_float(xor_lane<8>(__float_as_uint(part)));
  part = part + __uint_as_float(xor_lane<4>(__float_as_uint(part)));
  part = part + __uint_as_float(xor_lane<2>(__float_as_uint(part)));
  part = part + __uint_as_float(xor_lane<1>(__float_as_uint(part)));
  const float inv = 1.0f / sqrtf(part * (1.0f / 128.0f) + eps);
  float zz[8], sz[8], wf[8], n[8];
  unpack8(zv, zz);
  unpack8(wv, wf);
  silu8(zz, sz);
#pragma unroll
  for (int j = 0; j < 8; ++j) n[j] = ((v[j] * inv) * wf[j]) * sz[j];
  return pack8_hw(n);
}

// Per-head gated RMSNorm (head = 128 = 16 groups; norm before the gate, weight without +1):
// n = bf16(((x * (1 / sqrt(sum_head(x^2) / 128 + eps))) * w) * silu(z)). The head sums stay
// inside 16 lanes and the row reduction is the amax, so any T (a multiple of 64) gives the same
// bits.
template <int G, int T>
__global__ __launch_bounds__(T) void gdn_norm_quant(
    const uint4* __restrict__ x, const uint16_t* __restrict__ z, long zs,
    const uint4* __restrict__ w, uint8_t* __restrict__ q, float* __restrict__ scale, int N,
    float eps, int tiled) {
  const int row = blockIdx.x, tid = threadIdx.x, nv = N >> 3;
  x += (size_t)row * nv;
  const uint4* zr = reinterpret_cast<const uint4*>(z + (size_t)row * zs);
  uint4 xv[G], zv[G], wv[G], nb[G];
  load_groups<G, T>(x, nv, xv, zv, zr);
  const auto rw = __builtin_amdgcn_make_buffer_rsrc((void*)w, 0, 16 * 16, kBufferWord3);
#pragma unroll
  for (int i = 0; i < G; ++i) {
    wv[i] = load_group(rw, (tid + i * T) & 15);                     // the head's 16 groups
    nb[i] = make_uint4(0, 0, 0, 0);
  }
  if ((tid & ~63) < nv) {                     // the same for the whole wave: waves past the row skip
#pragma unroll
    for (int i = 0; i < G; ++i) nb[i] = gdn_group(xv[i], zv[i], wv[i], eps);
  }
  quant_tail<G, T>(nb, nv, q, scale, row, tiled);
}

// ---- silu_mul at few rows: each row split over one-wave workgroups ------------------------------
// With few rows, one workgroup per row leaves most CUs idle and runs VALU-bound (exp and two
// divisions per element) on the rest: 9.6 us for one row of 17408. Here a row's 8-element groups
// are cut into chunks of 64, one group per lane of a one-wave workgroup (grid S x M,
// S = ceil(groups / 64) <= 64). Pass 1 computes each chunk's bf16 output and writes its amax bits
// to part[row * S + chunk]; pass 2 computes the chunk again (same code, same bits), takes the
// row's amax over the S partials (max is exact in any order) and quantizes. The result equals the
// one-workgroup kernel's bit for bit; the price is a second launch and computing the chunk twice
// (5.8-6.0 us at 1 to 16 rows of 17408, against 8.4-8.6 us in one 1024-thread workgroup per row).
// It pays only where a 1024-thread workgroup holds three or more groups per thread: at N = 8704
// (two groups) one launch takes 5.4-6.1 us at 1 to 64 rows and the split 5.7-7.5 us. gdn_norm rows
// (N <= 10240) are faster in one launch too.
template <bool kQuant>
__device__ __forceinline__ void split_tail(const uint4 nb, bool in, uint8_t* __restrict__ q,
                                           float* __restrict__ scale, uint32_t* __restrict__ part,
                                           int row, int chunk, int S, int nv, bool tiled) {
  const int lane = threadIdx.x, g = chunk * 64 + lane;
  if constexpr (!kQuant) {
    const uint32_t am = wave_max(in ? abs_bits_max8(nb) : 0u);
    if (lane == 0) part[row * S + chunk] = am;
  } else {
    const float sc = row_scale(wave_max(lane < S ? part[row * S + lane] : 0u));
    if (chunk == 0 && lane == 0) scale[row] = sc;
    if (in)
      *reinterpret_cast<uint2*>(q + q_offset(row, g, nv, tiled)) =
          quant8_any_scale(nb, sc, 1.0f / sc);
  }
}

template <bool kQuant>
__global__ __launch_bounds__(64) void silu_mul_quant_split(const uint4* __restrict__ gu,
                                                           uint8_t* __restrict__ q,
                                                           float* __restrict__ scale,
                                                           uint32_t* __restrict__ part, int N,
                                                           int S, int tiled) {
  const int chunk = blockIdx.x, row = blockIdx.y, nv = N >> 3, g = chunk * 64 + threadIdx.x;
  const uint4* gate = gu + (size_t)row * 2 * nv;
  const bool in = g < nv;
  const uint4 nb = in ? silu_mul_group(gate[g], gate[nv + g]) : make_uint4(0, 0, 0, 0);
  split_tail<kQuant>(nb, in, q, scale, part, row, chunk, S, nv, tiled);
}

// Diagnostic: the fp32 silu of every producer (silu8, as the gated norm and SiLU-and-mul call
// it) on 8 bf16 inputs per thread, written unrounded, so tests can compare the quotient itself
// with the exactly dividing oracle for every bf16 input.
__global__ __launch_bounds__(256) void silu_probe(const uint4* __restrict__ x, float* __restrict__ y,
                                                  int groups) {
  const int g = blockIdx.x * 256 + threadIdx.x;
  if (g >= groups) return;
  float a[8], s[8];
  unpack8(x[g], a);
  silu8(a, s);
#pragma unroll
  for (int j = 0; j < 8; ++j) y[8 * g + j] = s[j];
}

}  // namespace

hipError_t launch_silu_probe(const void* x, float* y, int groups, hipStream_t stream) {
  if (groups == 0) return hipSuccess;
  hipLaunchKernelGGL(silu_probe, dim3(ceil_div(groups, 256)), dim3(256), 0, stream,
                     (const uint4*)x, y, groups);
  return hipGetLastError();
}

// Rows at or below which silu_mul splits rows of more than 2048 groups (N > 16384) over one-wave
// workgroups (when the caller registered scratch for the partial maxima); at 128 rows one
// workgroup per row is faster.
#ifndef W4A8_SPLIT_ROWS_MAX
#define W4A8_SPLIT_ROWS_MAX 64
#endif
constexpr int kSplitRowsMax = W4A8_SPLIT_ROWS_MAX;

size_t producer_split_bytes(int M, int N) { return (size_t)M * ceil_div(N >> 3, 64) * 4; }

// pass 2 reads a row's partials with one lane each
bool split_rows(int M, int N, const void* part, size_t part_bytes) {
  return M <= kSplitRowsMax && (N >> 3) > 2 * 1024 && ceil_div(N >> 3, 64) <= 64 && part &&
         producer_split_bytes(M, N) <= part_bytes;
}

hipError_t launch_add_rms_quant(const void* y, const void* res, const void* w, uint8_t* q,
                                float* scale, void* res_out, int M, int K, float eps, bool tiled,
                                hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int G = ceil_div(K >> 3, kThreads);
#define W4A8_ARQ(C)                                                                             \
  case C:                                                                                       \
    hipLaunchKernelGGL(add_rms_quant<C>, dim3(M), dim3(kThreads), 0, stream, (const uint4*)y,   \
                       (const uint4*)res, (const uint4*)w, q, scale, (uint4*)res_out, K, eps,   \
                       (int)tiled);                                                             \
    break;
  switch (G) {
    W4A8_ARQ(1) W4A8_ARQ(2) W4A8_ARQ(3) W4A8_ARQ(4) W4A8_ARQ(5)
    default: return hipErrorInvalidValue;
  }
#undef W4A8_ARQ
  return hipGetLastError();
}

// Rows of work per CU: with fewer rows than half the CUs, each row takes a 1024-thread workgroup.
constexpr int kWideRowsMax = 128;

hipError_t launch_silu_mul_quant(const void* gate_up, uint8_t* q, float* scale, void* out, int M,
                                 int N, void* part, size_t part_bytes, bool tiled,
                                 hipStream_t stream) {
  if (M == 0) return hipSuccess;
  if (!out && split_rows(M, N, part, part_bytes)) {
    const int S = ceil_div(N >> 3, 64);
    hipLaunchKernelGGL(silu_mul_quant_split<false>, dim3(S, M), dim3(64), 0, stream,
                       (const uint4*)gate_up, q, scale, (uint32_t*)part, N, S, (int)tiled);
    hipLaunchKernelGGL(silu_mul_quant_split<true>, dim3(S, M), dim3(64), 0, stream,
                       (const uint4*)gate_up, q, scale, (uint32_t*)part, N, S, (int)tiled);
    return hipGetLastError();
  }
  const bool wide = M <= kWideRowsMax;
  const int T = wide ? 1024 : kThreads;
  const int G = ceil_div(N >> 3, T);
#define W4A8_SMQ(C, TT)                                                                         \
  case C:                                                                                       \
    hipLaunchKernelGGL((silu_mul_quant<C, TT>), dim3(M), dim3(TT), 0, stream,                   \
                       (const uint4*)gate_up, q, scale, (uint4*)out, N, (int)tiled);            \
    break;
  if (wide) {
    switch (G) {
      W4A8_SMQ(1, 1024) W4A8_SMQ(2, 1024) W4A8_SMQ(3, 1024)
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (G) {
      W4A8_SMQ(1, 256) W4A8_SMQ(2, 256) W4A8_SMQ(3, 256) W4A8_SMQ(4, 256) W4A8_SMQ(5, 256)
      W4A8_SMQ(6, 256) W4A8_SMQ(7, 256) W4A8_SMQ(8, 256) W4A8_SMQ(9, 256)
      default: return hipErrorInvalidValue;
    }
  }
#undef W4A8_SMQ
  return hipGetLastError();
}

hipError_t launch_gdn_norm_quant(const void* x, const void* z, long zs, const void* w, uint8_t* q,
                                 float* scale, int M, int N, float eps, bool tiled,
                                 hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const bool wide = M <= kWideRowsMax;
  const int T = wide ? 1024 : kThreads;
  const int G = ceil_div(N >> 3, T);
#define W4A8_GNQ(C, TT)                                                                         \
  case C:                                                                                       \
    hipLaunchKernelGGL((gdn_norm_quant<C, TT>), dim3(M), dim3(TT), 0, stream, (const uint4*)x,  \
                       (const uint16_t*)z, zs, (const uint4*)w, q, scale, N, eps, (int)tiled);  \
    break;
  if (wide) {
    switch (G) {
      W4A8_GNQ(1, 1024) W4A8_GNQ(2, 1024)
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (G) {
      W4A8_GNQ(1, 256) W4A8_GNQ(2, 256) W4A8_GNQ(3, 256) W4A8_GNQ(4, 256) W4A8_GNQ(5, 256)
      default: return hipErrorInvalidValue;
    }
  }
#undef W4A8_GNQ
  return hipGetLastError();
}

}  // namespace w4a8
