// Register-resident throughput probe of the gfx950 scaled MFMA with fp4 A and fp8 B operands,
// the instruction every GEMM here issues. It pins the denominator the prefill GEMM's MFMA
// utilisation is quoted against, as the reference pinned its own fp8 WMMA rate on gfx1201
// (325.2 TFLOP/s register-resident, sly/mxfp4/radiance_mxfp4_fp8.hip:6-10).
// Each wave runs 8 independent accumulator chains so the issue rate, not the dependency latency,
// bounds it; operands never leave registers. One thread per wave writes a checksum so nothing is
// optimised away.
//
// Also a streaming-read probe with the decode GEMM's launch shape, the HBM ceiling the verify GEMM
// is compared against: 10-wave workgroups, every wave holding 20 KiB of 128-bit loads in flight,
// all issued before any is used (the shape of gemm_stream<5, 4, 10>), over one buffer.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void mfma_rate_16x16x128(float* out, int iters) {
  const int l = threadIdx.x;
  const v4i w = {0x22222222 ^ l, 0x13131313, 0x31313131 ^ (l << 8), 0x02020202};
  const v8i x = {0x38383838, 0x30303030 ^ l, 0x38303830, 0x30383038,
                 0x38383838, 0x30303030, 0x38303830 ^ (l << 16), 0x30383038};
  v4f acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = v4f{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = mfma_w4a8(w, x, acc[i], 120u + (uint32_t)i);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
  if ((l & 63) == 0) out[blockIdx.x * 4 + (l >> 6)] = s;
}

__global__ __launch_bounds__(256) void mfma_rate_32x32x64(float* out, int iters) {
  const int l = threadIdx.x;
  const v8i w = {0x22222222 ^ l, 0x13131313, 0x31313131, 0x02020202, 0, 0, 0, 0};
  const v8i x = {0x38383838, 0x30303030 ^ l, 0x38303830, 0x30383038,
                 0x38383838, 0x30303030, 0x38303830, 0x30383038};
  v16f acc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = v16f{};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc[i] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(w, x, acc[i], 4, 0, 0,
                                                               120 + i, 0, (int)kUnitScales);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) s += acc[i][j];
  if ((l & 63) == 0) out[blockIdx.x * 4 + (l >> 6)] = s;
}

// One wave per tile t < count: D = the scaled MFMA of raw lane operands, as the GEMMs issue it
// (fp4 A, fp8 B, scale byte 0 of each lane's scale dword).
__global__ __launch_bounds__(256) void mfma_tiles(const int* __restrict__ a,
                                                 const int* __restrict__ b,
                                                 const int* __restrict__ sa,
                                                 const int* __restrict__ sb,
                                                 float* __restrict__ d, int count) {
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6), l = threadIdx.x & 63;
  if (t >= count) return;
  const size_t tl = (size_t)t * 64 + l;
  const int* pa = a + tl * 4;
  const int* pb = b + tl * 8;
  const v4i av = {pa[0], pa[1], pa[2], pa[3]};
  const v8i bv = {pb[0], pb[1], pb[2], pb[3], pb[4], pb[5], pb[6], pb[7]};
  const v8i a8 = {av[0], av[1], av[2], av[3], 0, 0, 0, 0};
  const v4f acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
      a8, bv, v4f{0.f, 0.f, 0.f, 0.f}, 4, 0, 0, sa[tl], 0, sb[tl]);
  float* pd = d + tl * 4;
  pd[0] = acc[0];
  pd[1] = acc[1];
  pd[2] = acc[2];
  pd[3] = acc[3];
}

// Wave w of the grid reads bytes [w * kReadRun, (w + 1) * kReadRun) of buf as 64-lane 16-byte
// loads (non-temporal, like the GEMM's weight stream); loads past `bytes` return zero. The
// xor of everything read goes to out[0] only if it equals a value no data here produces.
constexpr int kReadWaves = 10, kReadUnits = 20, kReadRun = kReadUnits * 1024;

__global__ __launch_bounds__(kReadWaves * 64) void read_stream(const uint8_t* __restrict__ buf,
                                                              int bytes, int* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int w = blockIdx.x * kReadWaves + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)buf, 0, bytes, kBufferWord3);
  v4i v[kReadUnits];
#pragma unroll
  for (int u = 0; u < kReadUnits; ++u)
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, w * kReadRun + u * 1024 + lane * 16, 0,
                                                 kBufferNT);
  v4i acc = v[0];
#pragma unroll
  for (int u = 1; u < kReadUnits; ++u) acc ^= v[u];
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5A17C0DE) out[0] = w;
}

// The read ceiling over launch shapes: G workgroups of W waves, workgroup b reading bytes
// [b * wg_bytes, (b + 1) * wg_bytes) of buf (wg_bytes a multiple of 1 KiB; the last workgroup's
// range ends at `bytes`) and wave w of it the U KiB from w * U KiB of that range, as 64-lane
// 16-byte loads; loads past the range return zero without a memory access. R == U: every load
// issued before any is used (the decode GEMM's pattern); R < U: R loads in flight, each consumed
// (xor) before its register is refilled with the load R further on. NT: non-temporal loads.
template <int W, int U, int R, bool NT>
__global__ __launch_bounds__(W * 64) void read_sweep(const uint8_t* __restrict__ buf, int bytes,
                                                     int wg_bytes, int* __restrict__ out) {
  static_assert(W >= 1 && W <= 16 && U >= 1 && R >= 1 && R <= U && R <= 60, "read variant");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int base = blockIdx.x * wg_bytes;            // < bytes for every launched workgroup
  const int len = min(wg_bytes, bytes - base);
  const auto rs = __builtin_amdgcn_make_buffer_rsrc((void*)(buf + base), 0, len, kBufferWord3);
  const int off = wave * U * 1024 + lane * 16;
  constexpr int aux = NT ? kBufferNT : 0;
  v4i acc = {0, 0, 0, 0};
  v4i v[R];
#pragma unroll
  for (int u = 0; u < R; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + u * 1024, 0, aux);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int u = R; u < U; ++u) {
    acc ^= v[u % R];                                 // waits for the oldest load only
    v[u % R] = __builtin_amdgcn_raw_buffer_load_b128(rs, off + u * 1024, 0, aux);
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int u = U; u < U + R; ++u) acc ^= v[u % R];
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5A17C0DE) out[0] = blockIdx.x;
}

// (W, U, R, NT): W waves of U KiB each, R loads in flight per wave
#define W4A8_READ_TABLE(X)                                                                        \
  X(10, 20, 20, 1) X(10, 22, 22, 1) X(4, 46, 46, 1) X(8, 23, 23, 1) X(10, 19, 19, 1)              \
  X(12, 16, 16, 1) X(16, 12, 12, 1) X(10, 19, 19, 0) X(10, 19, 8, 1) X(16, 12, 4, 1)              \
  X(8, 23, 8, 1) X(8, 12, 12, 1) X(4, 12, 12, 1) X(16, 6, 6, 1) X(16, 12, 12, 0) X(8, 23, 12, 1)  \
  X(10, 26, 26, 1) X(10, 30, 30, 1) X(10, 35, 35, 1)

struct ReadCfg { int w, u, r, nt; };
#define W4A8_READ_CFG(w, u, r, nt) ReadCfg{w, u, r, nt},
constexpr ReadCfg kRead[] = {W4A8_READ_TABLE(W4A8_READ_CFG)};
#undef W4A8_READ_CFG
constexpr int kReadCount = sizeof(kRead) / sizeof(kRead[0]);

}  // namespace

int read_variant_count() { return kReadCount; }

int read_variant_info(int v, int* waves, int* units, int* window, int* nt) {
  if (v < 0 || v >= kReadCount) return 0;
  *waves = kRead[v].w;
  *units = kRead[v].u;
  *window = kRead[v].r;
  *nt = kRead[v].nt;
  return 1;
}

// Bytes per workgroup when `blocks` workgroups share `bytes` (a multiple of 1 KiB), or 0 when the
// variant cannot cover them or a workgroup would be left without bytes.
int read_shape_wg_bytes(int v, long bytes, int blocks) {
  if (v < 0 || v >= kReadCount || blocks < 1 || bytes < 1) return 0;
  const long per = ((bytes + blocks - 1) / blocks + 1023) / 1024 * 1024;
  if ((long)(blocks - 1) * per >= bytes) return 0;
  if ((long)kRead[v].w * kRead[v].u * 1024 < per) return 0;
  return (int)per;
}

hipError_t launch_read_shape(const void* buf, int bytes, int* out, int blocks, int v,
                             hipStream_t stream) {
  const int per = read_shape_wg_bytes(v, bytes, blocks);
  if (per == 0) return hipErrorInvalidValue;
  int idx = 0;
#define W4A8_READ_GO(w, u, r, nt)                                                                 \
  if (idx++ == v) {                                                                              \
    hipLaunchKernelGGL((read_sweep<w, u, r, nt != 0>), dim3(blocks), dim3(w * 64), 0, stream,    \
                       (const uint8_t*)buf, bytes, per, out);                                    \
    return hipGetLastError();                                                                    \
  }
  W4A8_READ_TABLE(W4A8_READ_GO)
#undef W4A8_READ_GO
  return hipErrorInvalidValue;
}

hipError_t launch_read_probe(const void* buf, int bytes, int* out, hipStream_t stream) {
  const int blocks = ceil_div(ceil_div(bytes, kReadRun), kReadWaves);
  hipLaunchKernelGGL(read_stream, dim3(blocks), dim3(kReadWaves * 64), 0, stream,
                     (const uint8_t*)buf, bytes, out);
  return hipGetLastError();
}

hipError_t launch_mfma_tiles(const int* a, const int* b, const int* sa, const int* sb, float* d,
                             int count, hipStream_t stream) {
  hipLaunchKernelGGL(mfma_tiles, dim3((unsigned)ceil_div(count, 4)), dim3(256), 0, stream, a, b,
                     sa, sb, d, count);
  return hipGetLastError();
}

// Launches `blocks` workgroups of 4 waves; returns the FLOP the launch performs in *flop.
hipError_t launch_mfma_probe(int shape, float* out, int blocks, int iters, double* flop,
                             hipStream_t stream) {
  const double waves = 4.0 * blocks;
  if (shape == 0) {
    hipLaunchKernelGGL(mfma_rate_16x16x128, dim3(blocks), dim3(256), 0, stream, out, iters);
    *flop = waves * iters * 8.0 * (2.0 * 16 * 16 * 128);
  } else {
    hipLaunchKernelGGL(mfma_rate_32x32x64, dim3(blocks), dim3(256), 0, stream, out, iters);
    *flop = waves * iters * 4.0 * (2.0 * 32 * 32 * 64);
  }
  return hipGetLastError();
}

}  // namespace w4a8
