// Streaming W4A8 GEMM for decode M (1..16) on gfx950: one workgroup per CU at most, every weight
// byte of a wave requested before the wave waits on anything.
//
// Counterpart of the reference's decode kernel (sly/mxfp4/radiance_mxfp4_fp8.hip:981-1228) for the
// M <= 16 band, redesigned around the MI355X memory system. At M <= 16 the GEMM is a weight stream
// (47 MB for the 17408 x 5120 gate/up), bounded by how early and how evenly the whole matrix is
// requested and by how little work is left once the last bytes land. Measured on MI355X:
//  * a read of that size is fastest with one workgroup per CU whose waves each hold ~20 KiB of
//    128-bit loads in flight, all issued before any is used;
//  * a per-wave timeline (s_memrealtime) of a design that staged the activations in LDS and gave
//    each wave one n-tile showed the stream done at ~7.5 us and then 1.6 us of MFMA work bound by
//    LDS reads (every wave re-read its 16-row activation fragments for every granule).
// So:
//  * The grid is at most one workgroup per CU, sized so every workgroup owns the same number of
//    n-tiles: workgroup b owns [b * NTILES / G, (b + 1) * NTILES / G), at most NT of them.
//  * Wave w owns the k-groups [KG w / W, KG (w + 1) / W) (4 k-tiles each, so one scale dword per
//    n-tile) of every n-tile of the workgroup. It loads its activation fragments for those
//    k-tiles straight into registers (lane l: token l % 16, k 16 (l / 16).. and 64 + 16 (l / 16)..;
//    tokens past M read as zero), then the scale dwords, then the granules k-tile by k-tile, and
//    multiplies each fragment into all NT n-tiles as their granules land: no LDS staging, no
//    barrier before the MFMAs, NT independent accumulator chains.
//  * Every global load goes through a buffer resource; loads past the workgroup's n-tiles or the
//    wave's k-range return zero without a memory access, so the code has no branches around loads
//    and the compiler counts outstanding loads exactly.
//  * The W partial sums of each n-tile meet once in LDS and are added in wave order
//    (deterministic), scaled by the per-token fp32 scale and stored as bf16. Nothing crosses
//    workgroups.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

// NT: n-tiles per workgroup at most; KPW: k-tiles per wave at most (a multiple of 4); W: waves.
// The host requires K % 512 == 0 (whole k-groups), M <= 16, 4 * ceil(KG / W) <= KPW.
template <int NT, int KPW, int W>
__global__ __launch_bounds__(W * 64) void gemm_stream(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KT,
    int KG, int NTILES, int vec_out) {
  static_assert(KPW % 4 == 0 && NT >= 1 && W >= 1 && W <= 16, "stream variant");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform work selection in scalar registers; 32-bit products only (the host bounds them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int ntb0 = b * NTILES / G, nth = (b + 1) * NTILES / G - ntb0;
  const int kr0 = 4 * (KG * wave / W), kr1 = 4 * (KG * (wave + 1) / W);

  // ---- 1. activation fragments of k-tiles kr0.. (L2): token lane % 16, two 16-byte runs.
  //         Tokens past M fall outside the buffer and read as zero; a k-tile past the wave's
  //         range re-reads the row's last k-tile (clamped in scalar arithmetic), which only ever
  //         meets zero weights ----
  const int m = lane & 15, g = lane >> 4;
  const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
  v4i xlo[KPW], xhi[KPW];
#pragma unroll
  for (int u = 0; u < KPW; ++u) {
    const int kt = min(kr0 + u, KT - 1);
    const int off = m * K + kt * kKTile + 16 * g;
    xlo[u] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off, 0, 0);
    xhi[u] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off + 64, 0, 0);
  }

  // ---- 2. scale dwords (one per n-tile and k-group), then the granules k-tile by k-tile.
  //         One buffer resource per n-tile, sized to end at the wave's k-range: loads past it,
  //         or of n-tile slots past the workgroup's share, return zero ----
  uint32_t sv[NT][KPW / 4];
  v4i wv[KPW][NT];
  {
    __amdgpu_buffer_rsrc_t w_src[NT], s_src[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool have = t < nth;
      w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(Wq + (size_t)(ntb0 + t) * KT * kGranuleBytes), 0,
          have ? kr1 * kGranuleBytes : 0, kBufferWord3);
      s_src[t] = __builtin_amdgcn_make_buffer_rsrc((void*)(Sq + (size_t)(ntb0 + t) * KG * 64), 0,
                                                   have ? (kr1 >> 2) * 256 : 0, kBufferWord3);
    }
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < KPW / 4; ++q)
        sv[t][q] = __builtin_amdgcn_raw_buffer_load_b32(
            s_src[t], (((kr0 >> 2) + q) * 64 + lane) * 4, 0, 0);
#pragma unroll
    for (int u = 0; u < KPW; ++u)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(
            w_src[t], (kr0 + u) * kGranuleBytes + lane * 16, 0, kBufferNT);
  }
  // the epilogue's per-token scale, last: it is needed last
  const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
  const float tok_scale = __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(as_src, (lane & 15) * 4, 0, 0));
  __builtin_amdgcn_sched_barrier(0);             // every load above is issued before any MFMA

  // ---- 3. MFMAs, branch-free: loads past the k-range or the n-tiles are zero and add nothing ----
  v4f acc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < KPW; ++u) {
    const v8i xf = {xlo[u][0], xlo[u][1], xlo[u][2], xlo[u][3],
                    xhi[u][0], xhi[u][1], xhi[u][2], xhi[u][3]};
#pragma unroll
    for (int t = 0; t < NT; ++t)
      acc[t] = mfma_w4a8(wv[u][t], xf, acc[t], sv[t][u / 4] >> (8 * (u & 3)));
  }

  // ---- 4. the W partial sums of each n-tile meet in LDS and are added in wave order ----
  v4f* red = reinterpret_cast<v4f*>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t];
  __syncthreads();
  const bool vec = vec_out != 0;
  for (int slot = tid; slot < nth * 64; slot += W * 64) {
    const int t = slot >> 6;                     // slot lane == this thread's lane
    v4f v = red[t * 64 + lane];
#pragma unroll 4
    for (int w = 1; w < W; ++w) v += red[(w * NT + t) * 64 + lane];
    const int n = (ntb0 + t) * kNTile + 4 * (lane >> 4);
    if (m < M) store_out4(C, N, m, n, N, v, tok_scale, vec);
  }
}

// (NT, KPW, W): NT * KPW granules and 2 KPW activation runs per wave in registers; W waves at
// most 4 per SIMD. Chosen per shape by the host: the fewest granules per wave, then the fewest
// n-tile slots, then the fewest waves.
#define W4A8_STREAM_TABLE(X)                                                                      \
  X(1, 4, 16) X(1, 8, 16) X(2, 4, 10) X(2, 4, 12) X(2, 4, 16) X(2, 8, 9) X(3, 4, 10)              \
  X(3, 4, 12) X(4, 4, 10) X(5, 4, 10) X(6, 4, 8) X(8, 4, 8)

#define W4A8_STREAM_CFG(nt, kpw, w) StreamCfg{nt, kpw, w, nt * kpw},
constexpr StreamCfg kStream[] = {W4A8_STREAM_TABLE(W4A8_STREAM_CFG)};
#undef W4A8_STREAM_CFG
constexpr int kStreamCount = sizeof(kStream) / sizeof(kStream[0]);

}  // namespace

int stream_variant_count() { return kStreamCount; }
StreamCfg stream_variant(int v) { return kStream[v]; }

// The fewest workgroups that keep the largest n-tile share of min(n-tiles, CUs) workgroups: every
// workgroup then carries the same share (N = 17408: 218 workgroups of 5 n-tiles rather than 256
// of 4 or 5), which measured 5 % faster on MI355X than one workgroup per CU.
int stream_grid(int N, int cus) {
  const int ntiles = padded_n(N) / kNTile;
  const int g = ntiles < cus ? ntiles : cus;
  return ceil_div(ntiles, ceil_div(ntiles, g));
}

size_t stream_lds_bytes(int variant, int M, int K) {
  (void)M;
  (void)K;
  const StreamCfg c = kStream[variant];
  return (size_t)c.waves * c.nt * 64 * sizeof(v4f);
}

// Granules the busiest wave of a variant streams for this shape (0: the variant cannot serve it).
int stream_granules(int variant, int N, int K, int cus) {
  const StreamCfg c = kStream[variant];
  if (K % 512) return 0;
  const int ntiles = padded_n(N) / kNTile;
  const int ntmax = ceil_div(ntiles, stream_grid(N, cus));
  const int kpw = 4 * ceil_div(K / kKAlign, c.waves);
  if (ntmax > c.nt || kpw > c.kpw) return 0;
  return ntmax * kpw;
}

bool stream_fits(int variant, int M, int N, int K, int cus, size_t lds_limit) {
  if (M < 1 || M > 16 || stream_granules(variant, N, K, cus) == 0) return false;
  const StreamCfg c = kStream[variant];
  // every offset the kernel forms stays in 32 bits
  const bool small = (long)M * K < (1L << 31) && (long)c.nt * (K / kKTile) * kGranuleBytes <
                     (1L << 31) && (long)padded_n(N) < (1L << 24);
  return small && stream_lds_bytes(variant, M, K) <= lds_limit;
}

hipError_t launch_stream(const GemmArgs& g, int variant, int cus, hipStream_t stream) {
  const int KT = g.K / kKTile, KG = KT / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(stream_grid(g.N, cus)), block(kStream[variant].waves * 64);
  const size_t lds = stream_lds_bytes(variant, g.M, g.K);
  int idx = 0;
#define W4A8_STREAM_LAUNCH(nt, kpw, w)                                                           \
  if (idx++ == variant) {                                                                        \
    if (lds > 64 * 1024) {                                                                       \
      const hipError_t e = hipFuncSetAttribute((const void*)gemm_stream<nt, kpw, w>,             \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                               (int)lds);                                        \
      if (e != hipSuccess) return e;                                                             \
    }                                                                                            \
    hipLaunchKernelGGL((gemm_stream<nt, kpw, w>), grid, block, lds, stream, g.a, g.a_scale, g.wq, \
                       g.sq, g.c, g.M, g.N, g.K, KT, KG, NTILES, vec_out);                       \
    return hipGetLastError();                                                                    \
  }
  W4A8_STREAM_TABLE(W4A8_STREAM_LAUNCH)
#undef W4A8_STREAM_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
