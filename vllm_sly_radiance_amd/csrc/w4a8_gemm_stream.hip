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
//    tokens past M read as zero; at M <= 8 one load per k-tile, see H8), then the scale dwords,
//    then the granules k-tile by k-tile, and multiplies each fragment into all NT n-tiles as
//    their granules land: no LDS staging, no barrier before the MFMAs, NT independent
//    accumulator chains.
//  * Every global load goes through a buffer resource; loads past the workgroup's n-tiles or the
//    wave's k-range return zero without a memory access, so the code has no branches around loads
//    and the compiler counts outstanding loads exactly.
//  * The W partial sums of each n-tile meet once in LDS and are added in wave order
//    (deterministic), scaled by the per-token fp32 scale and stored as bf16. Nothing crosses
//    workgroups.
//  * FQ = true takes bf16 activations (up to 8 rows; the host uses it for M x KPW <= 8) and
//    quantizes them itself, the whole linear in one launch. The waves of a workgroup together
//    cover all of K, so the per-token amax is a reduction inside the workgroup: each wave copies
//    its k-range of the (at most 8) rows into LDS (buffer_load ... lds, chunks XOR-swizzled by
//    token so the fragment reads are conflict-free), issues its scale and weight loads, takes the
//    amax of its range, and after one barrier every lane has its token's row amax. The codes then
//    come from the same steps as the plain quantizer's (w4a8_fp8.h), so the output equals
//    quantizer + GEMM bit for bit. A second barrier frees the staging area, which the final
//    reduction reuses.
#include "w4a8_fp8.h"

namespace w4a8 {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(n) with lgkmcnt and expcnt left open (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// A workgroup barrier after this wave's LDS accesses have completed, with no memory fence: the
// weight loads still in flight stay in flight (__syncthreads' release fence would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Fused-quant staging, per wave: KPW k-tiles x 8 tokens x 128 bf16 = 2 KPW KiB. Segment j (64
// elements of the wave's k-range, 1 KiB) holds token t's 16-byte chunk c at slot 8 t + (c ^ t).
template <int KPW>
__device__ __forceinline__ int stage_off(int seg, int t, int c) {
  return seg * 1024 + 16 * (8 * t + (c ^ t));
}

// NT: n-tiles per workgroup at most; KPW: k-tiles per wave at most (a multiple of 4); W: waves.
// The host requires K % 512 == 0 (whole k-groups), M <= 16 (M <= 8 with FQ or H8),
// 4 * ceil(KG / W) <= KPW. With FQ, A is the bf16 activation (row stride lda elements, 16-byte
// aligned rows) and As is not read. H8 (M <= 8, e4m3 A): one load per k-tile brings both 16-byte
// runs of the 8 live tokens (lanes 8..15 of each row of 16 load the second run of token r - 8,
// and a row rotation by 8 lanes hands it to lane r), half the activation loads; the MFMA columns
// of tokens 8..15 then hold other tokens' bytes, and those columns are never stored.
template <int NT, int KPW, int W, bool FQ, bool H8>
__global__ __launch_bounds__(W * 64) void gemm_stream(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, int M, int K, int NTILES, int G, int lda,
    uint16_t* __restrict__ C, int N, int vec_out) {
  static_assert(KPW % 4 == 0 && NT >= 1 && W >= 1 && W <= 16 && !(FQ && H8), "stream variant");
  const int KT = K / kKTile, KG = KT / kKGroup;  // K % 512 == 0
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform work selection in scalar registers; 32-bit products only (the host bounds them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int ntb0 = b * NTILES / G, nth = (b + 1) * NTILES / G - ntb0;
  const int kr0 = 4 * (KG * wave / W), kr1 = 4 * (KG * (wave + 1) / W);

  // ---- 1. activation fragments of k-tiles kr0.. (L2): token lane % 16, two 16-byte runs.
  //         Tokens past M fall outside the buffer and read as zero; a k-tile past the wave's
  //         range re-reads the row's last k-tile (clamped in scalar arithmetic), which only ever
  //         meets zero weights. FQ: the bf16 rows of the wave's k-range go to its LDS staging
  //         area instead, 8 tokens x 64 elements per load; tokens past M read zero ----
  const int m = lane & 15, g = lane >> 4;
  v4i xlo[KPW], xhi[KPW];
  uint8_t* const stage = lds + wave * KPW * 2048;
  if constexpr (FQ) {
    const auto x_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, (long)M * lda * 2,
                                                         kBufferWord3);
    const int t = lane >> 3, slot = lane & 7, c = slot ^ t;
#pragma unroll
    for (int j = 0; j < 2 * KPW; ++j) {
      // segment j of the wave's range; k-tiles past K (a range shorter than KPW) read zero
      const int k = kr0 * kKTile + 64 * j + 8 * c;
      const int off = k < K ? t * lda * 2 + 2 * k : 0x7FFFFFF0;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(x_src, (lds_ptr_t)(stage + j * 1024), 16, off,
                                               0, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);           // the staging copies go out first: the wait
                                                 // below counts the loads issued after them
  } else if constexpr (H8) {
    const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      const int kt = min(kr0 + u, KT - 1);
      xlo[u] = __builtin_amdgcn_raw_buffer_load_b128(
          a_src, (m & 7) * K + kt * kKTile + 64 * (m >> 3) + 16 * g, 0, 0);
    }
  } else {
    const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      const int kt = min(kr0 + u, KT - 1);
      const int off = m * K + kt * kKTile + 16 * g;
      xlo[u] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off, 0, 0);
      xhi[u] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off + 64, 0, 0);
    }
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
  float tok_scale;
  if constexpr (FQ) {
    __builtin_amdgcn_sched_barrier(0);           // every load above is issued before any wait
    // ---- 1b. amax of the wave's range per token (lanes 8 t .. 8 t + 7: token t), then the row
    //          amax over the waves, the scale and the codes, as the plain quantizer computes
    //          them ----
    wait_vm<NT * KPW + NT * (KPW / 4)>();         // this wave's staging copies have landed
    asm volatile("" ::: "memory");
    uint32_t* const amax_w = reinterpret_cast<uint32_t*>(lds + W * KPW * 2048);
    {
      const int t = lane >> 3, slot = lane & 7;
      uint32_t am = 0;
#pragma unroll
      for (int j = 0; j < 2 * KPW; ++j)
        am = max(am, fp8::abs_bits_max8(
                         *reinterpret_cast<const uint4*>(stage + j * 1024 + 16 * (8 * t + slot))));
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) am = max(am, (uint32_t)__shfl_xor((int)am, o, 64));
      if (slot == 0) amax_w[wave * 8 + t] = am;
    }
    lds_barrier();
    // the scales: lanes 0..7 of every wave take token lane's row amax over the waves and write
    // its scale and reciprocal next to the wave's maxima (read back by this wave only)
    float* const sc_w = reinterpret_cast<float*>(amax_w + W * 8) + wave * 16;
    if (lane < 8) {
      uint32_t am = 0;
#pragma unroll
      for (int w = 0; w < W; ++w) am = max(am, amax_w[w * 8 + lane]);
      const float sc = fp8::row_scale(am);
      sc_w[lane] = sc;
      sc_w[8 + lane] = 1.0f / sc;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): the wave's scales are written
    // Codes of the live chunks only (tokens < M; 16 KPW chunks a token), one 16-byte chunk per
    // lane per step, written as the fragment reads want them: half h of k-tile u holds lane
    // group g's 16 bytes of token t at ((2u + h) * 4 + g) * 8 + t (16-byte units). Step i reads
    // staged segments >= 8 i / M and writes into segments < 8 (i + 1) / M, which every lane of
    // the wave has read in earlier steps (or in this one, before it writes): the codes can
    // overwrite the staging area in place.
    const int live_chunks = M * 16 * KPW;
    for (int ci = lane; ci < ((live_chunks + 63) & ~63); ci += 64) {
      const bool in = ci < live_chunks;
      const int t = in ? ci % M : 0, qq = in ? ci / M : 0;
      const int seg = qq >> 3, c = qq & 7;
      const uint4 v = *reinterpret_cast<const uint4*>(stage + stage_off<KPW>(seg, t, c));
      const float sc = sc_w[t], rcp = sc_w[8 + t];
      __builtin_amdgcn_s_waitcnt(0xC07F);        // every lane's chunk is read before any write
      const uint2 q = fp8::quant8_any_scale(v, sc, rcp);
      if (in)
        *reinterpret_cast<uint2*>(stage + ((seg * 4 + (c >> 1)) * 8 + t) * 16 + 8 * (c & 1)) = q;
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    const int tm = m & 7;                        // lanes of tokens 8..15 mirror 0..7, then zero
    const bool live = m < M;
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      const v4i lo = *reinterpret_cast<const v4i*>(stage + (((2 * u) * 4 + g) * 8 + tm) * 16);
      const v4i hi = *reinterpret_cast<const v4i*>(stage + (((2 * u + 1) * 4 + g) * 8 + tm) * 16);
      xlo[u] = live ? lo : v4i{0, 0, 0, 0};
      xhi[u] = live ? hi : v4i{0, 0, 0, 0};
    }
    const float sc = sc_w[tm];
    tok_scale = sc;
    lds_barrier();                               // the staging area is free for the reduction
  } else {
    // the epilogue's per-token scale, last: it is needed last
    const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
    tok_scale = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(as_src, (lane & 15) * 4, 0, 0));
    __builtin_amdgcn_sched_barrier(0);           // every load above is issued before any MFMA
    if constexpr (H8) {
      // DPP row_ror:8 (within each row of 16 lanes, lane r takes lane (r + 8) % 16's value)
#pragma unroll
      for (int u = 0; u < KPW; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xhi[u][i] = __builtin_amdgcn_mov_dpp(xlo[u][i], 0x128, 0xF, 0xF, false);
    }
  }

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

size_t stream_lds_bytes(int variant, int M, int K, bool fused) {
  (void)M;
  (void)K;
  const StreamCfg c = kStream[variant];
  const size_t red = (size_t)c.waves * c.nt * 64 * sizeof(v4f);
  // fused: the staging area (2 KiB per k-tile per wave), then the waves' token maxima and their
  // scales; the final reduction reuses the staging area
  const size_t stage = (size_t)c.waves * c.kpw * 2048 + (size_t)c.waves * (8 + 16) * 4;
  return fused && stage > red ? stage : red;
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
  return small && stream_lds_bytes(variant, M, K, false) <= lds_limit;
}

// Every workgroup quantizes the whole activation, M x K elements, so the one-launch form pays off
// only for few rows: measured on MI355X over the four Qwen3.8-27B linear shapes, it beats the
// quantizer + GEMM pair by 0.3-1.1 us at M = 1 and by 0.3-0.6 us at M = 2 with 4 k-tiles per wave,
// and loses from M x KPW = 12 on (M = 2 on down's 8 k-tiles: 10.9 against 10.2 us).
bool stream_linear_fits(int variant, int M, int N, int K, long ldx, int cus, size_t lds_limit) {
  const StreamCfg c = kStream[variant];
  if (M * c.kpw > 8) return false;
  return stream_fits(variant, M, N, K, cus, lds_limit) && ldx >= K &&
         ldx % 8 == 0 && 16L * ldx < (1L << 31) &&   // row offsets of all 8 staged rows
         stream_lds_bytes(variant, M, K, true) <= lds_limit;
}

// fused: g.a is the bf16 activation with row stride lda elements (the quantizer runs in the
// kernel); otherwise g.a is e4m3 [M, K] and g.a_scale its per-token scales
hipError_t launch_stream(const GemmArgs& g, int variant, int cus, bool fused, long lda,
                         hipStream_t stream) {
  const int NTILES = padded_n(g.N) / kNTile;
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(stream_grid(g.N, cus)), block(kStream[variant].waves * 64);
  const size_t lds = stream_lds_bytes(variant, g.M, g.K, fused);
  int idx = 0;
#define W4A8_STREAM_GO(nt, kpw, w, fq, h8)                                                       \
  {                                                                                              \
    if (lds > 64 * 1024) {                                                                       \
      const hipError_t e = hipFuncSetAttribute((const void*)gemm_stream<nt, kpw, w, fq, h8>,     \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                               (int)lds);                                        \
      if (e != hipSuccess) return e;                                                             \
    }                                                                                            \
    hipLaunchKernelGGL((gemm_stream<nt, kpw, w, fq, h8>), grid, block, lds, stream, g.a,         \
                       g.a_scale, g.wq, g.sq, g.M, g.K, NTILES, (int)grid.x, (int)lda, g.c, g.N, \
                       vec_out);                                                                 \
    return hipGetLastError();                                                                    \
  }
#define W4A8_STREAM_LAUNCH(nt, kpw, w)                                                           \
  if (idx++ == variant) {                                                                        \
    if (fused) W4A8_STREAM_GO(nt, kpw, w, true, false)                                           \
    if (g.M <= 8) W4A8_STREAM_GO(nt, kpw, w, false, true)                                        \
    W4A8_STREAM_GO(nt, kpw, w, false, false)                                                     \
  }
  W4A8_STREAM_TABLE(W4A8_STREAM_LAUNCH)
#undef W4A8_STREAM_LAUNCH
#undef W4A8_STREAM_GO
  return hipErrorInvalidValue;
}

}  // namespace w4a8
