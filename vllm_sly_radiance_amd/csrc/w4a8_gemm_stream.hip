// Streaming W4A8 GEMM for decode M (1..16) on gfx950: one workgroup per CU, every weight byte of a
// wave requested before the wave waits on anything.
//
// Counterpart of the reference's decode kernel (sly/mxfp4/radiance_mxfp4_fp8.hip:981-1228) for the
// M <= 16 band, redesigned around the MI355X memory system. At M <= 16 the GEMM is a weight stream
// (47 MB for the 17408 x 5120 gate/up), bounded by how early and how evenly the whole matrix is
// requested and by how little instruction work sits between the loads. Measured on MI355X, a read
// of that size is fastest with one workgroup per CU whose waves each issue one contiguous
// ~20 KiB run of 128-bit loads before using any; a second round of workgroups, grid-stride loops
// or per-granule branching all cost 10-60 %. So:
//  * The grid is at most one workgroup per CU, sized so every workgroup owns the same number of
//    n-tiles (NTMAX = ceil(n-tiles / CUs)). Workgroup b owns the n-tile range
//    [b * NTILES / G, (b + 1) * NTILES / G) (at most NTMAX n-tiles); its W = NTMAX * S waves each
//    own one (n-tile, K split) pair, a contiguous run of whole 4-granule groups in the granule
//    layout ([n-tile][k-tile][lane][16 B]) - so no run crosses an n-tile and one scale dword
//    serves four granules.
//  * Every global load goes through a buffer resource; granules past the run load as zero without
//    a memory access, so the MFMA loop has no branches and the compiler counts outstanding loads
//    exactly. All of a wave's weight loads and scale dwords are issued before it waits.
//  * The activations (M rows x K, L2-resident, shared by every workgroup) are loaded after the
//    weights and staged in LDS, row-major with a 16-byte row pad so the 16 lanes of a fragment
//    read hit distinct banks, plus one zero row for the fragment lanes of tokens past the staged
//    rows.
//  * Run bounds and offsets are wave-uniform scalar arithmetic (the wave index comes through
//    readfirstlane), so the per-granule code is a load, a shift, two LDS reads and an MFMA.
//  * The S partial sums of an n-tile meet in LDS and are added in split order (deterministic),
//    scaled by the per-token fp32 scale and stored as bf16. Nothing crosses workgroups.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

// Byte offset of the split-reduction buffer: past the RP + 1 staged rows, 16-byte aligned.
template <int RP>
__host__ __device__ constexpr size_t red_offset_rp(int K) {
  return ((size_t)(RP + 1) * (K + 16) + 15) / 16 * 16;
}

// U: granules per wave at most (a multiple of 4); W: waves per workgroup; RP: activation rows
// staged (8 or 16, M <= RP); AM: 16-byte activation chunks per thread, so K <= AM * (64 W / RP) * 16.
// The host requires K % 512 == 0: whole k-tiles, whole 4-k-tile scale groups, no K padding.
template <int U, int W, int RP, int AM>
__global__ __launch_bounds__(W * 64) void gemm_stream(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KT,
    int KG, int NTILES, int S, int vec_out) {
  static_assert(U % 4 == 0 && (RP == 8 || RP == 16) && (W * 64) % RP == 0, "stream variant");
  constexpr int TPR = W * 64 / RP;               // staging threads per activation row
  constexpr int kOut = 0x7FFFFFF0;               // an offset past every buffer resource here
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform work selection in scalar registers; 32-bit products only (the host bounds them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int ntb0 = b * NTILES / G, ntb1 = (b + 1) * NTILES / G;
  const int j = wave / S, split = wave - j * S;            // this wave's n-tile (local), K split
  const bool active = j < ntb1 - ntb0;
  const int kr0 = 4 * ((KT >> 2) * split / S), kr1 = 4 * ((KT >> 2) * (split + 1) / S);
  const int ldr = K + 16;

  // the epilogue's per-token scale (token lane % 16), fetched first so it never waits at the end
  const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
  const float tok_scale = __builtin_bit_cast(
      float, __builtin_amdgcn_raw_buffer_load_b32(as_src, (lane & 15) * 4, 0, 0));

  // ---- 1. this wave's granules: n-tile ntb0 + j, k-tiles [kr0, kr1), at most U of them ----
  const int nt = ntb0 + j;
  const auto w_src = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Wq + (size_t)nt * KT * kGranuleBytes), 0, active ? kr1 * kGranuleBytes : 0,
      kBufferWord3);
  const auto s_src = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Sq + (size_t)nt * KG * 64), 0, active ? (kr1 >> 2) * 256 : 0, kBufferWord3);
  v4i wv[U];
  uint32_t sv[U / 4];
#pragma unroll
  for (int u = 0; u < U; ++u) {                  // granule u (and, every 4th, its scale dword)
    wv[u] = __builtin_amdgcn_raw_buffer_load_b128(w_src, (kr0 + u) * kGranuleBytes + lane * 16, 0,
                                                  kBufferNT);
    if (u % 4 == 0)
      sv[u / 4] = __builtin_amdgcn_raw_buffer_load_b32(s_src, ((kr0 + u) >> 2) * 256 + lane * 4, 0,
                                                       0);
  }

  // ---- 2. activation loads (L2), after the weights: they retire behind this wave's weight
  //         stream, so the MFMAs below run once every granule has landed - measured on MI355X,
  //         that beats putting ~40 KiB of L2 reads ahead of every workgroup's weight stream.
  //         Thread t stages row t / TPR, 16-byte chunks t % TPR + TPR * c; rows at or past M read
  //         as zero ----
  const int srow = tid / TPR, scol = tid % TPR;
  const auto ra_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
  v4i ra[AM];
#pragma unroll
  for (int c = 0; c < AM; ++c) {
    const int col = scol + c * TPR;
    ra[c] = __builtin_amdgcn_raw_buffer_load_b128(
        ra_src, col * 16 < K ? srow * K + col * 16 : kOut, 0, 0);
  }

  // ---- 3. stage the activations in LDS: rows 0..RP-1 (zero past M) plus a zero row RP that
  //         the fragment lanes of tokens >= RP read ----
#pragma unroll
  for (int c = 0; c < AM; ++c) {
    const int col = scol + c * TPR;
    if (col * 16 < K) *reinterpret_cast<v4i*>(lds + srow * ldr + col * 16) = ra[c];
  }
  for (int col = tid; col * 16 < K; col += W * 64)
    *reinterpret_cast<v4i*>(lds + RP * ldr + col * 16) = v4i{0, 0, 0, 0};
  __syncthreads();

  // ---- 4. MFMAs, branch-free: granules past the run are zero and add nothing. Fragment lane
  //         (token l % 16, g = l / 16) reads k 16g.. and 64 + 16g..; the fragment of granule
  //         u + 1 is read before granule u's MFMA, and four accumulator chains keep the MFMAs
  //         independent once the last granules land together ----
  constexpr int CH = 4;
  v4f acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = v4f{0.f, 0.f, 0.f, 0.f};
  const int m = lane & 15;
  const uint8_t* xrow = lds + (m < RP ? m : RP) * ldr + (lane >> 4) * 16;
  if (active) {
    auto frag = [&](int u) {
      const int kt = kr0 + u < KT ? kr0 + u : KT - 1;    // stays inside the staged row
      const v4i lo = *reinterpret_cast<const v4i*>(xrow + kt * kKTile);
      const v4i hi = *reinterpret_cast<const v4i*>(xrow + kt * kKTile + 64);
      return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    };
    v8i xf = frag(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const v8i cur = xf;
      if (u + 1 < U) xf = frag(u + 1);
      acc[u % CH] = mfma_w4a8(wv[u], cur, acc[u % CH], sv[u / 4] >> (8 * (u & 3)));
    }
  }
  v4f sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);

  // ---- 5. the S partial sums of each n-tile meet in LDS (a region of their own, past the
  //         staged rows) and are added in split order ----
  v4f* red = reinterpret_cast<v4f*>(lds + red_offset_rp<RP>(K));
  red[wave * 64 + lane] = sum;
  __syncthreads();
  const bool vec = vec_out != 0;
  for (int slot = tid; slot < (ntb1 - ntb0) * 64; slot += W * 64) {
    const int jj = slot >> 6;
    v4f v = red[(jj * S) * 64 + lane];
    for (int q = 1; q < S; ++q) v += red[(jj * S + q) * 64 + lane];
    const int mm = lane & 15;                    // slot lane == this thread's lane
    const int n = (ntb0 + jj) * kNTile + 4 * (lane >> 4);
    if (mm < M) store_out4(C, N, mm, n, N, v, tok_scale, vec);
  }
}

// (U, W, RP, AM). S = W / (n-tiles per workgroup) K splits per n-tile; a split holds at most U
// granules; M <= RP; K <= AM * (64 W / RP) * 16.
#define W4A8_STREAM_TABLE(X)                                                                      \
  X(20, 10, 8, 7) X(24, 10, 8, 7) X(12, 8, 8, 9) X(16, 8, 8, 9) X(20, 8, 8, 9) X(24, 8, 8, 9)     \
  X(12, 12, 8, 6) X(20, 6, 8, 12) X(8, 16, 8, 5) X(20, 10, 16, 14) X(12, 8, 16, 17)              \
  X(20, 8, 16, 17) X(12, 12, 16, 12)

#define W4A8_STREAM_CFG(u, w, rp, am) StreamCfg{rp, u, w, am},
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
  const StreamCfg c = kStream[variant];
  // RP rows + the zero row, then the split-reduction buffer
  const size_t act = c.mt == 8 ? red_offset_rp<8>(K) : red_offset_rp<16>(K);
  return act + (size_t)c.waves * 64 * sizeof(v4f);
}

// K splits per n-tile for a variant on this shape (0: the variant cannot serve it).
int stream_splits(int variant, int N, int K, int cus) {
  const StreamCfg c = kStream[variant];
  const int G = stream_grid(N, cus);
  const int ntmax = ceil_div(padded_n(N) / kNTile, G);
  const int S = c.waves / ntmax;
  if (S < 1 || K % 512) return 0;
  const int KT = K / kKTile;
  return 4 * ceil_div(KT / 4, S) <= c.t ? S : 0;
}

bool stream_fits(int variant, int M, int N, int K, int cus, size_t lds_limit) {
  const StreamCfg c = kStream[variant];
  if (K % 512 || M < 1 || M > c.mt || (long)K > (long)c.am * (64 * c.waves / c.mt) * 16) return false;
  const int ntiles = padded_n(N) / kNTile;
  const int G = stream_grid(N, cus);
  // every index the kernel forms stays in 32 bits
  const bool small = (long)(G + 1) * ntiles < (1L << 31) && (long)M * K < (1L << 31) &&
                     (long)(K / kKTile) * kGranuleBytes < (1L << 31);
  return small && G >= 1 && stream_splits(variant, N, K, cus) > 0 &&
         stream_lds_bytes(variant, M, K) <= lds_limit;
}

hipError_t launch_stream(const GemmArgs& g, int variant, int cus, hipStream_t stream) {
  const int KT = g.K / kKTile, KG = KT / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int S = stream_splits(variant, g.N, g.K, cus);
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(stream_grid(g.N, cus)), block(kStream[variant].waves * 64);
  const size_t lds = stream_lds_bytes(variant, g.M, g.K);
  int idx = 0;
#define W4A8_STREAM_LAUNCH(u, w, rp, am)                                                         \
  if (idx++ == variant) {                                                                        \
    if (lds > 64 * 1024) {                                                                       \
      const hipError_t e = hipFuncSetAttribute((const void*)gemm_stream<u, w, rp, am>,           \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                               (int)lds);                                        \
      if (e != hipSuccess) return e;                                                             \
    }                                                                                            \
    hipLaunchKernelGGL((gemm_stream<u, w, rp, am>), grid, block, lds, stream, g.a, g.a_scale,    \
                       g.wq, g.sq, g.c, g.M, g.N, g.K, KT, KG, NTILES, S, vec_out);              \
    return hipGetLastError();                                                                    \
  }
  W4A8_STREAM_TABLE(W4A8_STREAM_LAUNCH)
#undef W4A8_STREAM_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
