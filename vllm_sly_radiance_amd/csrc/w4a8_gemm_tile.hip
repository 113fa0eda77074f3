// Macro-tile W4A8 GEMM for prefill M on gfx950: LDS double-buffered scaled-MFMA tiles.
//
// Counterpart of the reference's folded / A-tiled prefill kernels
// (sly/mxfp4/radiance_mxfp4_fp8.hip:326-590, :664-944), redesigned for CDNA4:
//  * 4 wave64 in a 2 x 2 arrangement; each wave owns WM x WN MFMA tiles of 16 tokens x 16 columns,
//    so the workgroup tile is (32 WM) tokens x (32 WN) columns, one 128-k slab per stage.
//  * Stage = the activation slab in MFMA fragment order ([16-token block][run][lane][16 B]; run 0
//    holds k 16g..16g+15 and run 1 holds k 64+16g.. of fragment lane 16g + token) plus the weight
//    granules copied verbatim. Global loads are 128-bit and coalesced (granules are
//    contiguous 1 KiB; an activation row contributes 64 contiguous bytes per 16-lane group) and
//    every LDS write and ds_read_b128 touches 16 consecutive 16-byte slots per quarter-wave, so
//    neither side has bank conflicts. Two stages alternate with one barrier per slab; the next
//    slab's global loads are in flight while the current slab's MFMAs issue.
//  * The e8m0 scale dwords go straight from global (L2) to registers, one per n-fragment, issued
//    a slab ahead; the MFMA applies them, so no dequantisation happens anywhere.
//  * Workgroups are renumbered so each XCD (hardware places workgroup b on XCD b % 8) gets a
//    contiguous run of tiles, walked in groups of 8 row blocks, which keeps an XCD's activation
//    and weight panels in its own L2.
//  * Epilogue: lane holds 4 consecutive columns of one token; scaled by the per-token fp32 scale,
//    rounded to bf16 and stored 8 bytes at a time.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

constexpr int kThreads = 256;

template <int WM, int WN>
struct TileShape {
  static constexpr int BM = 2 * WM * 16;
  static constexpr int BN = 2 * WN * 16;
  static constexpr int A_BYTES = BM * kKTile;          // one fp8 slab
  static constexpr int W_BYTES = (BN / 16) * kGranuleBytes;
  static constexpr int STAGE = A_BYTES + W_BYTES;
  static constexpr int A_CHUNKS = A_BYTES / 16 / kThreads;   // 16-byte chunks per thread
  static constexpr int W_CHUNKS = W_BYTES / 16 / kThreads;
  static_assert(A_BYTES % (16 * kThreads) == 0 && W_BYTES % (16 * kThreads) == 0, "tile");
};

template <int WM, int WN>
__global__ __launch_bounds__(kThreads) void gemm_tile(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KTp,
    int KTe, int KG, int NTILES, int grid_m, int grid_n, int vec_out) {
  using S = TileShape<WM, WN>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * S::STAGE];

  // ---- tile order: XCD-contiguous runs, grouped by 8 row blocks ----
  const int total = grid_m * grid_n;
  int t = blockIdx.x;
  if (total % 8 == 0) t = (t % 8) * (total / 8) + t / 8;
  constexpr int GROUP = 8;
  const int per_group = GROUP * grid_n;
  const int first_m = (t / per_group) * GROUP;
  const int gm = min(grid_m - first_m, GROUP);
  const int bm = first_m + (t % per_group) % gm;
  const int bn = (t % per_group) / gm;
  const int m0 = bm * S::BM, nt_base = bn * (S::BN / 16);

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;

  // per-thread staging chunks
  uint4 ra[S::A_CHUNKS];
  v4i rw[S::W_CHUNKS];
  uint32_t sv[WN], sv_next[WN];

  auto load_slab = [&](int kt) {
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
      const int ch = tid + c * kThreads;           // (row block, 16-byte column, row in block)
      const int r16 = ch & 15, cc = (ch >> 4) & 7, rb = ch >> 7;
      const int row = m0 + rb * 16 + r16;
      const int kb = kt * kKTile + cc * 16;
      ra[c] = (row < M && kb < K) ? *reinterpret_cast<const uint4*>(A + (size_t)row * K + kb)
                                  : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < S::W_CHUNKS; ++c) {
      const int ch = tid + c * kThreads;
      const int nt = nt_base + (ch >> 6);
      rw[c] = nt < NTILES ? load_v4i_stream(Wq + (((size_t)nt * KTp + kt) * 64 + (ch & 63)) * 16)
                          : v4i{0, 0, 0, 0};
    }
  };
  auto load_scales = [&](int kt, uint32_t* dst) {
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int nt = nt_base + wn * WN + j;
      dst[j] = nt < NTILES ? Sq[((size_t)nt * KG + (kt >> 2)) * 64 + lane] >> (8 * (kt & 3))
                           : 127u;
    }
  };
  auto store_slab = [&](int buf) {
    uint8_t* sA = lds + buf * S::STAGE;
#pragma unroll
    for (int c = 0; c < S::A_CHUNKS; ++c) {
      const int ch = tid + c * kThreads;
      const int r16 = ch & 15, cc = (ch >> 4) & 7, rb = ch >> 7;
      // 16-byte column cc (k = 16 cc ..) of row r16 is run cc >> 2 of fragment lane (cc & 3) * 16 + r16
      *reinterpret_cast<uint4*>(sA + rb * 2048 + (cc >> 2) * 1024 + ((cc & 3) * 16 + r16) * 16) =
          ra[c];
    }
    uint8_t* sW = sA + S::A_BYTES;
#pragma unroll
    for (int c = 0; c < S::W_CHUNKS; ++c)
      *reinterpret_cast<v4i*>(sW + (tid + c * kThreads) * 16) = rw[c];
  };

  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  load_slab(0);
  load_scales(0, sv);
  store_slab(0);
  __syncthreads();

  for (int kt = 0; kt < KTe; ++kt) {
    const int buf = kt & 1;
    const bool more = kt + 1 < KTe;
    if (more) {
      load_slab(kt + 1);
      load_scales(kt + 1, sv_next);
    }
    const uint8_t* sA = lds + buf * S::STAGE;
    const uint8_t* sW = sA + S::A_BYTES;
    v4i wf[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j)
      wf[j] = *reinterpret_cast<const v4i*>(sW + (wn * WN + j) * kGranuleBytes + lane * 16);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const uint8_t* pa = sA + (wm * WM + i) * 2048 + lane * 16;
      const v4i lo = *reinterpret_cast<const v4i*>(pa);
      const v4i hi = *reinterpret_cast<const v4i*>(pa + 1024);
      const v8i xf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = mfma_w4a8(wf[j], xf, acc[i][j], sv[j]);
    }
    if (more) {
      store_slab(buf ^ 1);
#pragma unroll
      for (int j = 0; j < WN; ++j) sv[j] = sv_next[j];
    }
    __syncthreads();
  }

  const bool vec = vec_out != 0;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = m0 + (wm * WM + i) * 16 + (lane & 15);
    if (m >= M) continue;
    const float sc = As[m];
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = (nt_base + wn * WN + j) * kNTile + 4 * (lane >> 4);
      store_out4(C, N, m, n, N, acc[i][j], sc, vec);
    }
  }
}

#define W4A8_TILE_TABLE(X) X(2, 4) X(4, 4) X(8, 4) X(4, 8) X(8, 8)

#define W4A8_TILE_CFG(wm, wn) TileCfg{wm, wn, TileShape<wm, wn>::BM, TileShape<wm, wn>::BN},
constexpr TileCfg kTile[] = {W4A8_TILE_TABLE(W4A8_TILE_CFG)};
#undef W4A8_TILE_CFG
constexpr int kTileCount = sizeof(kTile) / sizeof(kTile[0]);

}  // namespace

int tile_variant_count() { return kTileCount; }
TileCfg tile_variant(int v) { return kTile[v]; }

hipError_t launch_tile(const GemmArgs& g, int variant, hipStream_t stream) {
  const TileCfg c = kTile[variant];
  const int KTp = padded_k(g.K) / kKTile, KTe = ceil_div(g.K, kKTile), KG = KTp / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int grid_m = ceil_div(g.M, c.bm), grid_n = ceil_div(g.N, c.bn);
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(grid_m * grid_n), block(kThreads);
  int idx = 0;
#define W4A8_TILE_LAUNCH(wm, wn)                                                                 \
  if (idx++ == variant) {                                                                        \
    hipLaunchKernelGGL((gemm_tile<wm, wn>), grid, block, 0, stream, g.a, g.a_scale, g.wq, g.sq,  \
                       g.c, g.M, g.N, g.K, KTp, KTe, KG, NTILES, grid_m, grid_n, vec_out);       \
    return hipGetLastError();                                                                    \
  }
  W4A8_TILE_TABLE(W4A8_TILE_LAUNCH)
#undef W4A8_TILE_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
