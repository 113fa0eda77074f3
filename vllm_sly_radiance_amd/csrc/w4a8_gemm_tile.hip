// Macro-tile W4A8 GEMM for prefill M on gfx950: scaled-MFMA tiles fed by an NS-stage LDS pipeline
// that the loads fill directly (buffer_load ... lds), with no register staging.
//
// Counterpart of the reference's folded / A-tiled prefill kernels
// (sly/mxfp4/radiance_mxfp4_fp8.hip:326-590, :664-944), redesigned for CDNA4:
//  * 4 wave64 in a 2 x 2 arrangement; each wave owns WM x WN MFMA tiles of 16 tokens x 16
//    columns (up to 128 x 128 per wave), so the workgroup tile is (32 WM) tokens x (32 WN) columns
//    and a 128-k slab is 32 WM * 128 B of activations, 2 WN weight granules and their scale dwords.
//  * One load instruction moves one 1 KiB unit of a slab straight into LDS: a weight granule
//    verbatim (already in MFMA fragment order), or 8 tokens x 128 k of activations. For the latter,
//    8 consecutive lanes read one token's 128-byte line: lanes that read scattered tokens instead
//    (the fragment order) cut the L2-to-LDS rate by 3.5x on MI355X. The LDS-direct form writes
//    lane l's 16 bytes at unit + 16 l, so each lane picks its chunk such that token R's chunk c
//    sits at slot 8 (R % 8) + (c ^ ((R / 2) % 8)): the ds_read_b128 fragment reads then touch
//    every bank once per 16 lanes.
//  * The fills go straight from memory to LDS, so the pipeline depth costs LDS, not registers:
//    NS stages, slab k+NS-1 requested while slab k is multiplied, its fills issued in shares
//    between the MFMA groups. One barrier per slab; the wait before it is explicit (every wave's
//    own fills of slab k), and the barrier is a bare s_barrier - __syncthreads' release fence
//    would wait for the younger slabs' fills too.
//  * Buffer resources bound every fill: the K tail, rows past M and n-tiles past N fill zeros.
//  * The e8m0 scale dwords change every 4 slabs (one dword per lane per k-group), so they live in
//    a ring of 3 k-groups outside the stages; each slab's fills carry a quarter of the next
//    k-group's rows. The MFMA applies the scales, so no dequantisation happens anywhere.
//  * Workgroups are renumbered so each XCD (hardware places workgroup b on XCD b % 8) gets a
//    contiguous run of tiles, walked in groups of 8 row blocks, which keeps an XCD's activation
//    and weight panels in its own L2.
//  * Epilogue: a lane holds 4 consecutive columns of one token; scaled by the per-token fp32 scale,
//    rounded to bf16 and stored 8 bytes at a time.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

constexpr int kThreads = 256;
constexpr int kOut = 0x7FFFFFF0;                 // an offset past every buffer resource here

template <int WM, int WN>
struct TileShape {
  static constexpr int BM = 2 * WM * 16;
  static constexpr int BN = 2 * WN * 16;
  static constexpr int A_UNITS = BM / 8;         // 1 KiB units per slab: 8 tokens x 128 k each
  static constexpr int W_UNITS = 2 * WN;         // weight granules per slab
  static constexpr int S_ROWS = 2 * WN;          // 256 B scale-dword rows per k-group (one per n-tile)
  static constexpr int A_PER_WAVE = A_UNITS / 4;
  static constexpr int W_PER_WAVE = ceil_div(W_UNITS, 4);
  static constexpr int S_QUARTER = ceil_div(S_ROWS, 4);        // rows filled per slab
  static constexpr int S_PER_WAVE = ceil_div(S_QUARTER, 4);
  static constexpr int OPS = A_PER_WAVE + W_PER_WAVE + S_PER_WAVE;   // fills per wave per slab
  // every wave issues the same number of fills; the surplus ones (past W_UNITS, or past a
  // quarter's scale rows) are zero fills into padding slots of their own
  static constexpr int W_OFF = A_UNITS * 1024;
  static constexpr int STAGE = W_OFF + 4 * W_PER_WAVE * 1024;
  // scale ring: 3 k-groups of S_ROWS rows, plus one junk row
  static constexpr int S_SLOT = (4 * S_QUARTER + 1) * 256;
  static_assert(A_UNITS % 4 == 0, "tile");
};

typedef __attribute__((address_space(3))) void* lds_ptr_t;

// s_waitcnt vmcnt(n) with lgkmcnt and expcnt left open (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// A workgroup barrier that orders the compiler's memory operations but emits no memory fence.
__device__ __forceinline__ void bare_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int WM, int WN, int NS>
__global__ __launch_bounds__(kThreads) void gemm_tile(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KTp,
    int KTe, int KG, int NTILES, int grid_m, int grid_n, int vec_out) {
  using S = TileShape<WM, WN>;
  static_assert(NS >= 2 && NS <= 5 && (NS - 2) * S::OPS < 64, "pipeline depth");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * S::STAGE + 3 * S::S_SLOT];
  uint8_t* const sring = lds + NS * S::STAGE;

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

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;

  // buffer resources: activations (all M x K), this tile's weight granules and scale dwords
  const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
  const int ntiles_here = min(S::BN / 16, NTILES - nt_base);
  const auto w_src = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Wq + (size_t)nt_base * KTp * kGranuleBytes), 0, ntiles_here * KTp * kGranuleBytes,
      kBufferWord3);
  const auto s_src = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(Sq + (size_t)nt_base * KG * 64), 0, ntiles_here * KG * 256, kBufferWord3);

  // Activation units: 8 consecutive lanes read one token's 128 k-bytes (one cache line), and the
  // 16 B chunks land XOR-swizzled so the fragment reads below hit every LDS bank once. Token R of
  // a 16-token block (unit 2b + R / 8) keeps chunk c at slot 8 (R % 8) + (c ^ ((R / 2) % 8)).
  const int a_row = lane >> 3;                              // token within the 8-token unit
  const int a_chunk = (lane & 7) ^ (a_row >> 1);            // chunk for even units; odd: ^ 4
  // MFMA fragment of lane l: token l % 16, chunks l / 16 and 4 + l / 16 of the 16-token block
  const int f_row = lane & 15;
  const int f_lo = 1024 * (f_row >> 3) + 16 * (8 * (f_row & 7) + ((lane >> 4) ^ ((f_row >> 1) & 7)));
  const int f_hi = f_lo ^ 64;                               // chunk + 4: slot bit 2 flips

  // Fill op o of slab kt into stage base: an activation unit (o < A_PER_WAVE), a weight granule,
  // or a scale row. Scale rows are per k-group of 4 slabs: the fills of slab kt carry quarter
  // kt % 4 of the rows of k-group kt / 4 + 1, into ring slot (kt / 4 + 1) % 3.
  auto fill_op = [&](int kt, uint8_t* base, int o) {
    const bool kin = kt < KTe;
    if (o < S::A_PER_WAVE) {
      const int unit = wave * S::A_PER_WAVE + o;
      const int row = m0 + unit * 8 + a_row;
      const int col = kt * kKTile + 16 * (a_chunk ^ ((unit & 1) << 2));
      const int off = (kin & (col < K) & (row < M)) ? row * K + col : kOut;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_src, (lds_ptr_t)(base + unit * 1024), 16, off, 0,
                                               0, 0);
    } else if (o < S::A_PER_WAVE + S::W_PER_WAVE) {
      const int g = wave * S::W_PER_WAVE + (o - S::A_PER_WAVE);
      const int off = (kin & (g < S::W_UNITS)) ? (g * KTp + kt) * kGranuleBytes + lane * 16 : kOut;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_src, (lds_ptr_t)(base + S::W_OFF + g * 1024), 16,
                                               off, 0, 0, kBufferNT);
    } else {
      const int grp = (kt >> 2) + 1, q = kt & 3;
      const int i = wave * S::S_PER_WAVE + (o - S::A_PER_WAVE - S::W_PER_WAVE);
      const int r = q * S::S_QUARTER + i;
      const bool real = (i < S::S_QUARTER) & (r < S::S_ROWS);
      const int off = (real & (grp < KG)) ? ((r * KG + grp) * 64 + lane) * 4 : kOut;
      const int slot = grp % 3;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          s_src, (lds_ptr_t)(sring + slot * S::S_SLOT + (real ? r : 4 * S::S_QUARTER) * 256), 4,
          off, 0, 0, 0);
    }
  };
  auto fill = [&](int kt, int st) {
    uint8_t* base = lds + st * S::STAGE;
#pragma unroll
    for (int o = 0; o < S::OPS; ++o) fill_op(kt, base, o);
  };

  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Multiply slab kt out of stage st while issuing the fills of slab fkt into stage fst: fragment
  // i+1 is read and a share of the fills is issued before fragment i's MFMAs, and a scheduling
  // barrier keeps the compiler from sinking them below the MFMAs.
  auto compute = [&](int st, int kt, int fkt, int fst) {
    const uint8_t* base = lds + st * S::STAGE;
    uint8_t* fbase = lds + fst * S::STAGE;
    const uint8_t* srow = sring + ((kt >> 2) % 3) * S::S_SLOT + lane * 4;
    v4i wf[WN];
    uint32_t sc[WN];
    const int sh = 8 * (kt & 3);
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      wf[j] = *reinterpret_cast<const v4i*>(base + S::W_OFF + (wn * WN + j) * 1024 + lane * 16);
      sc[j] = *reinterpret_cast<const uint32_t*>(srow + (wn * WN + j) * 256) >> sh;
    }
    const uint8_t* pa = base + wm * WM * 2048;
    v4i lo = *reinterpret_cast<const v4i*>(pa + f_lo), hi = *reinterpret_cast<const v4i*>(pa + f_hi);
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const v8i xf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      if (i + 1 < WM) {
        lo = *reinterpret_cast<const v4i*>(pa + (i + 1) * 2048 + f_lo);
        hi = *reinterpret_cast<const v4i*>(pa + (i + 1) * 2048 + f_hi);
      }
#pragma unroll
      for (int o = i * S::OPS / WM; o < (i + 1) * S::OPS / WM; ++o) fill_op(fkt, fbase, o);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < WN; ++j) acc[i][j] = mfma_w4a8(wf[j], xf, acc[i][j], sc[j]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- NS-stage pipeline: slab kt+NS-1 is requested while slab kt is multiplied ----
  // k-group 0's scale rows first (4 quarters), so the wait for slab 0 covers them too
  {
    const int i = wave * S::S_PER_WAVE;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < S::S_PER_WAVE; ++e) {
        const int r = q * S::S_QUARTER + i + e;
        const bool real = (i + e < S::S_QUARTER) & (r < S::S_ROWS);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            s_src, (lds_ptr_t)(sring + (real ? r : 4 * S::S_QUARTER) * 256), 4,
            real ? (r * KG * 64 + lane) * 4 : kOut, 0, 0, 0);
      }
  }
#pragma unroll
  for (int p = 0; p < NS - 1; ++p) fill(p, p);
  int st = 0;
  for (int kt = 0; kt < KTe; ++kt) {
    wait_vmcnt<(NS - 2) * S::OPS>();             // this wave's fills of slab kt have landed
    bare_barrier();                              // ... and every wave's; slab kt-1 is consumed
    const int nxt = st == 0 ? NS - 1 : st - 1;   // stage of slab kt+NS-1 == stage of slab kt-1
    compute(st, kt, kt + NS - 1, nxt);           // issues slab kt+NS-1's fills in shares
    st = st + 1 == NS ? 0 : st + 1;
  }
  wait_vmcnt<0>();                               // no fill may outlive the workgroup's LDS

  // per-token scales of this lane's WM tokens, all requested before the first is used
  const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
  float tsc[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = m0 + (wm * WM + i) * 16 + (lane & 15);
    tsc[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           as_src, m < M ? m * 4 : kOut, 0, 0));
  }
  const bool vec = vec_out != 0;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = m0 + (wm * WM + i) * 16 + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = (nt_base + wn * WN + j) * kNTile + 4 * (lane >> 4);
      store_out4(C, N, m, n, N, acc[i][j], tsc[i], vec);
    }
  }
}

// (WM, WN, NS): wave tile 16 WM x 16 WN, NS-stage LDS pipeline (LDS = NS * STAGE <= 160 KiB)
#define W4A8_TILE_TABLE(X)                                                                        \
  X(2, 4, 4) X(4, 4, 3) X(4, 4, 4) X(8, 4, 3) X(4, 8, 3) X(8, 8, 3) X(8, 5, 3) X(4, 8, 4)          \
  X(4, 2, 4) X(1, 2, 4) X(2, 2, 4) X(1, 4, 4) X(2, 2, 5)

#define W4A8_TILE_CFG(wm, wn, ns) TileCfg{wm, wn, TileShape<wm, wn>::BM, TileShape<wm, wn>::BN},
constexpr TileCfg kTile[] = {W4A8_TILE_TABLE(W4A8_TILE_CFG)};
#undef W4A8_TILE_CFG
constexpr int kTileCount = sizeof(kTile) / sizeof(kTile[0]);

}  // namespace

int tile_variant_count() { return kTileCount; }
TileCfg tile_variant(int v) { return kTile[v]; }

bool tile_fits(int M, int N, int K) {
  // 32-bit buffer offsets: the activations and one tile's weight stripe
  return (long)M * K < (1L << 31) && (long)16 * padded_k(K) / 2 * 16 < (1L << 31) &&
         (long)N < (1L << 24);
}

hipError_t launch_tile(const GemmArgs& g, int variant, hipStream_t stream) {
  const TileCfg c = kTile[variant];
  const int KTp = padded_k(g.K) / kKTile, KTe = ceil_div(g.K, kKTile), KG = KTp / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int grid_m = ceil_div(g.M, c.bm), grid_n = ceil_div(g.N, c.bn);
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(grid_m * grid_n), block(kThreads);
  int idx = 0;
#define W4A8_TILE_LAUNCH(wm, wn, ns)                                                           \
  if (idx++ == variant) {                                                                        \
    hipLaunchKernelGGL((gemm_tile<wm, wn, ns>), grid, block, 0, stream, g.a, g.a_scale, g.wq,  \
                       g.sq,                                                                      \
                       g.c, g.M, g.N, g.K, KTp, KTe, KG, NTILES, grid_m, grid_n, vec_out);       \
    return hipGetLastError();                                                                    \
  }
  W4A8_TILE_TABLE(W4A8_TILE_LAUNCH)
#undef W4A8_TILE_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
