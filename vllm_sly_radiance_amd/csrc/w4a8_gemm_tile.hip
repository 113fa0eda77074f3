// Macro-tile W4A8 GEMM for prefill M on gfx950: scaled-MFMA tiles fed by an NS-stage LDS pipeline
// that the loads fill directly (buffer_load ... lds), with no register staging.
//
// Counterpart of the reference's folded / A-tiled prefill kernels
// (sly/mxfp4/radiance_mxfp4_fp8.hip:326-590, :664-944), redesigned for CDNA4:
//  * NW wave64 (4 or 8) in an (NW / 2) x 2 arrangement; each wave owns WM x WN MFMA tiles of 16
//    tokens x 16 columns, so the workgroup tile is (8 NW WM) tokens x (32 WN) columns (up to
//    256 x 256) and a 128-k slab is 8 NW WM * 128 B of activations, 2 WN weight granules and their
//    scale dwords.
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
//    a ring of k-groups outside the stages (ring_slots(NS) of them: enough that no refill lands
//    on a k-group some slab still reads); every fourth slab's fills carry the rows of a k-group
//    ahead. The MFMA applies the scales, so no dequantisation happens anywhere.
//  * Workgroups are renumbered so each XCD (hardware places workgroup b on XCD b % 8) gets a
//    contiguous run of tiles, walked in groups of 8 row blocks, which keeps an XCD's activation
//    and weight panels in its own L2.
//  * Epilogue: a lane holds 4 consecutive columns of one token; scaled by the per-token fp32 scale,
//    rounded to bf16 and stored 8 bytes at a time.
//  * AT = true reads the activations in the fragment-tiled layout the producers can write (16-token
//    blocks of 16 x K bytes; in block b, k-tile t, half h, lane l's 16 bytes at
//    ((b KT + t) 2 + h) 1024 + 16 l are token 16 b + l % 16, k-bytes 128 t + 16 (4 h + l / 16)):
//    each activation unit is then one contiguous KiB, copied to LDS as it is, and the fragment
//    reads are lane-contiguous. Only the addresses differ, so both layouts give the same bits.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

constexpr int kOut = 0x7FFFFFF0;                 // an offset past every buffer resource here

// NW waves in an (NW / 2) x 2 arrangement, each owning WM x WN MFMA tiles of 16 x 16.
template <int WM, int WN, int NW>
struct TileShape {
  static constexpr int WVM = NW / 2, WVN = 2;
  static constexpr int BM = WVM * WM * 16;
  static constexpr int BN = WVN * WN * 16;
  static constexpr int A_UNITS = BM / 8;         // 1 KiB units per slab: 8 tokens x 128 k each
  static constexpr int W_UNITS = BN / 16;        // weight granules per slab
  static constexpr int S_ROWS = BN / 16;         // 256 B scale-dword rows per k-group (one per n-tile)
  static constexpr int A_PER_WAVE = A_UNITS / NW;
  static constexpr int W_PER_WAVE = ceil_div(W_UNITS, NW);
  // Every slab, each wave fills OPS units (activations and weight granules; surplus granule slots
  // past W_UNITS are zero fills into padding units of their own). Every fourth slab each wave
  // also fills one 1 KiB scale unit, 4 rows of the next k-group (waves past S_OPS fill a junk
  // unit), so a k-group's rows take one fill per wave instead of one 4-byte fill per row.
  static constexpr int OPS = A_PER_WAVE + W_PER_WAVE;
  static constexpr int S_OPS = ceil_div(S_ROWS, 4);          // 1 KiB scale units per k-group
  static constexpr int W_OFF = A_UNITS * 1024;
  static constexpr int STAGE = W_OFF + NW * W_PER_WAVE * 1024;
  // scale ring: 3 k-groups of S_ROWS rows (rounded up to whole units)
  static constexpr int S_SLOT = S_OPS * 1024;
  // the tile's per-token fp32 scales, one 256-byte row per 64 tokens
  static constexpr int TSCALE = 256 * ceil_div(BM, 64);
  static_assert(NW % 2 == 0 && A_UNITS % NW == 0 && S_OPS <= NW, "tile");
  // fills one wave issues for slab s: the scale unit rides with every slab s % 4 == 0
  static constexpr int fills(int s) { return OPS + (s % 4 == 0 ? 1 : 0); }
  // fills issued for slabs s0 + 1 .. s0 + n (all younger than slab s0's), s0 known modulo 4
  static constexpr int fills_after(int s0, int n) {
    int t = 0;
    for (int d = 1; d <= n; ++d) t += fills(s0 + d);
    return t;
  }
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

template <int Q>
struct IntC {
  static constexpr int value = Q;
};

// k-groups in the scale ring of an NS-stage pipeline. The refill issued during slab kt (after its
// barrier) is slab kt + NS - 1 (kt + NS on the deep-tile path) and, when that slab starts a
// k-group, carries the rows of the k-group after it, g' = (kt + NS - 1) / 4 + 1. It lands on the
// slot of k-group g' - R, which slabs up to 4 (g' - R) + 3 read (the deep-tile path reads a
// group's rows once, at slab 4 g - 1). Those reads must precede slab kt, so 4 (g' - R) + 3 < kt,
// which holds for NS < 4 R - 6: R = 3 up to 5 stages, 4 up to 9, 5 up to 13, 6 up to 17.
constexpr int ring_slots(int ns) { return ns + 6 < 12 ? 3 : (ns + 6) / 4 + 1; }
// every depth the kernel accepts: enough slots (NS < 4 R - 6), and no more than that needs
// (tests/test_tile_scale_ring_cpu.py checks the condition against a model of the schedule)
constexpr bool ring_slots_hold() {
  for (int ns = 2; ns <= 16; ++ns) {
    const int r = ring_slots(ns);
    if (ns >= 4 * r - 6 || (r > 3 && ns < 4 * (r - 1) - 6)) return false;
  }
  return true;
}
static_assert(ring_slots_hold(), "scale ring: NS < 4 R - 6");

// The kernel body; the two entry points below differ only in the order of their arguments.
// SPLIT: K split over workgroup rows. Row blockIdx.y = s of `splits` covers the k-groups
// [KG s / splits, KG (s + 1) / splits) and writes its unscaled fp32 sums to P[s][M][N] (N % 16 == 0);
// split_reduce adds them in split order, scales and rounds. A compile-time switch: the unsplit
// kernels keep exactly their own code (a run-time k-range cost the 256 x 256 tile 20 spilled
// registers and 28 % of its speed).
template <int WM, int WN, int NS, int NW, bool AT, bool SPLIT>
__device__ __forceinline__ void tile_body(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KTp,
    int KTe, int KG, int NTILES, int grid_m, int grid_n, int ldc, int vec_out,
    float* __restrict__ P, int splits) {
  using S = TileShape<WM, WN, NW>;
  static_assert(NS >= 2 && NS <= 16 && (NS - 1) * (S::OPS + 1) < 64, "pipeline depth");
  constexpr int RING = ring_slots(NS);
  __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * S::STAGE + RING * S::S_SLOT + 1024 +
                                                         S::TSCALE];
  uint8_t* const sring = lds + NS * S::STAGE;
  uint8_t* const junk = sring + RING * S::S_SLOT;  // where the surplus scale fills land
  uint8_t* const tscale = junk + 1024;             // the tile's per-token fp32 scales

  // ---- tile order: XCD-contiguous runs, grouped by 8 row blocks. Unsigned, and no division at
  //      all for one row of tiles (the decode band): the workgroup's waves share one scalar unit,
  //      and this runs before their first requests ----
  constexpr unsigned GROUP = 8;
  const unsigned total = (unsigned)(grid_m * grid_n);
  unsigned t = blockIdx.x;
  if ((total & 7) == 0) t = (t & 7) * (total >> 3) + (t >> 3);
  unsigned bm = 0, bn = t;
  if (grid_m > 1) {
    const unsigned per_group = GROUP * (unsigned)grid_n;
    const unsigned grp = t / per_group, r = t - grp * per_group;
    const unsigned first_m = grp * GROUP;
    const unsigned gm = min((unsigned)grid_m - first_m, GROUP);
    bn = r / gm;
    bm = first_m + (r - bn * gm);
  }
  const int m0 = (int)bm * S::BM, nt_base = (int)bn * (S::BN / 16);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;      // (NW / 2) x 2 waves

  // this workgroup's slabs: whole k-groups [kt0, kt1); fills at or past kend read zero
  const int split = SPLIT ? (int)blockIdx.y : 0;
  const int kt0 = SPLIT ? 4 * (KG * split / splits) : 0;
  const int kt1 = SPLIT ? 4 * (KG * (split + 1) / splits) : (KTe + 3) & ~3;
  const int kend = SPLIT ? min(kt1, KTe) : KTe;

  // buffer resources: activations (all M x K; tiled: whole 16-token blocks), this tile's weight
  // granules and scale dwords
  const int mblocks = ceil_div(M, 16);
  const auto a_src =
      __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, AT ? mblocks * 16 * K : M * K, kBufferWord3);
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
  // (tiled: the block's two halves as they are)
  const int f_row = lane & 15;
  const int f_lo =
      AT ? 16 * lane
         : 1024 * (f_row >> 3) + 16 * (8 * (f_row & 7) + ((lane >> 4) ^ ((f_row >> 1) & 7)));
  const int f_hi = AT ? f_lo + 1024 : f_lo ^ 64;            // chunk + 4: slot bit 2 flips

  // Fill op o of slab kt into stage base: an activation unit (o < A_PER_WAVE) or a weight granule.
  auto fill_op = [&](int kt, uint8_t* base, int o) {
    const bool kin = kt < kend;
    if (o < S::A_PER_WAVE) {
      const int unit = wave * S::A_PER_WAVE + o;
      int off;
      if constexpr (AT) {
        // unit = half (unit & 1) of the tile's 16-token block unit / 2; K is whole k-tiles
        const int blk = (m0 >> 4) + (unit >> 1);
        off = (kin & (blk < mblocks)) ? ((blk * KTe + kt) * 2 + (unit & 1)) * 1024 + lane * 16
                                      : kOut;
      } else {
        const int row = m0 + unit * 8 + a_row;
        const int col = kt * kKTile + 16 * (a_chunk ^ ((unit & 1) << 2));
        off = (kin & (col < K) & (row < M)) ? row * K + col : kOut;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(a_src, (lds_ptr_t)(base + unit * 1024), 16, off, 0,
                                               0, 0);
    } else if (o < S::A_PER_WAVE + S::W_PER_WAVE) {
      const int g = wave * S::W_PER_WAVE + (o - S::A_PER_WAVE);
      const int off = (kin & (g < S::W_UNITS)) ? (g * KTp + kt) * kGranuleBytes + lane * 16 : kOut;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(w_src, (lds_ptr_t)(base + S::W_OFF + g * 1024), 16,
                                               off, 0, 0, kBufferNT);
    }
  };
  // Scale unit of k-group grp into ring slot grp % RING: wave w < S_OPS moves rows 4w .. 4w+3 (lanes
  // 16 r .. 16 r + 15 read row 4w + r's 256 bytes, which land contiguously); the other waves move
  // zeros into the junk unit. Rows past S_ROWS or k-groups past KG read zero.
  auto fill_scales = [&](int grp) {
    const int r = 4 * wave + (lane >> 4);
    const bool mine = wave < S::S_OPS;
    const int off = (mine & (r < S::S_ROWS) & (grp < KG)) ? (r * KG + grp) * 256 + (lane & 15) * 16
                                                          : kOut;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        s_src, (lds_ptr_t)(mine ? sring + (grp % RING) * S::S_SLOT + wave * 1024 : junk), 16, off, 0,
        0, 0);
  };
  // Fill op o < S::fills(kt) of slab kt: the slab's units, then (kt % 4 == 0) k-group kt/4 + 1's
  // scale unit, which slabs 4 (kt/4 + 1) .. + 3 read.
  auto fill_any = [&](int kt, uint8_t* base, int o) {
    if (o < S::OPS) fill_op(kt, base, o);
    else fill_scales((kt >> 2) + 1);
  };
  auto fill = [&](int kt, int st) {
    uint8_t* base = lds + st * S::STAGE;
#pragma unroll
    for (int o = 0; o < S::OPS; ++o) fill_op(kt, base, o);
    if ((kt & 3) == 0) fill_scales((kt >> 2) + 1);
  };

  v4f acc[WM][WN];
#pragma unroll
  for (int i = 0; i < WM; ++i)
#pragma unroll
    for (int j = 0; j < WN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  // Fragment reads: this wave's weight fragments and scale dwords of slab kt from stage st (the
  // MFMA takes the dword's byte kt % 4: shift it by 8 (kt % 4) where it is used), and its
  // activation fragment i (tokens 16 (wm WM + i) ..) of the same stage.
  auto read_w = [&](int st, int kt, v4i* wf, uint32_t* sc) {
    const uint8_t* base = lds + st * S::STAGE;
    const uint8_t* srow = sring + ((kt >> 2) % RING) * S::S_SLOT + lane * 4;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      wf[j] = *reinterpret_cast<const v4i*>(base + S::W_OFF + (wn * WN + j) * 1024 + lane * 16);
      sc[j] = *reinterpret_cast<const uint32_t*>(srow + (wn * WN + j) * 256);
    }
  };
  auto read_a = [&](int st, int i, v4i& lo, v4i& hi) {
    const uint8_t* pa = lds + st * S::STAGE + (wm * WM + i) * 2048;
    lo = *reinterpret_cast<const v4i*>(pa + f_lo);
    hi = *reinterpret_cast<const v4i*>(pa + f_hi);
  };

  // The epilogue's per-token scales (the tile's BM tokens) go straight to LDS before anything
  // else: they are older than every fill, so the first fill wait and barrier cover them, and their
  // latency hides under the main loop at no register cost.
  {
    const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
    const int r = wave * 64 + lane;
    if (wave * 64 < S::BM)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(as_src, (lds_ptr_t)(tscale + wave * 256), 4,
                                               (r < S::BM && m0 + r < M) ? (m0 + r) * 4 : kOut,
                                               0, 0, 0);
  }

  // the first k-group's scale unit goes out first, so the wait for the first slab covers it too
  fill_scales(kt0 >> 2);

  // The k-loops run whole k-groups (4 slabs, the last group padded with zero slabs: the weight
  // stripes are padded to whole k-groups and activations past K fill zeros), unrolled so that
  // every slab knows at compile time whether its refill carries a scale unit, and so how many
  // fills its wait may leave in flight.

  if constexpr (WM >= 3) {
    // ---- NS-stage pipeline, barrier two MFMA groups before the end of each slab. At the
    //      barrier of slab kt every wave has its own fills of slab kt+1 landed and has finished
    //      every read of slab kt; past it, the wave reads slab kt+1's weight fragments, scales
    //      and first activation fragment, and refills slab kt's stage with slab kt+NS, while the
    //      last two groups of slab kt's MFMAs run. A slab is requested NS-1 slabs before its
    //      barrier, and no wave idles at a barrier with an empty MFMA queue behind it. ----
    // MFMA groups past the barrier: 3, or 2 for the 8-wave 256-wide tile, whose waves have 256
    // registers each (the third group's fragments would spill)
    constexpr int R = WM >= 4 ? ((NW == 8 && WN >= 8) ? 2 : 3) : 2;
    constexpr int P = WM - R;
#pragma unroll
    for (int p = 0; p < NS; ++p) fill(kt0 + p, p);
    wait_vmcnt<S::fills_after(0, NS - 1)>();     // the first slab and its scales have landed
    bare_barrier();
    v4i wf[WN], lo, hi;
    uint32_t sc[WN];
    read_w(0, kt0, wf, sc);
    read_a(0, 0, lo, hi);
    __builtin_amdgcn_s_waitcnt(0xC07F);          // lgkmcnt(0): the loop starts with nothing pending
    int st = 0;
    auto slab = [&](int kt, auto qc) {
      constexpr int q = decltype(qc)::value;    // kt % 4
      constexpr int NF = S::fills(q + NS);       // fills of the refill, slab kt + NS
      asm volatile("" : "+s"(kt));               // kt opaque: no per-copy loop invariants
      const int nst = st + 1 == NS ? 0 : st + 1;
      uint8_t* fbase = lds + st * S::STAGE;      // slab kt's stage, refilled with slab kt+NS
      v4i wfn[WN], lon, hin;
      uint32_t scn[WN];
      v8i xr[R];                                 // fragments of groups P.., read before the barrier
#pragma unroll
      for (int i = 0; i < P; ++i) {
        const v8i xf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        if (i + 1 < P) {
          read_a(st, i + 1, lo, hi);
        } else {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            v4i l, h;
            read_a(st, P + r, l, h);
            xr[r] = v8i{l[0], l[1], l[2], l[3], h[0], h[1], h[2], h[3]};
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = mfma_w4a8(wf[j], xf, acc[i][j], sc[j] >> (8 * q));
        __builtin_amdgcn_sched_barrier(0);
      }
      {
        // the last R groups: their fragments are read before the barrier; past it, the next
        // slab's fragment reads and this slab's refill go out one or two per MFMA, so the MFMA
        // queue never waits behind a run of memory instructions
        wait_vmcnt<S::fills_after(q + 1, NS - 2)>();  // this wave's fills of slab kt+1 landed
        __builtin_amdgcn_s_waitcnt(0xC07F);      // lgkmcnt(0): this wave's reads of slab kt done
        bare_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* nbase = lds + nst * S::STAGE;
        const uint8_t* srow = sring + (((kt + 1) >> 2) % RING) * S::S_SLOT + lane * 4;
#pragma unroll
        for (int m = 0; m < R * WN; ++m) {
          const int r = m / WN, j = m % WN;
          acc[P + r][j] = mfma_w4a8(wf[j], xr[r], acc[P + r][j], sc[j] >> (8 * q));
          __builtin_amdgcn_sched_barrier(0);
          if (m < WN) {
            wfn[m] = *reinterpret_cast<const v4i*>(nbase + S::W_OFF + (wn * WN + m) * 1024 +
                                                   lane * 16);
            // a k-group's scale dwords serve its 4 slabs: read them only for its first slab
            if constexpr (q == 3)
              scn[m] = *reinterpret_cast<const uint32_t*>(srow + (wn * WN + m) * 256);
          }
          if (m == WN) read_a(nst, 0, lon, hin);
#pragma unroll
          for (int o = m * NF / (R * WN); o < (m + 1) * NF / (R * WN); ++o)
            fill_any(kt + NS, fbase, o);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
      // slab kt+1's fragments (read right after the barrier, a group of MFMAs ago) are in: said
      // here, the compiler does not make the next slab's first MFMAs wait on every LDS read
      __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        wf[j] = wfn[j];
        if constexpr (q == 3) sc[j] = scn[j];
      }
      lo = lon;
      hi = hin;
      st = nst;
    };
    for (int kt = kt0; kt < kt1; kt += 4) {
      slab(kt, IntC<0>{});
      slab(kt + 1, IntC<1>{});
      slab(kt + 2, IntC<2>{});
      slab(kt + 3, IntC<3>{});
    }
  } else {
    // ---- NS-stage pipeline, barrier at the head of each slab: slab kt+NS-1 is requested in
    //      shares between the MFMA groups of slab kt; fragment i+1 is read before fragment i's
    //      MFMAs, and scheduling barriers keep the compiler from sinking either below them ----
#pragma unroll
    for (int p = 0; p < NS - 1; ++p) fill(kt0 + p, p);
    int st = 0;
    auto slab = [&](int kt, auto qc) {
      constexpr int q = decltype(qc)::value;    // kt % 4
      constexpr int NF = S::fills(q + NS - 1);   // fills of the refill, slab kt + NS - 1
      wait_vmcnt<S::fills_after(q, NS - 2)>();   // this wave's fills of slab kt have landed
      bare_barrier();                            // ... and every wave's; slab kt-1 is consumed
      const int fst = st == 0 ? NS - 1 : st - 1; // stage of slab kt+NS-1 == stage of slab kt-1
      uint8_t* fbase = lds + fst * S::STAGE;
      v4i wf[WN], lo, hi;
      uint32_t sc[WN];
      read_w(st, kt, wf, sc);
      read_a(st, 0, lo, hi);
#pragma unroll
      for (int i = 0; i < WM; ++i) {
        const v8i xf = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        if (i + 1 < WM) read_a(st, i + 1, lo, hi);
#pragma unroll
        for (int o = i * NF / WM; o < (i + 1) * NF / WM; ++o)
          fill_any(kt + NS - 1, fbase, o);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < WN; ++j)
          acc[i][j] = mfma_w4a8(wf[j], xf, acc[i][j], sc[j] >> (8 * q));
        __builtin_amdgcn_sched_barrier(0);
      }
      st = st + 1 == NS ? 0 : st + 1;
    };
    for (int kt = kt0; kt < kt1; kt += 4) {
      slab(kt, IntC<0>{});
      slab(kt + 1, IntC<1>{});
      slab(kt + 2, IntC<2>{});
      slab(kt + 3, IntC<3>{});
    }
  }
  wait_vmcnt<0>();                               // no fill may outlive the workgroup's LDS

  if constexpr (SPLIT) {
    // split K: this k-range's unscaled sums, 4 consecutive columns of one token per lane
    float* const ps = P + (size_t)split * M * N;
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int m = m0 + (wm * WM + i) * 16 + (lane & 15);
      if (m >= M) continue;
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int n = (nt_base + wn * WN + j) * kNTile + 4 * (lane >> 4);
        if (n < N) *reinterpret_cast<v4f*>(ps + (size_t)m * N + n) = acc[i][j];
      }
    }
    return;
  }

  float tsc[WM];
#pragma unroll
  for (int i = 0; i < WM; ++i)
    tsc[i] = reinterpret_cast<const float*>(tscale)[(wm * WM + i) * 16 + (lane & 15)];

  // Epilogue. A lane holds 4 consecutive columns of one token per MFMA tile, so direct stores
  // touch 16 rows per instruction (measured: ~7.5 us per 256 x 256 tile on MI355X). A full tile
  // is therefore staged through the freed pipeline stages, row-major with a 16-byte row pad, and
  // written out as 16-byte row-contiguous stores; edge tiles store directly.
  constexpr int OROW = S::BN * 2 + 16;
  constexpr bool kStaged = S::BM * OROW <= NS * S::STAGE;
  if (kStaged && vec_out == 2 && m0 + S::BM <= M && nt_base * kNTile + S::BN <= N) {
    bare_barrier();                              // every wave is done with the stages
#pragma unroll
    for (int i = 0; i < WM; ++i) {
      const int r = (wm * WM + i) * 16 + (lane & 15);
#pragma unroll
      for (int j = 0; j < WN; ++j) {
        const int col = (wn * WN + j) * kNTile + 4 * (lane >> 4);
        const v4f v = acc[i][j];
        // the hardware convert (bf16x2_rne: 4 operations per pair against ~11) wherever it leaves
        // the main loop's register allocation alone; the fragment-tiled 256 x 256 tile would spill
        // in its k-loop with it, so that form keeps the software rounding (the same bits)
        uint2 b;
        if constexpr (!AT) {
          b = make_uint2(bf16x2_rne(v[0] * tsc[i], v[1] * tsc[i]),
                         bf16x2_rne(v[2] * tsc[i], v[3] * tsc[i]));
        } else {
          b = make_uint2(f32_to_bf16(v[0] * tsc[i]) | (f32_to_bf16(v[1] * tsc[i]) << 16),
                         f32_to_bf16(v[2] * tsc[i]) | (f32_to_bf16(v[3] * tsc[i]) << 16));
        }
        *reinterpret_cast<uint2*>(lds + r * OROW + col * 2) = b;
      }
    }
    __syncthreads();
    constexpr int CH = S::BN * 2 / 16;           // 16-byte chunks per row
    uint16_t* const crow = C + (size_t)m0 * ldc + nt_base * kNTile;
    for (int idx = tid; idx < S::BM * CH; idx += NW * 64) {
      const int r = idx / CH, c = idx - r * CH;
      *reinterpret_cast<v4i*>(crow + (size_t)r * ldc + c * 8) =
          *reinterpret_cast<const v4i*>(lds + r * OROW + c * 16);
    }
    return;
  }
  const bool vec = vec_out != 0;
#pragma unroll
  for (int i = 0; i < WM; ++i) {
    const int m = m0 + (wm * WM + i) * 16 + (lane & 15);
    if (m >= M) continue;
#pragma unroll
    for (int j = 0; j < WN; ++j) {
      const int n = (nt_base + wn * WN + j) * kNTile + 4 * (lane >> 4);
      store_out4(C, ldc, m, n, N, acc[i][j], tsc[i], vec);
    }
  }
}

// Entry points. The first 14 argument dwords arrive in SGPRs at wave launch (kernarg preloading),
// so gemm_tile_pre puts what the first requests depend on there and derives KTe and KG: the
// 32- and 64-token tiles of the decode band (4 waves), whose launches are short, measured
// 0.15-0.25 us faster with it. The larger tiles keep the original order, with which their
// register allocation spills least (the 8-wave 256 x 256 tile measured 8 % slower with the other).
template <int WM, int WN, int NS, int NW, bool AT>
__global__ __launch_bounds__(NW * 64) void gemm_tile(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KTp,
    int KTe, int KG, int NTILES, int grid_m, int grid_n, int ldc, int vec_out) {
  tile_body<WM, WN, NS, NW, AT, false>(A, As, Wq, Sq, C, M, N, K, KTp, KTe, KG, NTILES, grid_m,
                                       grid_n, ldc, vec_out, nullptr, 1);
}

template <int WM, int WN, int NS, int NW, bool AT>
__global__ __launch_bounds__(NW * 64) void gemm_tile_pre(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, int M, int K, int KTp, int NTILES, int grid_m, int grid_n,
    int N, int ldc, int vec_out, uint16_t* __restrict__ C) {
  tile_body<WM, WN, NS, NW, AT, false>(A, As, Wq, Sq, C, M, N, K, KTp, ceil_div(K, kKTile),
                                       KTp / kKGroup, NTILES, grid_m, grid_n, ldc, vec_out,
                                       nullptr, 1);
}

// The K-split form of the 4-wave band tiles (WM <= 2): the preloaded argument order of
// gemm_tile_pre, then the partials and the split count.
template <int WM, int WN, int NS, int NW, bool AT>
__global__ __launch_bounds__(NW * 64) void gemm_tile_split(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, int M, int K, int KTp, int NTILES, int grid_m, int grid_n,
    int N, int splits, float* __restrict__ P) {
  tile_body<WM, WN, NS, NW, AT, true>(A, As, Wq, Sq, nullptr, M, N, K, KTp, ceil_div(K, kKTile),
                                      KTp / kKGroup, NTILES, grid_m, grid_n, N, 0, P, splits);
}


// (WM, WN, NS, NW): NW waves of 16 WM x 16 WN in an (NW / 2) x 2 arrangement, NS-stage LDS
// pipeline (LDS = NS * STAGE + ring_slots(NS) scale slots + token scales <= 160 KiB)
#define W4A8_TILE_TABLE(X)                                                                        \
  X(2, 4, 4, 4) X(4, 4, 3, 4) X(4, 4, 4, 4) X(8, 4, 3, 4) X(4, 8, 3, 4) X(8, 8, 3, 4)            \
  X(8, 5, 3, 4) X(4, 8, 4, 4) X(4, 2, 4, 4) X(1, 2, 4, 4) X(2, 2, 4, 4) X(1, 4, 4, 4)            \
  X(2, 2, 5, 4) X(4, 8, 3, 8) X(4, 5, 3, 8) X(2, 3, 4, 4) X(2, 1, 5, 4) X(1, 3, 4, 4)            \
  X(1, 1, 5, 4) X(1, 1, 8, 4) X(1, 2, 8, 4) X(1, 3, 8, 4) X(1, 3, 5, 8) X(1, 4, 8, 4)            \
  X(2, 4, 4, 8) X(2, 8, 4, 8) X(4, 4, 3, 8)

#define W4A8_TILE_CFG(wm, wn, ns, nw)                                                             \
  TileCfg{wm, wn, TileShape<wm, wn, nw>::BM, TileShape<wm, wn, nw>::BN, nw,                        \
          ns * TileShape<wm, wn, nw>::STAGE + ring_slots(ns) * TileShape<wm, wn, nw>::S_SLOT +   \
              1024 +                                                                             \
              TileShape<wm, wn, nw>::TSCALE,                                                     \
          ns},
constexpr TileCfg kTile[] = {W4A8_TILE_TABLE(W4A8_TILE_CFG)};
#undef W4A8_TILE_CFG
constexpr int kTileCount = sizeof(kTile) / sizeof(kTile[0]);

}  // namespace

int tile_variant_count() { return kTileCount; }
bool tile_splits(int v) { return kTile[v].nw == 4 && kTile[v].wm <= 2; }
size_t tile_split_bytes(int M, int N, int splits) { return (size_t)splits * M * N * sizeof(float); }
TileCfg tile_variant(int v) { return kTile[v]; }

bool tile_fits(int M, int N, int K) {
  // 32-bit buffer offsets: the activations (tiled: whole 16-token blocks) and one tile's weight
  // stripe
  return (long)ceil_div(M, 16) * 16 * K < (1L << 31) &&
         (long)16 * padded_k(K) / 2 * 16 < (1L << 31) && (long)N < (1L << 24);
}

hipError_t launch_tile_body(const GemmArgs& g, int variant, bool a_tiled, hipStream_t stream,
                            float* P, int splits, int KTp, int KTe, int KG, int NTILES,
                            int grid_m, int grid_n, int vec_out, dim3 grid, dim3 block);

// Adds the `splits` fp32 partial sums P[s][M][N] of a split-K tile launch in split order, scales
// by the per-token scale and stores bf16: one thread per 4 consecutive columns of one token.
__global__ __launch_bounds__(256) void split_reduce(const float* __restrict__ P,
                                                    const float* __restrict__ As,
                                                    uint16_t* __restrict__ C, int M, int N,
                                                    int ldc, int splits, int vec_out) {
  const int n4 = N >> 2;
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)M * n4) return;
  const int m = (int)(idx / n4), n = 4 * (int)(idx - (long)m * n4);
  const size_t plane = (size_t)M * N, at = (size_t)m * N + n;
  v4f v = *reinterpret_cast<const v4f*>(P + at);
  for (int s = 1; s < splits; ++s) v += *reinterpret_cast<const v4f*>(P + s * plane + at);
  store_out4(C, ldc, m, n, N, v, As[m], vec_out != 0);
}

hipError_t launch_split_reduce(const float* partial, const GemmArgs& g, int splits,
                               hipStream_t stream) {
  const long threads = (long)g.M * (g.N / 4);
  hipLaunchKernelGGL(split_reduce, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream,
                     partial, g.a_scale, g.c, g.M, g.N, g.ldc, splits,
                     (g.ldc % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0);
  return hipGetLastError();
}

hipError_t launch_tile(const GemmArgs& g, int variant, bool a_tiled, hipStream_t stream,
                       float* partial, int splits) {
  const TileCfg c = kTile[variant];
  const int KTp = padded_k(g.K) / kKTile, KTe = ceil_div(g.K, kKTile), KG = KTp / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int grid_m = ceil_div(g.M, c.bm), grid_n = ceil_div(g.N, c.bn);
  // 2: 16-byte row stores possible (staged epilogue), 1: 8-byte stores, 0: scalar stores
  const int vec_out = (g.N % 8 == 0 && g.ldc % 8 == 0 && ((uintptr_t)g.c % 16) == 0)  ? 2
                      : (g.N % 4 == 0 && g.ldc % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1
                                                                                         : 0;
  float* const P = splits > 1 ? partial : nullptr;
  const dim3 grid(grid_m * grid_n, P ? splits : 1), block(c.nw * 64);
  if (P) {
    // the partial launch, then the reduction on the same stream
    const hipError_t e = launch_tile_body(g, variant, a_tiled, stream, P, splits, KTp, KTe, KG,
                                          NTILES, grid_m, grid_n, vec_out, grid, block);
    if (e != hipSuccess) return e;
    return launch_split_reduce(P, g, splits, stream);
  }
  return launch_tile_body(g, variant, a_tiled, stream, nullptr, 1, KTp, KTe, KG, NTILES, grid_m,
                          grid_n, vec_out, grid, block);
}

hipError_t launch_tile_body(const GemmArgs& g, int variant, bool a_tiled, hipStream_t stream,
                            float* P, int splits, int KTp, int KTe, int KG, int NTILES,
                            int grid_m, int grid_n, int vec_out, dim3 grid, dim3 block) {
  int idx = 0;
#define W4A8_TILE_GO(wm, wn, ns, nw, at)                                                         \
  {                                                                                              \
    if (P) {                                                                                     \
      if constexpr (nw == 4 && wm <= 2)                                                          \
        hipLaunchKernelGGL((gemm_tile_split<wm, wn, ns, nw, at>), grid, block, 0, stream, g.a,   \
                           g.a_scale, g.wq, g.sq, g.M, g.K, KTp, NTILES, grid_m, grid_n, g.N,   \
                           splits, P);                                                           \
      else                                                                                       \
        return hipErrorInvalidValue;                                                             \
    } else if constexpr (nw == 8 || wm > 2) {                                                    \
      hipLaunchKernelGGL((gemm_tile<wm, wn, ns, nw, at>), grid, block, 0, stream, g.a,           \
                         g.a_scale, g.wq, g.sq, g.c, g.M, g.N, g.K, KTp, KTe, KG, NTILES, grid_m, \
                         grid_n, g.ldc, vec_out);                                                \
    } else {                                                                                     \
      hipLaunchKernelGGL((gemm_tile_pre<wm, wn, ns, nw, at>), grid, block, 0, stream, g.a,       \
                         g.a_scale, g.wq, g.sq, g.M, g.K, KTp, NTILES, grid_m, grid_n, g.N,     \
                         g.ldc, vec_out, g.c);                                                   \
    }                                                                                            \
    return hipGetLastError();                                                                    \
  }
#define W4A8_TILE_LAUNCH(wm, wn, ns, nw)                                                       \
  if (idx++ == variant) {                                                                        \
    if (a_tiled) W4A8_TILE_GO(wm, wn, ns, nw, true)                                              \
    W4A8_TILE_GO(wm, wn, ns, nw, false)                                                          \
  }
  W4A8_TILE_TABLE(W4A8_TILE_LAUNCH)
#undef W4A8_TILE_LAUNCH
#undef W4A8_TILE_GO
  return hipErrorInvalidValue;
}

}  // namespace w4a8
