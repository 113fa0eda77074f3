// Pipelined streaming W4A8 GEMM for the decode / speculative-verify band above 16 tokens
// (M <= 16 * MF, MF = 1..4 sixteen-token fragments) on gfx950.
//
// Counterpart of the reference's decode kernel (sly/mxfp4/radiance_mxfp4_fp8.hip:981-1228), which
// serves M up to DECODE_MAX_M with one weight pass (:1497-1527). At these M the GEMM is still a
// weight stream (47 MB for the 17408 x 5120 gate/up against 0.3 MB of activations at M = 64), but
// the activations no longer fit in registers next to a whole k-range of weights, as they do in the
// M <= 16 streaming kernel: every workgroup covers all of K for its n-tiles and so needs the whole
// M x K activation (320 KiB at M = 64, K = 5120), more than a CU's register file holds beside the
// weights. So each wave runs a software pipeline over its k-range instead of issuing it at once:
//  * The grid is at most one workgroup per CU, each owning the same number of n-tiles (at most NT)
//    and all of K; wave w owns the contiguous k-tiles [KT w / W, KT (w + 1) / W).
//  * A stage is one k-tile: the NT weight granules (one 128-bit non-temporal load each) and the
//    MF activation fragments (two 128-bit loads each, straight from L2 into registers). A wave may
//    have at most 63 loads in flight (its load counter), so the e8m0 scale dwords stay out of the
//    stages: each wave moves the scale rows of its k-range (one 256-byte row per n-tile and
//    k-group) into its own LDS region once, ahead of the first stage, and reads each stage's
//    dwords from there. D stages are in flight per wave: the loop consumes stage
//    j (MF * NT scaled MFMAs, NT * MF independent accumulator chains) and refills its registers
//    with the k-tile D ahead, so the weight stream never drains while the wave computes. The
//    loop is unrolled by D so every stage lives in fixed registers; the compiler counts the
//    outstanding loads exactly (loads return in order), so a stage's wait leaves the D - 1 later
//    stages in flight.
//  * Every global load goes through a buffer resource. Weight loads past the wave's k-range or
//    the workgroup's n-tiles, activation rows past M and runs past K return zero without a memory
//    access. The last round is padded with stages past the range, whose zero weights add nothing,
//    so the loop has no branches around loads.
//  * The W partial sums of each output meet in LDS, one 16-token fragment at a time, and are
//    added in wave order (deterministic), scaled by the per-token fp32 scale and stored as bf16.
//    Nothing crosses workgroups.
//  * AT: the activations arrive fragment-tiled (16-token blocks, k-tile after k-tile, each
//    fragment half one contiguous KiB in lane order), so every activation load is a contiguous
//    1 KiB instead of 16 token rows x 64 bytes; same operands, same bits as the row-major form.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

constexpr int kOutOfRange = 0x7FFFFFF0;   // an offset past every buffer resource here

typedef __attribute__((address_space(3))) void* lds_ptr_t;

template <int MF, int NT, int D, int W, bool AT>
__global__ __launch_bounds__(W * 64) void gemm_ring(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int N, int K, int KT,
    int KG, int NTILES, int SG, int vec_out) {
  static_assert(MF >= 1 && MF <= 4 && NT >= 1 && D >= 1 && W >= 1 && W <= 16, "ring variant");
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = gridDim.x, b = blockIdx.x;
  const int ntb0 = b * NTILES / G, nth = (b + 1) * NTILES / G - ntb0;
  const int kb = KT * wave / W, ke = KT * (wave + 1) / W;     // this wave's k-tiles
  const int rounds = ceil_div(ke - kb, D);

  // ---- buffer resources: one per n-tile for weights and scales, bounded by the wave's k-range
  //      (weights) and the workgroup's n-tiles; one for the activations, bounded by M rows ----
  __amdgpu_buffer_rsrc_t w_src[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
    w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(Wq + (size_t)(ntb0 + t) * KT * kGranuleBytes), 0,
        t < nth ? ke * kGranuleBytes : 0, kBufferWord3);

  // ---- this wave's scale rows (k-groups g0 .. g0 + SG - 1 of each n-tile) into its LDS region,
  //      one 256-byte row per load, before any stage: the first stage's wait covers them ----
  const int g0 = kb >> 2, glast = (ke - 1) >> 2;
  uint8_t* const srows = lds + W * NT * 64 * sizeof(v4f) + wave * NT * SG * 256;
  {
    const auto s_all = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(Sq + (size_t)ntb0 * KG * 64), 0, nth * KG * 256, kBufferWord3);
#pragma unroll
    for (int t = 0; t < NT; ++t)
      for (int r = 0; r < SG; ++r)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            s_all, (lds_ptr_t)(srows + (t * SG + r) * 256), 4,
            g0 + r <= glast ? (t * KG + g0 + r) * 256 + lane * 4 : kOutOfRange, 0, 0, 0);
  }

  // tiled: whole 16-token blocks, the last one's padding tokens zero (K % 128 == 0)
  const int a_bytes = AT ? (M + 15) / 16 * 16 * K : M * K;
  const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, a_bytes, kBufferWord3);
  const int m = lane & 15, g = lane >> 4;
  // activation offset of fragment f's lane run at k-tile 0, and the k (per lane) from which the
  // lane's low / high run would leave its row: such runs are pointed past the buffer (K % 32 == 0,
  // so a 16-byte run is wholly inside a row or wholly past it). Rows past M read as zero.
  int a_row[MF];
#pragma unroll
  for (int f = 0; f < MF; ++f) a_row[f] = (16 * f + m) * K + 16 * g;
  const int lo_end = K - 16 * g, hi_end = K - 64 - 16 * g;

  v4i wv[D][NT];
  v4i xlo[D][MF], xhi[D][MF];

  // Loads of k-tile kt into stage j's registers. Past the wave's range the weights read as zero
  // (the resource ends there); the activation reads of such a stage may see another wave's
  // k-tiles of the same rows, which only meet zero weights: they change nothing, except that a
  // NaN there would turn the product NaN, and a NaN activation of the same row already makes
  // that output NaN in the exact result. Past K the activation runs read as zero.
  auto issue = [&](int j, int kt) {
    const int kx = kt * kKTile;
#pragma unroll
    for (int t = 0; t < NT; ++t)
      wv[j][t] = __builtin_amdgcn_raw_buffer_load_b128(w_src[t], kt * kGranuleBytes + lane * 16,
                                                       0, kBufferNT);
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      if constexpr (AT) {
        // block f, k-tile kt of the layout's K / 128 (not the weights' padded KT): halves at +0 /
        // +1 KiB; a k-tile past K would be the next block's tokens, so it reads as zero; blocks
        // past the last end the buffer and read as zero
        const int kta = K >> 7;
        const int base = kt < kta ? (f * kta + kt) * 2048 + lane * 16 : kOutOfRange;
        xlo[j][f] = __builtin_amdgcn_raw_buffer_load_b128(a_src, base, 0, 0);
        xhi[j][f] = __builtin_amdgcn_raw_buffer_load_b128(
            a_src, kt < kta ? base + 1024 : kOutOfRange, 0, 0);
      } else {
        const int lo = kx < lo_end ? a_row[f] + kx : kOutOfRange;
        const int hi = kx < hi_end ? a_row[f] + kx + 64 : kOutOfRange;
        xlo[j][f] = __builtin_amdgcn_raw_buffer_load_b128(a_src, lo, 0, 0);
        xhi[j][f] = __builtin_amdgcn_raw_buffer_load_b128(a_src, hi, 0, 0);
      }
    }
  };

  v4f acc[NT][MF];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[t][f] = v4f{0.f, 0.f, 0.f, 0.f};

  // stage j holds k-tile kt: MF * NT scaled MFMAs; the scale byte of k-tile kt from its dword in
  // the wave's LDS rows (a stage past the range reads the last k-group's dwords: same columns)
  auto consume = [&](int j, int kt) {
    const int sh = 8 * (kt & 3);
    const int r = min(kt >> 2, glast) - g0;
    uint32_t sc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t)
      sc[t] = *reinterpret_cast<const uint32_t*>(srows + (t * SG + r) * 256 + lane * 4) >> sh;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
      const v8i xf = {xlo[j][f][0], xlo[j][f][1], xlo[j][f][2], xlo[j][f][3],
                      xhi[j][f][0], xhi[j][f][1], xhi[j][f][2], xhi[j][f][3]};
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t][f] = mfma_w4a8(wv[j][t], xf, acc[t][f], sc[t]);
    }
  };

#pragma unroll
  for (int j = 0; j < D; ++j) issue(j, kb + j);
  __builtin_amdgcn_sched_barrier(0);
  for (int r = 0; r + 1 < rounds; ++r) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int kt = kb + r * D + j;
      consume(j, kt);
      __builtin_amdgcn_sched_barrier(0);
      issue(j, kt + D);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int j = 0; j < D; ++j) consume(j, kb + (rounds - 1) * D + j);

  // ---- cross-wave reduction in LDS, one fragment at a time, added in wave order ----
  v4f* red = reinterpret_cast<v4f*>(lds);
  const bool vec = vec_out != 0;
  const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
#pragma unroll
  for (int f = 0; f < MF; ++f) {
    if (f) __syncthreads();                       // the previous fragment's reads are done
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t][f];
    __syncthreads();
    const int mo = 16 * f + m;
    const float tok = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(as_src, mo * 4, 0, 0));
    for (int slot = tid; slot < nth * 64; slot += W * 64) {
      const int t = slot >> 6;                    // slot lane == this thread's lane
      v4f v = red[t * 64 + lane];
#pragma unroll 4
      for (int w = 1; w < W; ++w) v += red[(w * NT + t) * 64 + lane];
      const int n = (ntb0 + t) * kNTile + 4 * (lane >> 4);
      if (mo < M) store_out4(C, N, mo, n, N, v, tok, vec);
    }
  }
}

// (MF, NT, D, W): MF 16-token fragments, at most NT n-tiles per workgroup, D stages in flight per
// wave, W waves. Per wave: D * (NT + 2 MF) loads in flight (the counter holds 63) and about
// D * (4 NT + 8 MF) + 4 NT MF registers.
#define W4A8_RING_TABLE(X)                                                                        \
  X(1, 5, 8, 4) X(1, 5, 4, 8)                                                                     \
  X(2, 5, 7, 4) X(2, 5, 4, 8) X(2, 3, 7, 4)                                                       \
  X(3, 5, 5, 4) X(3, 5, 3, 8) X(3, 3, 5, 4)                                                       \
  X(4, 5, 4, 4) X(4, 5, 2, 8) X(4, 3, 4, 4) X(4, 3, 3, 8)

#define W4A8_RING_CFG(mf, nt, d, w) RingCfg{mf, nt, d, w},
constexpr RingCfg kRing[] = {W4A8_RING_TABLE(W4A8_RING_CFG)};
#undef W4A8_RING_CFG
constexpr int kRingCount = sizeof(kRing) / sizeof(kRing[0]);

}  // namespace

int ring_variant_count() { return kRingCount; }
RingCfg ring_variant(int v) { return kRing[v]; }

// The fewest workgroups that keep the smallest share of n-tiles per workgroup the variant allows
// (at most NT), at most one per CU.
int ring_grid(int variant, int N, int cus) {
  const int ntiles = padded_n(N) / kNTile;
  const int per = ceil_div(ntiles, ntiles < cus ? ntiles : cus);
  return per > kRing[variant].nt ? 0 : ceil_div(ntiles, per);
}

// k-groups a wave's k-range can touch: its k-tiles span at most ceil(KT / W) + 3 k-tiles
int ring_scale_groups(int variant, int K) {
  const int KT = padded_k(K) / kKTile;
  return ceil_div(ceil_div(KT, kRing[variant].waves) + 3, kKGroup);
}

size_t ring_lds_bytes(int variant, int K) {
  const RingCfg c = kRing[variant];
  return (size_t)c.waves * c.nt * 64 * sizeof(v4f) +
         (size_t)c.waves * c.nt * ring_scale_groups(variant, K) * 256;
}

bool ring_fits(int variant, int M, int N, int K, int cus, size_t lds_limit) {
  const RingCfg c = kRing[variant];
  if (M < 1 || M > 16 * c.mf || K % 32 || ring_grid(variant, N, cus) == 0) return false;
  // every offset the kernel forms stays in 32 bits; each wave owns at least one k-tile
  const int KT = padded_k(K) / kKTile;
  const bool small = (long)64 * K < (1L << 31) && (long)KT * kGranuleBytes < (1L << 31) &&
                     (long)padded_n(N) < (1L << 24);
  return small && KT >= c.waves && ring_lds_bytes(variant, K) <= lds_limit;
}

hipError_t launch_ring(const GemmArgs& g, int variant, int cus, bool a_tiled, hipStream_t stream) {
  const int KT = padded_k(g.K) / kKTile, KG = KT / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(ring_grid(variant, g.N, cus)), block(kRing[variant].waves * 64);
  const size_t lds = ring_lds_bytes(variant, g.K);
  const int SG = ring_scale_groups(variant, g.K);
  int idx = 0;
#define W4A8_RING_GO(mf, nt, d, w, at)                                                           \
  {                                                                                              \
    if (lds > 64 * 1024) {                                                                       \
      const hipError_t e = hipFuncSetAttribute((const void*)gemm_ring<mf, nt, d, w, at>,         \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                               (int)lds);                                        \
      if (e != hipSuccess) return e;                                                             \
    }                                                                                            \
    hipLaunchKernelGGL((gemm_ring<mf, nt, d, w, at>), grid, block, lds, stream, g.a, g.a_scale,  \
                       g.wq, g.sq, g.c, g.M, g.N, g.K, KT, KG, NTILES, SG, vec_out);             \
    return hipGetLastError();                                                                    \
  }
#define W4A8_RING_LAUNCH(mf, nt, d, w)                                                           \
  if (idx++ == variant) {                                                                        \
    if (a_tiled) W4A8_RING_GO(mf, nt, d, w, true)                                               \
    W4A8_RING_GO(mf, nt, d, w, false)                                                            \
  }
  W4A8_RING_TABLE(W4A8_RING_LAUNCH)
#undef W4A8_RING_LAUNCH
#undef W4A8_RING_GO
  return hipErrorInvalidValue;
}

}  // namespace w4a8
