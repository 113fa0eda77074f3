// Decode-band W4A8 GEMM (17..64 tokens) on gfx950: weight waves stream the granules through
// registers while activation waves feed them the token fragments through LDS.
//
// Counterpart of the reference's decode kernel above 16 tokens (sly/mxfp4/radiance_mxfp4_fp8.hip:
// 981-1228, its M <= DECODE_MAX_M band) for MI355X. At these M a workgroup that covers all of K
// for its n-tiles needs the whole M x K activation panel (320 KiB at M = 64, K = 5120) besides its
// share of the weights (about 200 KiB), and on MI355X the two streams add up per CU: measured with
// plain reads, 200 KiB of HBM and 320 KiB of L2-resident data per CU take 11.4 us together against
// 8.7 and 4.1 us apart, at the best split of the two over the waves. A wave's loads retire in
// order, so a wave that mixed the two would wait on the slow weight loads for every activation
// fragment; here they are on different waves:
//  * Weight waves (4, one per SIMD): wave w owns the k-tiles [KT w / 4, KT (w + 1) / 4) of the
//    workgroup's n-tiles (at most NT) and keeps R k-tiles of granules in flight in registers
//    (non-temporal 128-bit loads), its scale dwords loaded once ahead of them. Per k-tile it waits
//    for its activation slot, reads the MF 16-token fragments from LDS, releases the slot and runs
//    NT * MF scaled MFMAs, NT * MF independent accumulator chains.
//  * Activation waves (4): activation wave a serves weight wave a, copying each of its k-tiles'
//    16 MF token rows (128 bytes each) into a ring of D slots by LDS-DMA (8 tokens x 128 bytes per
//    64-lane load, rows past M read as zero), L k-tiles in flight, and posting each slot when its
//    copies have landed. Chunk c of token t lands at chunk position c ^ swz(t % 16) of the row, so
//    the fragment reads (16 tokens, one 16-byte chunk each) are free of bank conflicts.
//  * The slots are handed over through LDS counters (ready / consumed per weight wave, relaxed
//    atomics after the wave's own waits, no fence), every wait bounded: a wait that runs out marks
//    the workgroup failed and its outputs NaN, never plausible numbers. No wave waits for a wave
//    that is itself waiting on it (L <= D), and the workgroup's waves are all resident.
//  * The 4 partial sums of each output meet in LDS and are added in wave order (deterministic),
//    scaled and stored as bf16; or, split over K (grid rows), stored unscaled in fp32 for
//    split_reduce. Nothing crosses workgroups.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

constexpr int kBandWW = 4;             // weight waves (and as many activation waves)
constexpr int kBandSpin = 1 << 20;     // s_sleep(1) rounds a wait takes at most (~0.05 s)

// A workgroup barrier after this wave's LDS operations, with no memory fence: loads in flight
// (the activation waves' first slots, at the start) stay in flight
__device__ __forceinline__ void band_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

template <int N>
__device__ __forceinline__ void band_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// LDS chunk position of 16-byte chunk c of token t (t % 16): distinct for the 8 even and the 8
// odd tokens of a fragment, and for any 8 consecutive tokens
__device__ __forceinline__ int band_swz(int t) { return ((t >> 1) & 7) ^ ((t & 1) << 2); }

// The counters are read and written by inline LDS instructions: the compiler cannot tell a
// counter from the LDS-DMA destinations, and before every LDS access it can see it waits for
// every DMA of the wave in flight (vmcnt(0)), which would leave an activation wave one k-tile in
// flight. The asm carries its own wait; the DMAs are ordered by the explicit vmcnt waits.
typedef __attribute__((address_space(3))) int band_lds_int;
__device__ __forceinline__ uint32_t band_addr(const int* counter) {
  return (uint32_t)(uintptr_t)(const band_lds_int*)counter;
}

// the counter reaches `target` (wave-uniform, bounded); false when the wait ran out
__device__ __forceinline__ bool band_wait(const int* counter, int target) {
  const uint32_t a = band_addr(counter);
  for (int it = 0; it < kBandSpin; ++it) {
    int n;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(n) : "v"(a) : "memory");
    if (__builtin_amdgcn_readfirstlane(n) >= target) return true;
    __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// publish `v` after this wave's LDS reads have completed (LDS serves a wave in order); every
// lane writes the same value, so no lane mask sits next to the MFMAs
__device__ __forceinline__ void band_post(int* counter, int v) {
  __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
  asm volatile("ds_write_b32 %0, %1" ::"v"(band_addr(counter)), "v"(v) : "memory");
}

// MF: 16-token fragments (M <= 16 MF); NT: n-tiles per workgroup at most; SG: scale dwords per
// n-tile a weight wave holds (its k-range spans at most SG k-groups); R: k-tiles of granules in
// flight per weight wave; D activation slots per weight wave, L of them in flight per activation
// wave (L <= D). mks = M | (KS << 8): KS k-tiles per grid row (0: no split). The body is a device
// function under the kernel, as the tile kernel's is: with the activation waves' 16-byte LDS-DMA
// loads in the __global__ function itself, the host pass emitted no launch stub for it.
template <int MF, int NT, int SG, int R, int D, int L>
__device__ __forceinline__ void band_body(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, void* __restrict__ out, int mks, int K, int N, int S) {
  static_assert(MF >= 1 && MF <= 4 && NT >= 1 && SG >= 2 && R >= 1, "band variant");
  static_assert(L >= 1 && L <= D && (L - 1) * 2 * MF < 64, "an activation wave may not run past "
                "the slots it owns, and its loads in flight fit the load counter");
  constexpr int WW = kBandWW, SLOT = MF * 2048;
  constexpr int RING = WW * D * SLOT, PART = WW * NT * MF * 1024;
  constexpr int BODY = RING > PART ? RING : PART;
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  int* const ctr = reinterpret_cast<int*>(lds + BODY);   // ready[WW], consumed[WW], failed
  float* const tsc = reinterpret_cast<float*>(lds + BODY + 64);   // the 64 token scales
  const int M = mks & 0xFF, KS = mks >> 8;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // K, N > 0: unsigned shifts, no sign fix-ups in the scalar prologue (the CU's 8 waves share
  // one scalar unit, and it runs before their first requests)
  const int KT = (int)((unsigned)K / kKTile);                        // activation k-tiles
  const int KTW = (int)(((unsigned)K + kKAlign - 1) / kKAlign) * 4;  // weight k-tiles
  const int NTILES = (int)(((unsigned)N + kNTile - 1) / kNTile);
  const int b = blockIdx.x;
  // S n-tiles per workgroup (from the host: no division by the grid size), the last what is left
  const int ntb0 = b * S, nth = min(S, NTILES - ntb0);
  const int ks0 = KS ? (int)blockIdx.y * KS : 0, ks1 = KS ? min(ks0 + KS, KT) : KT;
  const int wv = wave & (WW - 1);
  const int kb = ks0 + (int)((unsigned)((ks1 - ks0) * wv) / WW);
  const int ke = ks0 + (int)((unsigned)((ks1 - ks0) * (wv + 1)) / WW);
  const int nk = ke - kb;
  if (tid <= 2 * WW) ctr[tid] = 0;
  band_barrier();

  bool ok = true;
  v4f acc[NT][MF];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int f = 0; f < MF; ++f) acc[t][f] = v4f{0.f, 0.f, 0.f, 0.f};

  if (wave < WW) {
    // ---- weight wave. Its loads go out after the activation waves' first ones (the barrier):
    //      a CU's loads come back in order, and the first activation slots gate every MFMA ----
    band_barrier();
    __amdgpu_buffer_rsrc_t w_src[NT];
    uint32_t sv[NT][SG];
    const int g0 = kb >> 2;
    // the workgroup's first stripe and scale rows (one 64-bit product), then 32-bit offsets (the
    // host keeps NT stripes below 2^31 bytes)
    const uint8_t* const wbase = Wq + (size_t)ntb0 * KTW * kGranuleBytes;
    const uint8_t* const sbase = reinterpret_cast<const uint8_t*>(Sq) + (size_t)ntb0 * KTW * 64;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool have = t < nth;
      w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(wbase + (uint32_t)(t * KTW * kGranuleBytes)), 0,
          have ? ke * kGranuleBytes : 0, kBufferWord3);
      const auto s_src = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(sbase + (uint32_t)(t * KTW * 64)), 0,
          have ? ((ke + 3) >> 2) * 256 : 0, kBufferWord3);
#pragma unroll
      for (int q = 0; q < SG; ++q)
        sv[t][q] = __builtin_amdgcn_raw_buffer_load_b32(s_src, ((g0 + q) * 64 + lane) * 4, 0, 0);
    }
    // R k-tiles of granules in flight; granules past the k-range or the workgroup's n-tiles read
    // as zero without a memory access
    v4i wr[R][NT];
#pragma unroll
    for (int jj = 0; jj < R; ++jj)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wr[jj][t] = __builtin_amdgcn_raw_buffer_load_b128(
            w_src[t], (kb + jj) * kGranuleBytes + lane * 16, 0, kBufferNT);
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* const ring = lds + wave * D * SLOT;
    const int ts = lane & 15, c = lane >> 4;
    const int lo_pos = (c ^ band_swz(ts)) * 16, hi_pos = ((c + 4) ^ band_swz(ts)) * 16;
    const int rounds = (nk + R - 1) / R;
    for (int r = 0; r < rounds; ++r) {
#pragma unroll
      for (int jj = 0; jj < R; ++jj) {
        // Every round runs all R stages, the loads and MFMAs of each unconditionally (past the
        // k-range the granules and fragments are zero and add nothing), so on every path the
        // same loads are in flight and the compiler's in-order load count stays exact: a stage's
        // wait then leaves the R - 1 later stages in flight
        const int j = r * R + jj;
        v8i xf[MF];
        if (j < nk) {                            // wave-uniform
          ok &= band_wait(&ctr[wave], j + 1);
          const uint8_t* const slot = ring + (j % D) * SLOT;
#pragma unroll
          for (int f = 0; f < MF; ++f) {
            const uint8_t* const row = slot + (16 * f + ts) * 128;
            const v4i lo = *reinterpret_cast<const v4i*>(row + lo_pos);
            const v4i hi = *reinterpret_cast<const v4i*>(row + hi_pos);
            xf[f] = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          }
          band_post(&ctr[WW + wave], j + 1);     // the slot's reads are done: it may refill
        } else {
#pragma unroll
          for (int f = 0; f < MF; ++f) xf[f] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
        }
        const int kt = kb + j, sh = 8 * (kt & 3), q = (kt >> 2) - g0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          uint32_t sc = sv[t][0];
#pragma unroll
          for (int qq = 1; qq < SG; ++qq) sc = q == qq ? sv[t][qq] : sc;
          sc >>= sh;
#pragma unroll
          for (int f = 0; f < MF; ++f) acc[t][f] = mfma_w4a8(wr[jj][t], xf[f], acc[t][f], sc);
          // the n-tile's granule R k-tiles on, as soon as its MFMAs are issued
          wr[jj][t] = __builtin_amdgcn_raw_buffer_load_b128(
              w_src[t], (kb + j + R) * kGranuleBytes + lane * 16, 0, kBufferNT);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  } else {
    // ---- activation wave: the served weight wave's k-tiles into its D slots, L in flight; rows
    //      past M read as zero ----
    const int a = wave - WW;
    const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
    uint8_t* const ring = lds + a * D * SLOT;
    const int tl = lane >> 3, p = lane & 7;
    int off[2 * MF];
#pragma unroll
    for (int i = 0; i < 2 * MF; ++i) {
      const int t = 8 * i + tl;
      off[i] = t * K + 16 * (p ^ band_swz(t & 15));
    }
    auto issue = [&](int j) {
      const int kx = (kb + j) * kKTile;
      uint8_t* const slot = ring + (j % D) * SLOT;
#pragma unroll
      for (int i = 0; i < 2 * MF; ++i)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(a_src, (lds_ptr_t)(slot + i * 1024), 16,
                                                 off[i] + kx, 0, 0, 0);
    };
#pragma unroll
    for (int j = 0; j < L; ++j)
      if (j < nk) issue(j);                      // ahead of every weight load of the CU
    band_barrier();
    for (int j = L; j < nk; ++j) {
      band_wait_vm<(L - 1) * 2 * MF>();          // k-tiles 0 .. j - L have landed
      band_post(&ctr[a], j - L + 1);
      if (j >= D) ok &= band_wait(&ctr[WW + a], j - D + 1);   // slot j % D is free
      issue(j);
    }
    band_wait_vm<0>();
    band_post(&ctr[a], nk);
    if (a == 0 && lane < M) tsc[lane] = As[lane];   // the epilogue's token scales
  }
  if (!ok) __hip_atomic_store(&ctr[2 * WW], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);

  // ---- the weight waves' partial sums meet in LDS (over the ring, now idle), added in wave
  //      order; every lane writes (no branch around the MFMA results) ----
  __syncthreads();
  v4f* const part = reinterpret_cast<v4f*>(lds);
  if (wave < WW) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int f = 0; f < MF; ++f) part[((wave * NT + t) * MF + f) * 64 + lane] = acc[t][f];
  }
  __syncthreads();
  const bool failed = ctr[2 * WW] != 0;
  for (int sl = tid; sl < nth * MF * 64; sl += 2 * WW * 64) {
    const int t = sl / (MF * 64), f = (sl >> 6) % MF, l = sl & 63;
    const int m = 16 * f + (l & 15), n = (ntb0 + t) * kNTile + 4 * (l >> 4);
    if (m >= M) continue;
    v4f pw[WW];
#pragma unroll
    for (int w = 0; w < WW; ++w) pw[w] = part[((w * NT + t) * MF + f) * 64 + l];
    v4f v = pw[0];
#pragma unroll
    for (int w = 1; w < WW; ++w) v += pw[w];
    if (failed) v = v4f{__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                        __builtin_nanf("")};
    if (KS) {
      // unscaled fp32 sums, P[s][M][N] (the host requires N % 16 == 0)
      float* const P = reinterpret_cast<float*>(out) + (size_t)blockIdx.y * M * N;
      *reinterpret_cast<v4f*>(P + (size_t)m * N + n) = v;
    } else {
      const float sc = tsc[m];
      uint16_t* const row = reinterpret_cast<uint16_t*>(out) + (size_t)m * N;
      if (N % 4 == 0 && ((uintptr_t)out & 7) == 0 && n + 3 < N) {
        *reinterpret_cast<uint2*>(row + n) =
            make_uint2(bf16x2_rne(v[0] * sc, v[1] * sc), bf16x2_rne(v[2] * sc, v[3] * sc));
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (n + i < N) row[n + i] = (uint16_t)f32_to_bf16(v[i] * sc);
      }
    }
  }
}

// The 14 argument dwords are the preloaded ones.
template <int MF, int NT, int SG, int R, int D, int L>
__global__ __launch_bounds__(2 * kBandWW * 64) void gemm_band(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, void* __restrict__ out, int mks, int K, int N, int S) {
  band_body<MF, NT, SG, R, D, L>(A, As, Wq, Sq, out, mks, K, N, S);
}

// (MF, NT, SG, R, D, L): MF 16-token fragments, at most NT n-tiles per workgroup, SG scale dwords
// per n-tile (a weight wave's k-range spans at most 4 (SG - 1) + 1 k-tiles), R granule k-tiles in
// flight per weight wave, D activation slots per weight wave (96-128 KiB of LDS in all), L of them
// in flight per activation wave. Registers per weight wave: 16 NT MF accumulators, 4 R NT granule
// registers, NT SG scale dwords, 8 MF fragment registers.
#define W4A8_BAND_TABLE(X)                                                                        \
  X(2, 5, 4, 3, 8, 6) X(3, 5, 4, 3, 5, 4) X(4, 5, 4, 3, 4, 3)                                     \
  X(2, 3, 4, 3, 8, 6) X(3, 3, 4, 3, 5, 4) X(4, 3, 4, 3, 4, 3)                                     \
  X(2, 2, 6, 4, 8, 6) X(3, 2, 6, 4, 5, 4) X(4, 2, 6, 4, 4, 3)                                     \
  X(2, 4, 3, 3, 8, 6) X(3, 4, 3, 3, 5, 4) X(4, 4, 3, 3, 4, 3)

#define W4A8_BAND_CFG(mf, nt, sg, r, d, l) BandCfg{mf, nt, sg, r, d, l},
constexpr BandCfg kBand[] = {W4A8_BAND_TABLE(W4A8_BAND_CFG)};
#undef W4A8_BAND_CFG
constexpr int kBandCount = sizeof(kBand) / sizeof(kBand[0]);

size_t band_lds_bytes(const BandCfg& c) {
  const size_t ring = (size_t)kBandWW * c.d * c.mf * 2048;
  const size_t part = (size_t)kBandWW * c.nt * c.mf * 1024;
  return (ring > part ? ring : part) + 64 + 64 * sizeof(float);   // + counters, token scales
}

}  // namespace

int band_variant_count() { return kBandCount; }
BandCfg band_variant(int v) { return kBand[v]; }

// Balanced n-tile shares as the streaming kernel's (at most one workgroup per CU and split).
int band_grid(int N, int cus, int splits) {
  const int ntiles = padded_n(N) / kNTile;
  const int per_row = splits > 0 ? cus / splits : cus;
  const int g = ntiles < per_row ? ntiles : (per_row > 0 ? per_row : 1);
  return ceil_div(ntiles, ceil_div(ntiles, g));
}

bool band_fits(int variant, int M, int N, int K, int cus, int splits, size_t lds_limit) {
  if (variant < 0 || variant >= kBandCount) return false;
  const BandCfg c = kBand[variant];
  if (M < 1 || M > 16 * c.mf || K % kKTile || splits < 1) return false;
  const int KT = K / kKTile;
  if (splits > KT / kBandWW) return false;              // every weight wave owns a k-tile
  if (splits > 1 && N % kNTile) return false;           // the partial layout split_reduce reads
  const int ntiles = padded_n(N) / kNTile;
  if (ceil_div(ntiles, band_grid(N, cus, splits)) > c.nt) return false;
  // a weight wave's k-range: at most ceil(KS / 4) k-tiles, spanning at most SG k-groups
  const int ks = ceil_div(KT, splits), kw = ceil_div(ks, kBandWW);
  if ((kw + 2) / 4 + 1 > c.sg) return false;
  const bool small = (long)64 * K < (1L << 31) && (long)c.nt * padded_k(K) / kKTile *
                     kGranuleBytes < (1L << 31) && (long)padded_n(N) < (1L << 24) && ks < (1 << 23);
  return small && band_lds_bytes(c) <= lds_limit;
}

size_t band_split_bytes(int M, int N, int splits) {
  return splits > 1 ? (size_t)splits * M * N * sizeof(float) : 0;
}

hipError_t launch_band(const GemmArgs& g, int variant, int cus, int splits, float* partial,
                       hipStream_t stream) {
  const BandCfg c = kBand[variant];
  const int KT = g.K / kKTile;
  const int ks = splits > 1 ? ceil_div(KT, splits) : 0;
  const int rows = splits > 1 ? ceil_div(KT, ks) : 1;
  const int G = band_grid(g.N, cus, splits > 1 ? splits : 1);
  const int share = ceil_div(padded_n(g.N) / kNTile, G);   // n-tiles per workgroup
  const size_t lds = band_lds_bytes(c);
  void* const out = splits > 1 ? (void*)partial : (void*)g.c;
  const int mks = g.M | (ks << 8);
  int idx = 0;
#define W4A8_BAND_LAUNCH(mf, nt, sg, r, d, l)                                                    \
  if (idx++ == variant) {                                                                        \
    if (lds > 64 * 1024) {                                                                       \
      const hipError_t e = hipFuncSetAttribute((const void*)gemm_band<mf, nt, sg, r, d, l>,      \
                                               hipFuncAttributeMaxDynamicSharedMemorySize,       \
                                               (int)lds);                                        \
      if (e != hipSuccess) return e;                                                             \
    }                                                                                            \
    hipLaunchKernelGGL((gemm_band<mf, nt, sg, r, d, l>), dim3(G, rows), dim3(2 * kBandWW * 64),  \
                       lds, stream, g.a, g.a_scale, g.wq, g.sq, out, mks, g.K, g.N, share);     \
    const hipError_t e = hipGetLastError();                                                      \
    if (e != hipSuccess || splits <= 1) return e;                                                \
    return launch_split_reduce(partial, g, rows, stream);                                        \
  }
  W4A8_BAND_TABLE(W4A8_BAND_LAUNCH)
#undef W4A8_BAND_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
