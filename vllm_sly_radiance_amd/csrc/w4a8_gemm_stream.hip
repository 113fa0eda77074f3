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
//    n-tiles S (the last one what is left): workgroup b owns [b S, min((b + 1) S, NTILES)), at
//    most NT of them. S comes from the host, so no wave divides by the grid size, and the buffer
//    resources of its n-tiles are one 64-bit base plus 32-bit offsets. The CU's waves share one
//    scalar unit, and this prologue runs before any wave's first request: cutting it from ~170
//    to ~85 scalar instructions per wave (the divisions, the per-n-tile 64-bit products, then
//    unsigned shifts and byte offsets) made every streaming shape 0.05-0.2 us faster (A/B on
//    MI355X, same bits).
//  * Wave w owns the k-groups [KG w / W, KG (w + 1) / W) (4 k-tiles each, so one scale dword per
//    n-tile) of every n-tile of the workgroup. It loads its activation fragments for those
//    k-tiles straight into registers (lane l: token l % 16, k 16 (l / 16).. and 64 + 16 (l / 16)..;
//    tokens past M read as zero; at M <= 8 one load per k-tile, see H8), the scale dwords and the
//    granules k-tile by k-tile (where the wave's range is one k-group, the scale dwords and the
//    first k-tile's granules go out before the activation loads), and multiplies each fragment
//    into all NT n-tiles as their granules land: no LDS staging, no barrier before the MFMAs, NT
//    independent accumulator chains.
//  * Every global load goes through a buffer resource; loads past the workgroup's n-tiles or the
//    wave's k-range return zero without a memory access, so the code has no branches around loads
//    and the compiler counts outstanding loads exactly.
//  * The W partial sums of each n-tile meet once in LDS and are added in wave order
//    (deterministic), scaled by the per-token fp32 scale and stored as bf16. Nothing crosses
//    workgroups.
//  * gemm_stream_fq (below) is the whole linear in one launch: bf16 activations, the per-token
//    quantizer run by extra waves of each workgroup while the weight waves stream.
#include "w4a8_fp8.h"
#include "w4a8_silu.h"

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

// NT: n-tiles per workgroup at most; KPW: k-tiles per wave at most (a multiple of 4); W: waves.
// The host requires K % 512 == 0 (whole k-groups), M <= 16 (M <= 8 with H8),
// 4 * ceil(KG / W) <= KPW. H8 (M <= 8): one load per k-tile brings both 16-byte runs of the 8
// live tokens (lanes 8..15 of each row of 16 load the second run of token r - 8, and a row
// rotation by 8 lanes hands it to lane r), half the activation loads; the MFMA columns of tokens
// 8..15 then hold other tokens' bytes, and those columns are never stored.
// The 14 argument dwords are exactly what the kernel arguments preloaded into SGPRs hold, so no
// wave reads the kernarg segment, not even for the epilogue (whose scalar load used to sit on the
// critical path after the last MFMA); the n-tile count and the store width follow from N and C.
template <int NT, int KPW, int W, bool H8>
__global__ __launch_bounds__(W * 64) void gemm_stream(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, int M, int K, int N, int S) {
  static_assert(KPW % 4 == 0 && NT >= 1 && W >= 1 && W <= 16, "stream variant");
  // K % 512 == 0; K, N > 0 (unsigned shifts: no sign fix-ups in the scalar prologue)
  const int KT = (int)((unsigned)K / kKTile), KG = (int)((unsigned)KT / kKGroup);
  const int NTILES = (int)(((unsigned)N + kNTile - 1) / kNTile);
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  const int tid = threadIdx.x, lane = tid & 63;
  // Wave-uniform work selection in scalar registers; 32-bit products only (the host bounds them).
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int ntb0 = b * S, nth = min(S, NTILES - ntb0);
  // the workgroup's first granule stripe and scale rows (one 64-bit product); an n-tile's stripe
  // is t KT KiB further, below 2^31 for the NT n-tiles of a workgroup (the host checks it)
  const uint8_t* const wbase = Wq + (size_t)ntb0 * KT * kGranuleBytes;
  const uint8_t* const sbase = reinterpret_cast<const uint8_t*>(Sq) + (size_t)ntb0 * KG * 256;
  // the epilogue: thread tid adds the partials of output slot tid (below); at M <= 8 a slot is one
  // of the 32 lanes of an n-tile that hold tokens 0..7
  constexpr int LIVE = H8 ? 32 : 64;
  const int om = H8 ? (tid & 7) : (tid & 15), og = (tid % LIVE) / (H8 ? 8 : 16);
  const int kr0 = 4 * (int)((unsigned)(KG * wave) / W);
  const int kr1 = 4 * (int)((unsigned)(KG * (wave + 1)) / W);

  // ---- 1. the activation fragments of k-tiles kr0.. (L2), the scale dwords (one per n-tile and
  //         k-group) and the granules k-tile by k-tile. Where a wave's range is one k-group
  //         (KPW = 4: 4 activation loads against 4 NT granules) the scale dwords and the first
  //         k-tile's granules go out before the activation loads, so the HBM stream starts
  //         earlier: 0.2-0.4 us less at N = 17408 K = 5120, M = 8..16 (A/B on MI355X). With
  //         longer ranges (8-12 activation loads against 2-3 granules per k-tile) the activations
  //         stay first: that order measured 0.05-0.35 us faster there.
  //         One buffer resource per n-tile, sized to end at the wave's k-range: loads past it,
  //         or of n-tile slots past the workgroup's share, return zero.
  //         Activations: token lane % 16, two 16-byte runs. Tokens past M fall outside the
  //         buffer and read as zero; a k-tile past the wave's range re-reads the row's last
  //         k-tile (clamped in scalar arithmetic), which only ever meets zero weights ----
  constexpr bool kHbmFirst = KPW == 4;
  const int m = lane & 15, g = lane >> 4;
  v4i xlo[KPW], xhi[KPW];
  if constexpr (!kHbmFirst) {
    if constexpr (H8) {
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
  }
  uint32_t sv[NT][KPW / 4];
  v4i wv[KPW][NT];
  {
    __amdgpu_buffer_rsrc_t w_src[NT], s_src[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool have = t < nth;
      w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(wbase + (uint32_t)(t * KT * kGranuleBytes)), 0,
          have ? kr1 * kGranuleBytes : 0, kBufferWord3);
      s_src[t] = __builtin_amdgcn_make_buffer_rsrc((void*)(sbase + (uint32_t)(t * KG * 256)), 0,
                                                   have ? (kr1 >> 2) * 256 : 0, kBufferWord3);
    }
    // Scale dwords are read once, like the granules. Where they go out first at M <= 8, loading
    // them non-temporal measured 0.06-0.11 us faster at N = 17408, K = 5120 (A/B on MI355X, three
    // boxes). With KPW >= 8 (activations first) it was 0.03-0.12 us slower, at M > 8 it was within
    // noise, and in gemm_stream_fq's weight waves it was slower (+0.19 us at M = 2).
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int q = 0; q < KPW / 4; ++q)
        sv[t][q] = __builtin_amdgcn_raw_buffer_load_b32(
            s_src[t], (((kr0 >> 2) + q) * 64 + lane) * 4, 0, kHbmFirst && H8 ? kBufferNT : 0);
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      if constexpr (kHbmFirst) {
        if (u == 1) {
          // KPW = 4: the activation loads, behind the first k-tile's granules
          const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
#pragma unroll
          for (int v = 0; v < KPW; ++v) {
            const int kt = min(kr0 + v, KT - 1);
            if constexpr (H8) {
              xlo[v] = __builtin_amdgcn_raw_buffer_load_b128(
                  a_src, (m & 7) * K + kt * kKTile + 64 * (m >> 3) + 16 * g, 0, 0);
            } else {
              const int off = m * K + kt * kKTile + 16 * g;
              xlo[v] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off, 0, 0);
              xhi[v] = __builtin_amdgcn_raw_buffer_load_b128(a_src, off + 64, 0, 0);
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < NT; ++t)
        wv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(
            w_src[t], (kr0 + u) * kGranuleBytes + lane * 16, 0, kBufferNT);
    }
  }
  float tok_scale;
  {
    // the epilogue's per-token scale (of the token this thread stores), last: it is needed last
    const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
    tok_scale = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(as_src, om * 4, 0, 0));
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

  // ---- 4. the W partial sums of each n-tile meet in LDS and are added in wave order. Every lane
  //         writes its partials (no branch here: the compiler would sink the MFMA operands' lane
  //         arithmetic under it, and the MFMA reads every lane); only the lanes that hold tokens
  //         are read back (at M <= 8 half of them: lanes 8..15 of each row of 16 hold other
  //         tokens' bytes). Slot c of n-tile t is (token, column group) (c % 8, c / 8) at M <= 8,
  //         (c % 16, c / 16) above, lane 16 (c / 8) + c % 8 or c. One slot per thread, every
  //         partial read before the first add ----
  v4f* red = reinterpret_cast<v4f*>(lds);
#pragma unroll
  for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t];
  __syncthreads();
  if (tid < nth * LIVE && om < M) {
    const int t = tid / LIVE, c = tid % LIVE;
    const int cl = H8 ? ((c >> 3) << 4) | (c & 7) : c;
    v4f p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = red[(w * NT + t) * 64 + cl];
    v4f v = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) v += p[w];
    const int n = (ntb0 + t) * kNTile + 4 * og;
    uint16_t* row = C + (size_t)om * N;
    if (N % 4 == 0 && ((uintptr_t)C & 7) == 0 && n + 3 < N) {
      *reinterpret_cast<uint2*>(row + n) = make_uint2(bf16x2_rne(v[0] * tok_scale, v[1] * tok_scale),
                                                      bf16x2_rne(v[2] * tok_scale, v[3] * tok_scale));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < N) row[n + i] = (uint16_t)f32_to_bf16(v[i] * tok_scale);
    }
  }
}

// gemm_stream<NT, KPW, W, true>'s loads alone (M <= 8), to measure what its load pattern costs
// without the MFMAs, the reduction and the stores. The statements of the GEMM's section 1 and its
// token-scale load: the same grid, buffer resources, offsets, cache policies and order,
// every load issued before any is used. PARTS (kStreamLoad*) picks the weight granules, the
// scale dwords, and the activation fragments with the token scale. The xor of everything read
// goes to out[0] only if it equals a fixed pattern, so the compiler cannot drop a load.
constexpr int kStreamLoadWeights = 1, kStreamLoadScales = 2, kStreamLoadActivations = 4;

template <int NT, int KPW, int W, int PARTS>
__global__ __launch_bounds__(W * 64) void gemm_stream_loads(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, int* __restrict__ out, int M, int K, int N, int S) {
  static_assert(KPW % 4 == 0 && NT >= 1 && W >= 1 && W <= 16, "stream variant");
  // K % 512 == 0; K, N > 0 (unsigned shifts: no sign fix-ups in the scalar prologue)
  const int KT = (int)((unsigned)K / kKTile), KG = (int)((unsigned)KT / kKGroup);
  const int NTILES = (int)(((unsigned)N + kNTile - 1) / kNTile);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int ntb0 = b * S, nth = min(S, NTILES - ntb0);
  // the workgroup's first granule stripe and scale rows (one 64-bit product); an n-tile's stripe
  // is t KT KiB further, below 2^31 for the NT n-tiles of a workgroup (the host checks it)
  const uint8_t* const wbase = Wq + (size_t)ntb0 * KT * kGranuleBytes;
  const uint8_t* const sbase = reinterpret_cast<const uint8_t*>(Sq) + (size_t)ntb0 * KG * 256;
  const int om = tid & 7;
  const int kr0 = 4 * (int)((unsigned)(KG * wave) / W);
  const int kr1 = 4 * (int)((unsigned)(KG * (wave + 1)) / W);
  const int m = lane & 15, g = lane >> 4;
  v4i xlo[KPW];
  uint32_t sv[NT][KPW / 4];
  v4i wv[KPW][NT];
  float tok_scale = 0.0f;
#pragma unroll
  for (int u = 0; u < KPW; ++u) {
    xlo[u] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int t = 0; t < NT; ++t) wv[u][t] = v4i{0, 0, 0, 0};
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int q = 0; q < KPW / 4; ++q) sv[t][q] = 0;
  // the GEMM's order: the activation loads first, or behind the first k-tile's granules where
  // a wave's range is one k-group
  constexpr bool kHbmFirst = KPW == 4;
  auto activations = [&]() {
    if constexpr ((PARTS & kStreamLoadActivations) != 0) {
      const auto a_src = __builtin_amdgcn_make_buffer_rsrc((void*)A, 0, M * K, kBufferWord3);
#pragma unroll
      for (int u = 0; u < KPW; ++u) {
        const int kt = min(kr0 + u, KT - 1);
        xlo[u] = __builtin_amdgcn_raw_buffer_load_b128(
            a_src, (m & 7) * K + kt * kKTile + 64 * (m >> 3) + 16 * g, 0, 0);
      }
    }
  };
  if constexpr (!kHbmFirst) activations();
  {
    __amdgpu_buffer_rsrc_t w_src[NT], s_src[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const bool have = t < nth;
      w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
          (void*)(wbase + (uint32_t)(t * KT * kGranuleBytes)), 0,
          have ? kr1 * kGranuleBytes : 0, kBufferWord3);
      s_src[t] = __builtin_amdgcn_make_buffer_rsrc((void*)(sbase + (uint32_t)(t * KG * 256)), 0,
                                                   have ? (kr1 >> 2) * 256 : 0, kBufferWord3);
    }
    if constexpr ((PARTS & kStreamLoadScales) != 0) {
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int q = 0; q < KPW / 4; ++q)
          sv[t][q] = __builtin_amdgcn_raw_buffer_load_b32(
              s_src[t], (((kr0 >> 2) + q) * 64 + lane) * 4, 0, kHbmFirst ? kBufferNT : 0);
    }
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      if (kHbmFirst && u == 1) activations();
      if constexpr ((PARTS & kStreamLoadWeights) != 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
          wv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(
              w_src[t], (kr0 + u) * kGranuleBytes + lane * 16, 0, kBufferNT);
      }
    }
  }
  if constexpr ((PARTS & kStreamLoadActivations) != 0) {
    const auto as_src = __builtin_amdgcn_make_buffer_rsrc((void*)As, 0, M * 4, kBufferWord3);
    tok_scale = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(as_src, om * 4, 0, 0));
  }
  __builtin_amdgcn_sched_barrier(0);             // every load above is issued before any is used
  v4i acc = {0, 0, 0, __float_as_int(tok_scale)};
#pragma unroll
  for (int u = 0; u < KPW; ++u) {
    acc ^= xlo[u];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc ^= wv[u][t];
  }
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int q = 0; q < KPW / 4; ++q) acc[t & 3] ^= (int)sv[t][q];
  if ((acc[0] ^ acc[1] ^ acc[2] ^ acc[3]) == 0x5A17C0DE) out[0] = b;
}

// The whole linear in one launch (bf16 activations, M <= 8): the W weight waves stream the GEMM
// as gemm_stream does, without loading activations, while the other Q = 16 - W waves of the
// workgroup quantize the bf16 rows into LDS, each a 1/Q column range of every row. Nothing
// couples the weight waves to each other before the final reduction: each issues all its scale
// and weight loads, then waits until the quantizing waves have all counted themselves done (long
// before, the rows being small), reads its fragments from LDS and multiplies as its granules land.
// The quantizing waves meet once, to take each row's amax over their partial maxima (a counter in
// LDS). The codes come from the plain quantizer's steps (row amax, row_scale, the Markstein-
// corrected quotient), so the output equals quantizer + GEMM bit for bit.
// LDS: the codes [k-tile][half][lane group][8 tokens][16 B] (KT KiB), then 8 token scales, three
// counters, Q x 8 partial maxima (512 B in all), then the partial sums. X is bf16 [M, ldx], 16-byte
// aligned rows; the host requires M <= 8, 4 <= W <= 12, K % 512 == 0 and 16 ldx < 2^31.
// SILU: X is the gate/up output of the layer before, [M, ldx] with gate in columns 0..K-1 and up in
// K..2K-1, and the row quantized is the SiLU-and-mul producer's bf16 stage,
// bf16(bf16(silu(gate)) * up), computed with the producer's own steps (w4a8_silu.h); M <= 2.
constexpr int kFqWaves = 16;           // weight waves + quantizing waves
constexpr int kFqSpin = 1 << 20;       // s_sleep(2) rounds a wave waits at most (~0.1 s)
constexpr int kFqHeader = 512;         // scales, counters, partial maxima

// the counter reaches `target` (a wave-uniform wait; bounded, so it always ends). A wait that
// runs out marks the workgroup failed in `err`: its outputs are then NaN, never plausible numbers.
__device__ __forceinline__ void fq_wait(int* counter, int target, int* err) {
  for (int it = 0; it < kFqSpin; ++it) {
    const int n = __hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (__builtin_amdgcn_readfirstlane(n) >= target) {
      asm volatile("" ::: "memory");             // the reads after the wait stay after it
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_store(err, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  asm volatile("" ::: "memory");
}

// count this wave done after its LDS writes have landed: LDS serves one wave's operations in
// order, so a wave that sees the count and then reads sees the writes (relaxed atomics and
// compiler barriers: no fence, which would also wait for the weight loads in flight)
__device__ __forceinline__ void fq_signal(int* counter) {
  __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
  asm volatile("" ::: "memory");
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

template <int NT, int KPW, int W, bool SILU>
__global__ __launch_bounds__(kFqWaves * 64) void gemm_stream_fq(
    const uint8_t* __restrict__ X, const uint8_t* __restrict__ Wq, const uint32_t* __restrict__ Sq,
    uint16_t* __restrict__ C, int M, int K, int N, int S, int ldx) {
  constexpr int Q = kFqWaves - W;                // quantizing waves
  static_assert(KPW % 4 == 0 && NT >= 1 && W >= 1 && Q >= 4 && Q <= 12, "fq variant");
  // K % 512 == 0; K, N > 0 (unsigned shifts: no sign fix-ups in the scalar prologue)
  const int KT = (int)((unsigned)K / kKTile), KG = (int)((unsigned)KT / kKGroup);
  const int NTILES = (int)(((unsigned)N + kNTile - 1) / kNTile);
  extern __shared__ __attribute__((aligned(1024))) uint8_t lds[];
  uint8_t* const codes = lds;
  float* const tsc = reinterpret_cast<float*>(lds + KT * 1024);
  // cnt[0]: maxima posted, [1]: codes done, [2]: a wait ran out
  int* const cnt = reinterpret_cast<int*>(tsc + 8);
  uint32_t* const pam = reinterpret_cast<uint32_t*>(cnt + 3);  // [Q][8] partial maxima
  v4f* const red = reinterpret_cast<v4f*>(lds + KT * 1024 + kFqHeader);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int b = blockIdx.x;
  const int ntb0 = b * S, nth = min(S, NTILES - ntb0);
  // the workgroup's first granule stripe and scale rows (one 64-bit product); an n-tile's stripe
  // is t KT KiB further, below 2^31 for the NT n-tiles of a workgroup (the host checks it)
  const uint8_t* const wbase = Wq + (size_t)ntb0 * KT * kGranuleBytes;
  const uint8_t* const sbase = reinterpret_cast<const uint8_t*>(Sq) + (size_t)ntb0 * KG * 256;
  if (wave >= W) {
    // ---- quantizing wave q: chunk columns [c0, c1) of every row (a chunk: 8 elements, 16 B),
    //      column c0 + lane + 64 i in register i. The row loads go out before the barrier below
    //      lets the weight waves start, so they are ahead of the weight stream ----
    constexpr int CH = (KPW * W + 4 * Q - 1) / (4 * Q);     // >= ceil(K / 8 / Q / 64)
    const int q = wave - W, nch = K >> 3;
    const int c0 = q * nch / Q, c1 = (q + 1) * nch / Q;
    constexpr int MR = SILU ? 2 : 8;             // rows a launch may have
    const auto x_src = __builtin_amdgcn_make_buffer_rsrc((void*)X, 0, M * ldx * 2, kBufferWord3);
    uint4 v[MR][CH], up[SILU ? MR : 1][SILU ? CH : 1];
#pragma unroll
    for (int t = 0; t < MR; ++t) {
      if (t >= M) break;                         // rows past M: no loads issued at all
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int c = c0 + lane + 64 * i;
        const int off = c < c1 ? t * ldx * 2 + 16 * c : 0x7FFFFFF0;
        v[t][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(x_src, off, 0, 0));
        if constexpr (SILU)                      // the up half: K columns (2K bytes) further
          up[t][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                         x_src, c < c1 ? off + 2 * K : 0x7FFFFFF0, 0, 0));
      }
    }
    if (q == 0 && lane < 3)
      __hip_atomic_store(&cnt[lane], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    lds_barrier();                               // (the weight waves' barrier below: one barrier)
    if constexpr (SILU) {
      // the producer's bf16 stage; chunks past the range loaded zeros and stay zero
#pragma unroll
      for (int t = 0; t < MR; ++t) {
        if (t >= M) break;
#pragma unroll
        for (int i = 0; i < CH; ++i) v[t][i] = prod::silu_mul_group(v[t][i], up[t][i]);
      }
    }
    // partial maxima of this column range, then each row's amax over the Q ranges
#pragma unroll
    for (int t = 0; t < MR; ++t) {
      if (t >= M) break;
      uint32_t am = 0;
#pragma unroll
      for (int i = 0; i < CH; ++i) am = max(am, fp8::abs_bits_max8(v[t][i]));
      am = fp8::wave_max(am);
      if (lane == 0) pam[q * 8 + t] = am;
    }
    fq_signal(&cnt[0]);
    fq_wait(&cnt[0], Q, &cnt[2]);
#pragma unroll
    for (int t = 0; t < MR; ++t) {
      if (t >= M) break;
      uint32_t am = 0;
      for (int qq = 0; qq < Q; ++qq) am = max(am, pam[qq * 8 + t]);
      const float sc = fp8::row_scale(am), rcp = 1.0f / sc;
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int c = c0 + lane + 64 * i, k0 = 8 * c, kb = k0 & 127;
        if (c < c1)
          *reinterpret_cast<uint2*>(codes + ((((k0 >> 7) * 2 + (kb >> 6)) * 4 + ((kb & 63) >> 4)) *
                                                 8 + t) * 16 + (kb & 15)) =
              fp8::quant8_any_scale(v[t][i], sc, rcp);
      }
      if (q == 0 && lane == 0) tsc[t] = sc;
    }
    fq_signal(&cnt[1]);
  } else {
    // the scale dwords go out before the barrier (beside the quantizing waves' row loads), and
    // where a wave's range is one k-group the first k-tile's granules too, the rest after it:
    // gate_up at M = 1 / 2 0.34 / 0.23 us faster (A/B on MI355X, same bits), qkv, o_proj and
    // down 0.02-0.04 us; with their first granules early as well the longer-range variants
    // (o_proj, down) measured 0.2-0.4 us slower
    constexpr bool kHbmFirst = KPW == 4;
    const int kr0 = 4 * (int)((unsigned)(KG * wave) / W);
    const int kr1 = 4 * (int)((unsigned)(KG * (wave + 1)) / W);
    // ---- scale dwords and granules, as in gemm_stream ----
    uint32_t sv[NT][KPW / 4];
    v4i wv[KPW][NT];
    {
      __amdgpu_buffer_rsrc_t w_src[NT], s_src[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bool have = t < nth;
        w_src[t] = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(wbase + (uint32_t)(t * KT * kGranuleBytes)), 0,
            have ? kr1 * kGranuleBytes : 0, kBufferWord3);
        s_src[t] = __builtin_amdgcn_make_buffer_rsrc(
            (void*)(sbase + (uint32_t)(t * KG * 256)), 0, have ? (kr1 >> 2) * 256 : 0,
            kBufferWord3);
      }
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int qq = 0; qq < KPW / 4; ++qq)
          sv[t][qq] = __builtin_amdgcn_raw_buffer_load_b32(
              s_src[t], (((kr0 >> 2) + qq) * 64 + lane) * 4, 0, 0);
      if constexpr (!kHbmFirst) lds_barrier();   // the quantizing waves' counters are cleared
#pragma unroll
      for (int u = 0; u < KPW; ++u) {
        if (kHbmFirst && u == 1) lds_barrier();  // the quantizing waves' counters are cleared
#pragma unroll
        for (int t = 0; t < NT; ++t)
          wv[u][t] = __builtin_amdgcn_raw_buffer_load_b128(
              w_src[t], (kr0 + u) * kGranuleBytes + lane * 16, 0, kBufferNT);
      }
    }
    __builtin_amdgcn_sched_barrier(0);           // every load above is issued before the wait
    fq_wait(&cnt[1], Q, &cnt[2]);                // the quantizing waves' codes
    // fragments: lane (m, g) of k-tile kt, token m (tokens past M and k-tiles past K: zero)
    const int m = lane & 15, g = lane >> 4, tm = m & 7;
    v4i xlo[KPW], xhi[KPW];
#pragma unroll
    for (int u = 0; u < KPW; ++u) {
      const int kt = kr0 + u, kc = min(kt, KT - 1);
      const bool ok = m < M && kt < KT;
      const v4i lo = *reinterpret_cast<const v4i*>(codes + (((kc * 2) * 4 + g) * 8 + tm) * 16);
      const v4i hi = *reinterpret_cast<const v4i*>(codes + (((kc * 2 + 1) * 4 + g) * 8 + tm) * 16);
      xlo[u] = ok ? lo : v4i{0, 0, 0, 0};
      xhi[u] = ok ? hi : v4i{0, 0, 0, 0};
    }
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
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(wave * NT + t) * 64 + lane] = acc[t];
  }

  // ---- the W partial sums of each n-tile, added in wave order: only the lanes of tokens < M
  //      (slot c of an n-tile: token c % 8, column group c / 8, lane 16 (c / 8) + c % 8), one
  //      slot per thread, every partial read before the first add ----
  __syncthreads();
  const int om = tid & 7;
  if (tid < nth * 32 && om < M) {
    const int t = tid >> 5, c = tid & 31, cl = ((c >> 3) << 4) | om;
    const float tok_scale = cnt[2] ? __builtin_nanf("") : tsc[om];
    v4f p[W];
#pragma unroll
    for (int w = 0; w < W; ++w) p[w] = red[(w * NT + t) * 64 + cl];
    v4f v = p[0];
#pragma unroll
    for (int w = 1; w < W; ++w) v += p[w];
    const int n = (ntb0 + t) * kNTile + 4 * (c >> 3);
    uint16_t* row = C + (size_t)om * N;
    if (N % 4 == 0 && ((uintptr_t)C & 7) == 0 && n + 3 < N) {
      *reinterpret_cast<uint2*>(row + n) = make_uint2(bf16x2_rne(v[0] * tok_scale, v[1] * tok_scale),
                                                      bf16x2_rne(v[2] * tok_scale, v[3] * tok_scale));
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < N) row[n + i] = (uint16_t)f32_to_bf16(v[i] * tok_scale);
    }
  }
}

// (NT, KPW, W): NT * KPW granules and 2 KPW activation runs per wave in registers; W waves at
// most 4 per SIMD. Chosen per shape by the host (find_stream): on shapes that fill the chip the
// fewest waves whose loads fit the register budget, otherwise the fewest granules per wave.
#define W4A8_STREAM_TABLE(X)                                                                      \
  X(1, 4, 16) X(1, 8, 16) X(2, 4, 10) X(2, 4, 12) X(2, 4, 16) X(2, 8, 9) X(3, 4, 10)              \
  X(3, 4, 12) X(4, 4, 10) X(5, 4, 10) X(6, 4, 8) X(8, 4, 8) X(3, 8, 5) X(2, 8, 6) X(2, 12, 6)      \
  X(2, 12, 4)

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
  const StreamCfg c = kStream[variant];
  const size_t red = (size_t)c.waves * c.nt * 64 * sizeof(v4f);
  // fused: the codes (1 KiB per k-tile), the scales, counters and maxima, then the partial sums
  return fused ? (size_t)(K / kKTile) * 1024 + kFqHeader + red : red;
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

// The one-launch linear where it pays. Every workgroup quantizes all M x K elements, which stays
// hidden behind its weight waves' loads only while the rows are few against the granules a weight
// wave streams. Measured on MI355X over the four Qwen3.8-27B linear shapes with the plan's variants
// (us, one launch against quantizer + GEMM): M = 1 qkv 7.05 / 9.05, o_proj 5.37 / 7.68, gate_up
// 10.33 / 11.85, down 6.44 / 9.18; M = 2 qkv 7.05, o_proj 5.71, gate_up 10.36, down 7.12 (two
// launches 7.8-12.0); M = 4 wins with 3 or more n-tiles per workgroup (qkv 7.71 / 9.18, gate_up
// 10.37 / 12.12) or at most 4 quantizer chunks (16 bytes of a row) per lane of a quantizing wave
// (o_proj with 12 quantizing waves: 7.46 / 8.10), and loses otherwise (down, 7 chunks per lane:
// 10.1 / 9.75); M = 8 loses everywhere (13.3-16.7 against 8.5-12.5). Variants also need room for
// the quantizing waves (4 <= W <= 12) and registers for their granules (NT KPW <= 24), 16-byte
// rows, every row offset in 32 bits, and the codes and partial sums within the LDS.
bool stream_linear_fits(int variant, int M, int N, int K, long ldx, int cus, size_t lds_limit) {
  const StreamCfg c = kStream[variant];
  if (M < 1 || M > 4 || c.waves < 4 || c.waves > kFqWaves - 4) return false;
  const int chunks_per_lane = ceil_div(M * (K / 8), 64 * (kFqWaves - c.waves));
  if (M > 2 && c.nt < 3 && chunks_per_lane > 4) return false;
  return c.nt * c.kpw <= 24 &&
         stream_fits(variant, M, N, K, cus, lds_limit) && ldx >= K && ldx % 8 == 0 &&
         16L * ldx < (1L << 31) && stream_lds_bytes(variant, M, K, true) <= lds_limit;
}

// fused: g.a is the bf16 activation with row stride lda elements (the quantizer runs in the
// kernel); otherwise g.a is e4m3 [M, K] and g.a_scale its per-token scales
hipError_t launch_stream(const GemmArgs& g, int variant, int cus, bool fused, long lda,
                         hipStream_t stream, bool silu) {
  const dim3 grid(stream_grid(g.N, cus)), block(kStream[variant].waves * 64);
  const int share = ceil_div(padded_n(g.N) / kNTile, (int)grid.x);   // n-tiles per workgroup
  const size_t lds = stream_lds_bytes(variant, g.M, g.K, fused);
  int idx = 0;
#define W4A8_STREAM_ATTR(kern)                                                                   \
  if (lds > 64 * 1024) {                                                                         \
    const hipError_t e = hipFuncSetAttribute((const void*)kern,                                  \
                                             hipFuncAttributeMaxDynamicSharedMemorySize,         \
                                             (int)lds);                                          \
    if (e != hipSuccess) return e;                                                               \
  }
#define W4A8_STREAM_GO(nt, kpw, w, h8)                                                           \
  {                                                                                              \
    W4A8_STREAM_ATTR((gemm_stream<nt, kpw, w, h8>))                                              \
    hipLaunchKernelGGL((gemm_stream<nt, kpw, w, h8>), grid, block, lds, stream, g.a, g.a_scale,  \
                       g.wq, g.sq, g.c, g.M, g.K, g.N, share);                            \
    return hipGetLastError();                                                                    \
  }
#define W4A8_STREAM_LAUNCH(nt, kpw, w)                                                           \
  if (idx++ == variant) {                                                                        \
    if constexpr (w >= 4 && w <= kFqWaves - 4 && nt * kpw <= 24) {                               \
      if (fused && silu) {                                                                       \
        W4A8_STREAM_ATTR((gemm_stream_fq<nt, kpw, w, true>))                                     \
        hipLaunchKernelGGL((gemm_stream_fq<nt, kpw, w, true>), grid, dim3(kFqWaves * 64), lds,    \
                           stream, g.a, g.wq, g.sq, g.c, g.M, g.K, g.N, share, (int)lda);  \
        return hipGetLastError();                                                                \
      }                                                                                          \
      if (fused) {                                                                               \
        W4A8_STREAM_ATTR((gemm_stream_fq<nt, kpw, w, false>))                                    \
        hipLaunchKernelGGL((gemm_stream_fq<nt, kpw, w, false>), grid, dim3(kFqWaves * 64), lds,   \
                           stream, g.a, g.wq, g.sq, g.c, g.M, g.K, g.N, share, (int)lda);  \
        return hipGetLastError();                                                                \
      }                                                                                          \
    }                                                                                            \
    if (fused) return hipErrorInvalidValue;                                                      \
    if (g.M <= 8) W4A8_STREAM_GO(nt, kpw, w, true)                                               \
    W4A8_STREAM_GO(nt, kpw, w, false)                                                            \
  }
  W4A8_STREAM_TABLE(W4A8_STREAM_LAUNCH)
#undef W4A8_STREAM_LAUNCH
#undef W4A8_STREAM_GO
#undef W4A8_STREAM_ATTR
  return hipErrorInvalidValue;
}

hipError_t launch_stream_loads(const GemmArgs& g, int variant, int cus, int parts, int* out,
                               hipStream_t stream) {
  const dim3 grid(stream_grid(g.N, cus)), block(kStream[variant].waves * 64);
  const int share = ceil_div(padded_n(g.N) / kNTile, (int)grid.x);
  int idx = 0;
#define W4A8_STREAM_LOADS_GO(nt, kpw, w, p)                                                      \
  if (parts == (p)) {                                                                            \
    hipLaunchKernelGGL((gemm_stream_loads<nt, kpw, w, (p)>), grid, block, 0, stream, g.a,        \
                       g.a_scale, g.wq, g.sq, out, g.M, g.K, g.N, share);                 \
    return hipGetLastError();                                                                    \
  }
#define W4A8_STREAM_LOADS(nt, kpw, w)                                                            \
  if (idx++ == variant) {                                                                        \
    W4A8_STREAM_LOADS_GO(nt, kpw, w, kStreamLoadWeights)                                         \
    W4A8_STREAM_LOADS_GO(nt, kpw, w, kStreamLoadWeights | kStreamLoadScales)                     \
    W4A8_STREAM_LOADS_GO(nt, kpw, w,                                                             \
                         kStreamLoadWeights | kStreamLoadScales | kStreamLoadActivations)        \
    return hipErrorInvalidValue;                                                                 \
  }
  W4A8_STREAM_TABLE(W4A8_STREAM_LOADS)
#undef W4A8_STREAM_LOADS
#undef W4A8_STREAM_LOADS_GO
  return hipErrorInvalidValue;
}

}  // namespace w4a8
