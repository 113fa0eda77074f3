// Skinny W4A8 GEMM for decode / speculative-verify M (1..64) on gfx950: HBM streaming, split-K.
//
// Counterpart of the reference's radiance_mxfp4_fp8_gemm_decode and its split policy
// (sly/mxfp4/radiance_mxfp4_fp8.hip:981-1228, :1252-1343), redesigned for CDNA4:
//  * A workgroup owns NT n-tiles (16 columns each) and one K split; its WAVES waves take the
//    split's k-tiles round-robin, so at any moment the waves of a workgroup stream adjacent 1 KiB
//    granules. Each wave issues U k-tiles of loads (NT non-temporal 128-bit weight loads per k-tile,
//    the scale dword, MT activation fragments of two 128-bit loads each that hit L2) before the
//    U*MT*NT scaled MFMAs.
//  * The e8m0 block scale goes to the MFMA as the A-operand scale byte (the reference folds it into
//    the weight byte through kMag, exact only for exponent gaps <= 8; this is exact always).
//  * Waves reduce through LDS in wave order; K splits across workgroups (split_k > 1, used when N
//    is too small to fill the chip) write fp32 partials to caller-owned scratch, and the last
//    workgroup to arrive on an n-block sums them in split order and resets its counter. Every
//    thread fences before the agent-scope acq_rel counter bump (the reference's one-thread fence
//    bug, sly/mxfp4/radiance_mxfp4_fp8.hip:1204-1208, cannot occur). The summation order is fixed,
//    so a given (variant, split_k) is bit-reproducible from run to run.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

template <int MT, int NT, int WAVES, int U>
__global__ __launch_bounds__(WAVES * 64) void gemm_skinny(
    const uint8_t* __restrict__ A, const float* __restrict__ As, const uint8_t* __restrict__ Wq,
    const uint32_t* __restrict__ Sq, uint16_t* __restrict__ C, float* __restrict__ P,
    int* __restrict__ cnt, int M, int N, int K, int KTp, int KTe, int KG, int NTILES,
    int kt_per_split, int vec_out) {
  constexpr int SLOTS = MT * NT * 64;   // one v4f (4 outputs) per slot
  constexpr int NTHR = WAVES * 64;
  __shared__ v4f red[WAVES > 1 ? WAVES * SLOTS : 1];
  __shared__ int s_last;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb = blockIdx.x, ks = blockIdx.y, KS = gridDim.y;
  const int nt0 = nb * NT;
  const int kt_lo = ks * kt_per_split;
  const int kt_hi = min(KTe, kt_lo + kt_per_split);
  const int xm = lane & 15, xkb = lane >> 4;

  v4f acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; ++i)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int kt = kt_lo + wave; kt < kt_hi; kt += WAVES * U) {
    v4i wv[U][NT];
    uint32_t sv[U][NT];
    v8i xv[U][MT];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = kt + u * WAVES;
      const bool kin = k < kt_hi;
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        const int nt = nt0 + j;
        if (kin && nt < NTILES) {
          wv[u][j] = load_v4i_stream(Wq + (((size_t)nt * KTp + k) * 64 + lane) * 16);
          sv[u][j] = Sq[((size_t)nt * KG + (k >> 2)) * 64 + lane] >> (8 * (k & 3));
        } else {
          wv[u][j] = v4i{0, 0, 0, 0};
          sv[u][j] = 127u;
        }
      }
#pragma unroll
      for (int i = 0; i < MT; ++i) {
        const int m = i * 16 + xm;
        if (kin && m < M) xv[u][i] = load_x_frag(A + (size_t)m * K, k * kKTile, xkb, K);
        else xv[u][i] = v8i{0, 0, 0, 0, 0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[i][j] = mfma_w4a8(wv[u][j], xv[u][i], acc[i][j], sv[u][j]);
  }

  // slot = (i * NT + j) * 64 + lane  <->  tokens i*16 + lane%16, columns (nt0+j)*16 + 4*(lane/16)
  auto epilogue = [&](int slot, v4f v) {
    const int p = slot >> 6, l = slot & 63;
    const int m = (p / NT) * 16 + (l & 15);
    const int n = (nt0 + p % NT) * kNTile + 4 * (l >> 4);
    if (m < M) store_out4(C, N, m, n, N, v, As[m], vec_out != 0);
  };

  if constexpr (WAVES > 1) {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) red[(wave * MT * NT + i * NT + j) * 64 + lane] = acc[i][j];
    __syncthreads();
  }
  auto wave_sum = [&](int slot) -> v4f {
    v4f v = red[slot];
#pragma unroll
    for (int w = 1; w < WAVES; ++w) v += red[w * SLOTS + slot];
    return v;
  };

  if (KS == 1) {
    if constexpr (WAVES > 1) {
      for (int slot = threadIdx.x; slot < SLOTS; slot += NTHR) epilogue(slot, wave_sum(slot));
    } else {
#pragma unroll
      for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j) epilogue((i * NT + j) * 64 + lane, acc[i][j]);
    }
    return;
  }

  // ---- K split across workgroups: partials, then the last arrival reduces in split order ----
  v4f* Pt = reinterpret_cast<v4f*>(P) + (size_t)nb * KS * SLOTS;
  if constexpr (WAVES > 1) {
    for (int slot = threadIdx.x; slot < SLOTS; slot += NTHR) Pt[(size_t)ks * SLOTS + slot] = wave_sum(slot);
  } else {
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
      for (int j = 0; j < NT; ++j) Pt[(size_t)ks * SLOTS + (i * NT + j) * 64 + lane] = acc[i][j];
  }
  __threadfence();                       // release this thread's partials (every thread)
  __syncthreads();
  if (threadIdx.x == 0)
    s_last = __hip_atomic_fetch_add(&cnt[nb], 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
             KS - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();                       // acquire the other workgroups' partials
  for (int slot = threadIdx.x; slot < SLOTS; slot += NTHR) {
    v4f v = Pt[slot];
    for (int q = 1; q < KS; ++q) v += Pt[(size_t)q * SLOTS + slot];
    epilogue(slot, v);
  }
  if (threadIdx.x == 0) __hip_atomic_store(&cnt[nb], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// (MT, NT, WAVES, U) instantiations. WAVES * MT * NT <= 64 keeps the reduction buffer <= 64 KiB.
#define W4A8_SKINNY_TABLE(X)                                                                      \
  X(1, 1, 4, 4) X(1, 1, 8, 4) X(1, 2, 4, 4) X(1, 2, 8, 2) X(1, 4, 4, 2) X(1, 1, 16, 2)           \
  X(2, 1, 4, 4) X(2, 1, 8, 4) X(2, 2, 4, 4) X(2, 2, 8, 2) X(2, 4, 4, 2) X(2, 1, 16, 2)           \
  X(3, 1, 4, 4) X(3, 1, 8, 4) X(3, 2, 4, 2) X(3, 2, 8, 2) X(3, 4, 4, 2) X(3, 1, 16, 2)           \
  X(4, 1, 4, 4) X(4, 1, 8, 4) X(4, 2, 4, 2) X(4, 2, 8, 2) X(4, 4, 4, 2) X(4, 1, 16, 2)

#define W4A8_SKINNY_CFG(mt, nt, w, u) SkinnyCfg{mt, nt, w, u},
constexpr SkinnyCfg kSkinny[] = {W4A8_SKINNY_TABLE(W4A8_SKINNY_CFG)};
#undef W4A8_SKINNY_CFG
constexpr int kSkinnyCount = sizeof(kSkinny) / sizeof(kSkinny[0]);

}  // namespace

int skinny_variant_count() { return kSkinnyCount; }
SkinnyCfg skinny_variant(int v) { return kSkinny[v]; }

int skinny_counter_count(int variant, int N) {
  return ceil_div(padded_n(N) / kNTile, kSkinny[variant].nt);
}

size_t skinny_scratch_bytes(int variant, int N, int split_k) {
  const SkinnyCfg c = kSkinny[variant];
  return split_k <= 1 ? 0
                      : (size_t)skinny_counter_count(variant, N) * split_k * c.mt * c.nt * 64 *
                            sizeof(v4f);
}

hipError_t launch_skinny(const GemmArgs& g, int variant, int split_k, float* partial,
                         int* counters, hipStream_t stream) {
  const SkinnyCfg c = kSkinny[variant];
  const int KTp = padded_k(g.K) / kKTile, KTe = ceil_div(g.K, kKTile), KG = KTp / kKGroup;
  const int NTILES = padded_n(g.N) / kNTile;
  const int nblk = ceil_div(NTILES, c.nt);
  const int ks = split_k < 1 ? 1 : split_k;
  const int per = ceil_div(KTe, ks);
  const int vec_out = (g.N % 4 == 0 && ((uintptr_t)g.c % 8) == 0) ? 1 : 0;
  const dim3 grid(nblk, ks), block(c.waves * 64);
  int idx = 0;
#define W4A8_SKINNY_LAUNCH(mt, nt, w, u)                                                         \
  if (idx++ == variant) {                                                                        \
    hipLaunchKernelGGL((gemm_skinny<mt, nt, w, u>), grid, block, 0, stream, g.a, g.a_scale,      \
                       g.wq, g.sq, g.c, partial, counters, g.M, g.N, g.K, KTp, KTe, KG, NTILES,  \
                       per, vec_out);                                                            \
    return hipGetLastError();                                                                    \
  }
  W4A8_SKINNY_TABLE(W4A8_SKINNY_LAUNCH)
#undef W4A8_SKINNY_LAUNCH
  return hipErrorInvalidValue;
}

}  // namespace w4a8
