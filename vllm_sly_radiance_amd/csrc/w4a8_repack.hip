// One-time repack of checkpoint MXFP4 weights into MFMA granules (layout in w4a8_internal.h).
//
// Replaces the reference's load-time permute_w + psw_pack_w_ + psw_fold_ws and the scale
// transpose (sly/mxfp4/radiance_mxfp4.py:181-226, :311-316, :1083-1171). On CDNA4 no nibble
// needs to move inside a byte and no exponent needs folding: a granule lane is 16 consecutive
// checkpoint bytes, so the weight repack is a permutation of 16-byte chunks and the scale repack
// a gather of single bytes into per-lane dwords. Padding (N to 16, K to 512) is zero nibbles with
// scale 127, which contributes exactly 0 to every output.
#include "w4a8_internal.h"

namespace w4a8 {
namespace {

constexpr int kThreads = 256;

// One thread per destination 16-byte chunk: coalesced 1 KiB granule writes.
__global__ __launch_bounds__(kThreads) void repack_nibbles(const uint8_t* __restrict__ w,
                                                          uint8_t* __restrict__ wq, int N, int K,
                                                          int KT, size_t total) {
  const size_t d = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (d >= total) return;
  const int lane = (int)(d & 63);
  const size_t g = d >> 6;
  const int kt = (int)(g % KT);
  const int nt = (int)(g / KT);
  const int n = nt * kNTile + (lane & 15);
  const int kb = kt * 4 + (lane >> 4);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (n < N && kb < K / 32)
    v = *reinterpret_cast<const uint4*>(w + (size_t)n * (K / 2) + (size_t)kb * 16);
  reinterpret_cast<uint4*>(wq)[d] = v;
}

// One thread per destination scale dword: byte j = block (4 (4 kg + j) + lane / 16).
__global__ __launch_bounds__(kThreads) void repack_scales(const uint8_t* __restrict__ ws,
                                                         uint32_t* __restrict__ sq, int N, int K,
                                                         int KG, size_t total) {
  const size_t d = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (d >= total) return;
  const int lane = (int)(d & 63);
  const size_t g = d >> 6;
  const int kg = (int)(g % KG);
  const int nt = (int)(g / KG);
  const int n = nt * kNTile + (lane & 15);
  const int nb = K / 32;
  uint32_t v = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kb = (kg * 4 + j) * 4 + (lane >> 4);
    const uint32_t e = (n < N && kb < nb) ? ws[(size_t)n * nb + kb] : 127u;
    v |= e << (8 * j);
  }
  sq[d] = v;
}

}  // namespace

hipError_t launch_repack(const uint8_t* w, const uint8_t* ws, uint8_t* wq, uint32_t* sq, int N,
                         int K, hipStream_t stream) {
  const int NT = padded_n(N) / kNTile, KT = padded_k(K) / kKTile, KG = KT / kKGroup;
  const size_t chunks = (size_t)NT * KT * 64, dwords = (size_t)NT * KG * 64;
  if (chunks == 0) return hipSuccess;
  hipLaunchKernelGGL(repack_nibbles, dim3((unsigned)((chunks + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, w, wq, N, K, KT, chunks);
  hipLaunchKernelGGL(repack_scales, dim3((unsigned)((dwords + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, ws, sq, N, K, KG, dwords);
  return hipGetLastError();
}

}  // namespace w4a8
