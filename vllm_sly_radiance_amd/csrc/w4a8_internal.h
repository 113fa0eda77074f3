// Internals shared by the MXFP4 W4A8 kernels for gfx950 (CDNA4). Not part of the C ABI.
//
// Weight layout ("MFMA granules"): one granule is the fp4 A operand of one
// v_mfma_scale_f32_16x16x128_f8f6f4: 16 output columns x 128 k = 64 lanes x 16 bytes, lane l
// holding column n0 + (l % 16) and the 32-element MX block k0/32 + l/16 as 16 consecutive
// checkpoint bytes (low nibble = even k). Granules are stored [n-tile][k-tile][lane][16 B], so a
// wave streams 1 KiB of contiguous HBM per 128-bit load. The e8m0 block scales ride in one dword per
// lane per group of four k-tiles, [n-tile][k-group][lane][4 B], byte j = k-tile 4g + j; the MFMA's
// per-lane A-scale byte is exactly the scale of that lane's block.
//
// Activations are row-major e4m3 [M, K] with one fp32 scale per token; the activation fragment is
// the MFMA's fp8 B operand with scale byte 127, and the per-token scale is applied in the
// epilogue. The fp8 operand does not follow the fp4 one: lane l (token m0 + l % 16, g = l / 16)
// holds two 16-byte runs of its row, k0 + 16g .. +15 in bytes 0-15 and k0 + 64 + 16g .. +15 in
// bytes 16-31 (measured on MI355X with one-hot operands). With unit activation scales the block
// association of those runs does not matter. D = W . X^T, so lane l, register i holds output
// (token m0 + l % 16, column n0 + 4*(l/16) + i): four consecutive bf16 per lane.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace w4a8 {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kKTile = 128;          // k per granule
constexpr int kKGroup = 4;           // k-tiles per scale dword
constexpr int kKAlign = kKTile * kKGroup;
constexpr int kNTile = 16;           // output columns per granule
constexpr int kGranuleBytes = 1024;  // 64 lanes x 16 B
constexpr uint32_t kUnitScales = 0x7F7F7F7Fu;   // e8m0 127 = 1.0 in every byte

__host__ __device__ constexpr int ceil_div(int a, int b) { return (a + b - 1) / b; }
__host__ __device__ constexpr int padded_n(int N) { return ceil_div(N, kNTile) * kNTile; }
__host__ __device__ constexpr int padded_k(int K) { return ceil_div(K, kKAlign) * kKAlign; }

// acc(16 n x 16 m) += W(16 x 128, e2m1, lane scale byte 0 of ws) . X^T(128 x 16, e4m3, scale 1)
__device__ __forceinline__ v4f mfma_w4a8(const v4i w, const v8i x, const v4f acc, uint32_t ws) {
  const v8i a = {w[0], w[1], w[2], w[3], 0, 0, 0, 0};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, x, acc, 4, 0, 0, (int)ws, 0,
                                                         (int)kUnitScales);
}

// float -> bf16 bits, round to nearest even; NaN -> 0x7FC0 | sign
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return ((u >> 16) & 0x8000u) | 0x7FC0u;
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Word 3 of a raw (stride 0) buffer resource on gfx9-family GPUs: 32-bit data format, no swizzle.
// Loads through such a resource return 0 for offsets at or past num_records, without a memory access.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kBufferNT = 2;                    // cache-policy operand: non-temporal (streamed once)

__device__ __forceinline__ v4i load_v4i(const void* p) { return *reinterpret_cast<const v4i*>(p); }

__device__ __forceinline__ v4i load_v4i_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

// The 32 activation bytes of one fp8 B-operand lane of the k-tile starting at k0: two 128-bit
// loads, row[k0 + 16g ..] and row[k0 + 64 + 16g ..], each zero past K (K is a multiple of 32, so
// a run is either wholly inside the row or wholly past it). row must be 16-byte aligned.
__device__ __forceinline__ v8i load_x_frag(const uint8_t* row, int k0, int g, int K) {
  const int ka = k0 + 16 * g, kb = ka + 64;
  const v4i lo = ka < K ? *reinterpret_cast<const v4i*>(row + ka) : v4i{0, 0, 0, 0};
  const v4i hi = kb < K ? *reinterpret_cast<const v4i*>(row + kb) : v4i{0, 0, 0, 0};
  return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Two bf16 of the hardware convert (v_cvt_pk_bf16_f32: round to nearest even, the same bits as
// f32_to_bf16 for every non-NaN input), NaNs put back to f32_to_bf16's canonical 0x7FC0 | sign.
// The convert quiets a NaN, so a NaN half has a magnitude of 0x7FC0 or more, and every other
// half (inf included) at most 0x7F80: the packed 16-bit minimum of the magnitudes with 0x7FC0,
// under the sign bits, makes exactly the canonical NaNs and leaves everything else alone. Four
// operations for the pair, no compares.
typedef __bf16 w4a8_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float w4a8_f32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned short w4a8_u16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t bf16x2_rne(float lo, float hi) {
  const uint32_t r =
      __builtin_bit_cast(uint32_t, __builtin_convertvector(w4a8_f32x2_t{lo, hi}, w4a8_bf16x2_t));
  const w4a8_u16x2_t mag = __builtin_bit_cast(w4a8_u16x2_t, r & 0x7FFF7FFFu);
  const uint32_t m = __builtin_bit_cast(
      uint32_t, __builtin_elementwise_min(mag, w4a8_u16x2_t{0x7FC0, 0x7FC0}));
  return (r & 0x80008000u) | m;
}

// Four consecutive outputs of one token, scaled and rounded, as one 8-byte store when aligned.
__device__ __forceinline__ void store_out4(uint16_t* C, int ldc, int m, int n, int N, v4f v,
                                           float scale, bool vec_ok) {
  const uint32_t b0 = f32_to_bf16(v[0] * scale), b1 = f32_to_bf16(v[1] * scale);
  const uint32_t b2 = f32_to_bf16(v[2] * scale), b3 = f32_to_bf16(v[3] * scale);
  uint16_t* row = C + (size_t)m * ldc;
  if (vec_ok && n + 3 < N) {
    *reinterpret_cast<uint2*>(row + n) = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
  } else {
    if (n < N) row[n] = (uint16_t)b0;
    if (n + 1 < N) row[n + 1] = (uint16_t)b1;
    if (n + 2 < N) row[n + 2] = (uint16_t)b2;
    if (n + 3 < N) row[n + 3] = (uint16_t)b3;
  }
}

// ---- host-side launchers (one per kernel family) ---------------------------------------------
struct GemmArgs {
  const uint8_t* a;      // e4m3 [M, K] row-major (tile kernel: or fragment-tiled)
  const float* a_scale;  // [M]
  const uint8_t* wq;     // granules
  const uint32_t* sq;    // scale dwords
  uint16_t* c;           // bf16 [M, N] with row stride ldc (elements)
  int M, N, K;
  int ldc;               // N, except for a column slice of a wider output (macro-tile family)
};

hipError_t launch_quant(const uint16_t* x, long ldx, uint8_t* q, float* s, int M, int K,
                        hipStream_t stream);
hipError_t launch_repack(const uint8_t* w, const uint8_t* ws, uint8_t* wq, uint32_t* sq, int N,
                         int K, hipStream_t stream);
// tiled: q is written fragment-tiled (K or N a multiple of 128) instead of row-major
hipError_t launch_add_rms_quant(const void* y, const void* res, const void* w, uint8_t* q,
                                float* scale, void* res_out, int M, int K, float eps, bool tiled,
                                hipStream_t stream);
// silu_mul splits rows of small M over several workgroups when `part` (the registered scratch)
// holds producer_split_bytes(M, N); otherwise one workgroup per row. Same bits either way. With
// `out` set (bf16 [M, N]) it writes the bf16 stage instead of quantizing, one workgroup per row.
size_t producer_split_bytes(int M, int N);
hipError_t launch_silu_mul_quant(const void* gate_up, uint8_t* q, float* scale, void* out, int M,
                                 int N, void* part, size_t part_bytes, bool tiled,
                                 hipStream_t stream);
// diagnostic: the producers' fp32 silu of 8 * groups bf16 inputs (16-byte aligned), unrounded
hipError_t launch_silu_probe(const void* x, float* y, int groups, hipStream_t stream);
hipError_t launch_gdn_norm_quant(const void* x, const void* z, long zs, const void* w, uint8_t* q,
                                 float* scale, int M, int N, float eps, bool tiled,
                                 hipStream_t stream);

// Skinny split-K family (M <= 64). variant indexes the instantiated (MT, NT, WAVES, U) table.
struct SkinnyCfg { int mt, nt, waves, unroll; };
int skinny_variant_count();
SkinnyCfg skinny_variant(int v);
size_t skinny_scratch_bytes(int variant, int N, int split_k);
int skinny_counter_count(int variant, int N);
hipError_t launch_skinny(const GemmArgs& g, int variant, int split_k, float* partial,
                         int* counters, hipStream_t stream);

// Streaming family (M <= 16, K % 512 == 0): grid = at most one workgroup per CU, each with the
// same number of n-tiles (at most nt); each of the `waves` waves owns a k-range of at most kpw
// k-tiles across all of them (u = nt * kpw granules in registers). variant indexes the
// instantiated table.
struct StreamCfg { int nt, kpw, waves, u; };
int stream_variant_count();
StreamCfg stream_variant(int v);
int stream_grid(int N, int cus);
size_t stream_lds_bytes(int variant, int M, int K, bool fused);
int stream_granules(int variant, int N, int K, int cus);
bool stream_fits(int variant, int M, int N, int K, int cus, size_t lds_limit);
// The variant can also run the whole linear (bf16 activations with row stride ldx elements,
// quantized in the kernel) and it pays: few rows against the weight waves' granules (M <= 2, or
// M <= 4 with 3 or more n-tiles per workgroup or at most 4 row chunks per lane of a quantizing
// wave), room for the quantizing waves, 16-byte rows, LDS.
bool stream_linear_fits(int variant, int M, int N, int K, long ldx, int cus, size_t lds_limit);
// fused: g.a is bf16 [M, K] with row stride lda elements and g.a_scale is unused; with silu too,
// g.a is the gate/up output [M, 2K] (row stride lda) and the kernel quantizes its SiLU-and-mul
// stage (M <= 2)
hipError_t launch_stream(const GemmArgs& g, int variant, int cus, bool fused, long lda,
                         hipStream_t stream, bool silu = false);
// gemm_stream's loads alone (M <= 8; parts 1: weight granules, 3: and scale dwords, 7: and the
// activation fragments with the token scale), on the GEMM's grid; out: one int, written only if
// the data xor to a fixed pattern
hipError_t launch_stream_loads(const GemmArgs& g, int variant, int cus, int parts, int* out,
                               hipStream_t stream);

// Pipelined streaming family (M <= 16 * MF): grid = at most one workgroup per CU, each with the
// same number of n-tiles (at most nt) and all of K; each of the `waves` waves streams a contiguous
// k-range with d k-tile stages in flight. variant indexes the instantiated table.
// decode-band kernel (16 < M <= 64): weight waves and activation waves, optional K split over
// grid rows (fp32 partials, then split_reduce)
struct BandCfg { int mf, nt, sg, r, d, l; };
int band_variant_count();
BandCfg band_variant(int v);
int band_grid(int N, int cus, int splits);
bool band_fits(int variant, int M, int N, int K, int cus, int splits, size_t lds_limit);
size_t band_split_bytes(int M, int N, int splits);
hipError_t launch_band(const GemmArgs& g, int variant, int cus, int splits, float* partial,
                       hipStream_t stream);
// adds `splits` fp32 partial planes P[s][M][N] in split order, scales and stores bf16 into g.c
hipError_t launch_split_reduce(const float* partial, const GemmArgs& g, int splits,
                               hipStream_t stream);

struct RingCfg { int mf, nt, d, waves; };
int ring_variant_count();
RingCfg ring_variant(int v);
int ring_grid(int variant, int N, int cus);
size_t ring_lds_bytes(int variant, int K);
bool ring_fits(int variant, int M, int N, int K, int cus, size_t lds_limit);
hipError_t launch_ring(const GemmArgs& g, int variant, int cus, bool a_tiled,
                       hipStream_t stream);

// Macro-tile family (M > 16). variant indexes the instantiated (WM, WN, NS, NW) table: nw waves of
// wm x wn 16 x 16 MFMA tiles, a bm x bn workgroup tile.
struct TileCfg { int wm, wn, bm, bn, nw, lds, ns; };
int tile_variant_count();
TileCfg tile_variant(int v);
bool tile_fits(int M, int N, int K);
// a_tiled: the activations are fragment-tiled (16-token blocks; K a multiple of 128)
// splits > 1: K split over `splits` workgroup rows into fp32 partials [splits][M][N] (N % 16 == 0),
// then a reducing launch on the same stream
hipError_t launch_tile(const GemmArgs& g, int variant, bool a_tiled, hipStream_t stream,
                       float* partial = nullptr, int splits = 1);
size_t tile_split_bytes(int M, int N, int splits);
bool tile_splits(int variant);   // the variant has a K-split form (4-wave tiles, WM <= 2)

// Register-resident MFMA throughput probe (shape 0: 16x16x128, 1: 32x32x64).
hipError_t launch_read_probe(const void* buf, int bytes, int* out, hipStream_t stream);
// launch-shape sweep of the read probe: variant v of read_variant_count(), `blocks` workgroups
int read_variant_count();
int read_variant_info(int v, int* waves, int* units, int* window, int* nt);
int read_shape_wg_bytes(int v, long bytes, int blocks);
hipError_t launch_read_shape(const void* buf, int bytes, int* out, int blocks, int v,
                             hipStream_t stream);
hipError_t launch_mfma_probe(int shape, float* out, int blocks, int iters, double* flop,
                             hipStream_t stream);
// Raw scaled-MFMA tiles on caller-given lane operands (layout diagnostic).
hipError_t launch_mfma_tiles(const int* a, const int* b, const int* sa, const int* sb, float* d,
                             int count, hipStream_t stream);

}  // namespace w4a8
