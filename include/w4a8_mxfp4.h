/* C ABI of the MI355X (gfx950) MXFP4 W4A8 linear-layer library, libw4a8_mxfp4.so.
 *
 * Plain pointers, sizes and a HIP stream (as void*); no torch or C++ types cross this boundary.
 * Device pointers are HIP device addresses owned by the caller (torch allocates every buffer in the
 * Python host layer); the library never allocates device memory. Launches are asynchronous on the
 * given stream and contain no allocation, so they are HIP-graph-capture safe.
 *
 * Errors: every entry point validates its arguments BEFORE launching anything and returns
 * W4A8_OK (0) or a nonzero status; w4a8_last_error() then describes the failure (thread-local).
 * Launch failures are checked with hipGetLastError after every launch (the reference never checks,
 * sly/mxfp4/radiance_mxfp4_fp8.hip:1505-1512). This replaces the reference's std::runtime_error
 * thrown from launch_impl (sly/mxfp4/radiance_mxfp4_fp8.hip:1378-1385), which pybind11 surfaced as
 * a Python RuntimeError; the Python layer raises RuntimeError from the status.
 *
 * Formats: activations bf16 / e4m3fn [M, K] row-major with one fp32 scale per token; weights are
 * the checkpoint's packed e2m1 [N, K/2] (low nibble = even k) with e8m0 scales [N, K/32], repacked
 * once into "MFMA granules" (w4a8_repack). Output is bf16 [M, N] row-major.
 */
#ifndef W4A8_MXFP4_H_
#define W4A8_MXFP4_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A8_ABI_VERSION 2

enum {
  W4A8_OK = 0,
  W4A8_EINVAL = 1,    /* bad shape, pointer, alignment or plan */
  W4A8_ESCRATCH = 2,  /* a split-K plan was forced without enough registered scratch */
  W4A8_EHIP = 3       /* the HIP runtime reported an error at launch */
};

enum {
  W4A8_KERNEL_AUTO = 0,
  W4A8_KERNEL_SKINNY = 1,  /* split-K skinny kernel, any M <= 64 */
  W4A8_KERNEL_TILE = 2,    /* LDS-pipelined macro tiles (M > 16) */
  W4A8_KERNEL_STREAM = 3,  /* whole k-range of every wave in flight at once, M <= 16 */
  W4A8_KERNEL_RING = 4,    /* per-wave pipeline of k-tile stages, M <= 64 (forced plans only) */
  W4A8_KERNEL_TILE_AT = 5, /* the macro tiles on fragment-tiled activations (same variants) */
  W4A8_KERNEL_RING_AT = 6, /* the ring kernel on fragment-tiled activations (same variants) */
  W4A8_KERNEL_BAND = 7     /* weight waves + activation waves, 16 < M <= 64, optional K split */
};

/* Layouts of the producers' e4m3 output q (the q_layout argument).
 * W4A8_Q_ROWS: row-major [M, K].
 * W4A8_Q_TILED: fragment-tiled, the scaled MFMA's activation operand order. Tokens go in blocks
 *   of 16 (the last block padded; w4a8_tiled_bytes gives the size), each block 16 x K bytes;
 *   K % 128 == 0. In block b, k-tile t (128 k), half h (0, 1), lane l (0..63), the 16 bytes at
 *   byte ((b * K / 128 + t) * 2 + h) * 1024 + 16 * l are token 16 b + l % 16, k-bytes
 *   128 t + 16 (4 h + l / 16) .. + 15. Padding tokens are never written and never reach an output.
 * The reference's WMMA-fragment-tiled layout (sly/mxfp4/tile_layout.py:1-32) is the RDNA4 form of
 * the same idea; this one is MI355X's operand order and is not byte-compatible with it. */
enum { W4A8_Q_ROWS = 0, W4A8_Q_TILED = 1 };

/* ABI version of the loaded library (W4A8_ABI_VERSION). */
int w4a8_abi_version(void);

/* Description of the last failure on the calling thread ("" if none). */
const char* w4a8_last_error(void);

/* Capability probe, the counterpart of psw_reader_mode (sly/mxfp4/radiance_mxfp4_fp8.hip:2392):
 * the repacked weight layout this library reads. 1 = MFMA granules (16 n x 128 k, scale dwords
 * per 4 k-tiles). */
int w4a8_layout_version(void);

/* Bytes of the repacked weight (wq) and scale (sq) buffers for an N x K layer: N is padded to 16
 * and K to 512. Replaces the shape contract of permute_w / psw_pack_w_ / psw_fold_ws, which kept
 * [N, K/2] and [K/32, N] (sly/mxfp4/radiance_mxfp4.py:181-226, :311-316). */
int w4a8_packed_bytes(int N, int K, size_t* wq_bytes, size_t* sq_bytes);

/* (1) Dynamic per-token activation quantizer: bf16 x [M, K] (row stride ldx elements) ->
 * e4m3fn q [M, K] (contiguous) and fp32 scale [M]:
 *   scale = max(amax(|x|) * fl32(1/448), 1/(448*512)),  q = e4m3_rne(clamp(x / scale, +-448)).
 * Replaces the activation quant of radiance::mxfp4_linear: vllm's scaled_fp8_quant with
 * use_per_token_if_dynamic (sly/mxfp4/radiance_mxfp4.py:726-730) and its pure-torch form
 * _traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396), whose arithmetic this follows bit for bit. */
int w4a8_quant_per_token(const void* x, long ldx, void* q, float* scale, int M, int K,
                         void* stream);

/* (2) One-time weight repack: checkpoint w [N, K/2] + ws [N, K/32] -> wq, sq (w4a8_packed_bytes).
 * Out of place; the caller may copy the result back into the checkpoint storage when the sizes
 * match. Replaces the load-time repack of process_weights_after_loading: scale transpose,
 * make_row_ref, permute_w, psw_pack_w_, psw_fold_ws (sly/mxfp4/radiance_mxfp4.py:1083-1171). */
int w4a8_repack(const void* w, const void* ws, void* wq, void* sq, int N, int K, void* stream);

/* Register caller-owned split-K scratch for the current device: fp32 partials (the skinny kernel's
 * split-K and the macro tiles' K split in the decode band) and int counters (the skinny kernel's).
 * The counters must be zeroed once by the caller; the kernel's last-arriving workgroup resets each
 * counter it used, so they stay zeroed. Launches that overlap on one device race on it. Replaces
 * set_decode_scratch (sly/mxfp4/radiance_mxfp4_fp8.hip:1356-1360, registered from
 * sly/mxfp4/radiance_mxfp4.py:1054-1080). Pass NULLs to unregister. Registration is not
 * synchronized with launches on other host threads: register before they start. */
int w4a8_set_scratch(void* partial, size_t partial_bytes, void* counters, size_t counter_bytes);

/* (3) The GEMM: c[M, N] bf16 = (a[M, K] e4m3 * a_scale[m]) . dequant(wq, sq)^T, fp32 accumulate.
 * Picks the kernel from (M, N, K) (w4a8_plan). Replaces launch / launch_impl
 * (sly/mxfp4/radiance_mxfp4_fp8.hip:1375-1700): same operands, the weight in the granule layout
 * instead of fragment order + PSW + folded scales + wref. */
int w4a8_gemm(const void* a, const float* a_scale, const void* wq, const void* sq, void* c, int M,
              int N, int K, void* stream);

/* The plan w4a8_gemm would use: kernel (W4A8_KERNEL_*), variant index and K split. Counterpart of
 * the reference's band/split policy (sly/mxfp4/radiance_mxfp4_fp8.hip:1252-1343, :1390-1500) and
 * its Python replica band_map (sly/mxfp4/band_map.py:31-95). For a macro-tile plan whose
 * workgroups fill a CU each, w4a8_gemm may run the variant on the leading columns that fill whole
 * rounds of workgroups and a 128 x 128 tile variant on the rest (two launches on the stream); the
 * returned triple names the first. A tile plan with split_k > 1 (the decode band's K split) is
 * two launches under w4a8_gemm_planned too: the partial launch and the reducing launch. */
int w4a8_plan(int M, int N, int K, int* kernel, int* variant, int* split_k);

/* The GEMM on fragment-tiled activations (W4A8_Q_TILED, as the producers write them; K % 128 == 0):
 * the macro-tile kernel with the plan w4a8_gemm would take for a macro tile at this (M, N) (the
 * decode-band tiles at M <= 64). Same bits as w4a8_gemm on the row-major activations through the
 * same tile variant. Replaces launch_at (sly/mxfp4/radiance_mxfp4_fp8.hip:2236-2368). */
int w4a8_gemm_at(const void* a_tiled, const float* a_scale, const void* wq, const void* sq, void* c,
                 int M, int N, int K, void* stream);

/* Bytes of a fragment-tiled q of M tokens of K (whole 16-token blocks); K % 128 == 0. The
 * reference's producers allocate the same padded storage (sly/mxfp4/radiance_fused_norm.py:
 * 116-128). */
int w4a8_tiled_bytes(int M, int K, size_t* bytes);

/* w4a8_gemm with an explicit plan, for sweeps and tests (the reference forces cells through the
 * RADIANCE_MXFP4_DECODE_KS / _BK environment knobs, sly/mxfp4/radiance_mxfp4_fp8.hip:1464-1475).
 * split_k: the skinny kernel (1) splits K over split_k workgroups that meet in one launch
 * (registered scratch of w4a8_scratch_bytes()); the tile kernels (2, 5) with split_k > 1 run their
 * K-split form, which only the 4-wave tiles up to 64 tokens tall have (any other tile variant
 * returns W4A8_EINVAL): K over split_k workgroup rows writing fp32 partials to the registered
 * scratch (3 * M * N * 4 bytes for three splits), then a reducing launch; split_k 0 or 1 is one
 * launch. The band kernel (7) with split_k > 1 splits K over grid rows the same way (partials
 * of split_k * M * N * 4 bytes, then the reducing launch). The stream and ring kernels (3, 4, 6)
 * ignore split_k. Kernels 5 and 6 read fragment-tiled activations. */
int w4a8_gemm_planned(const void* a, const float* a_scale, const void* wq, const void* sq, void* c,
                      int M, int N, int K, int kernel, int variant, int split_k, void* stream);

/* w4a8_gemm_planned that allocates nothing and needs no registered scratch, for callers that
 * cannot allocate or register device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference. Split-K partials and counters
 * live in a static device array of the library (4 MiB + 16 KiB per device, held until the process
 * ends); the automatic plan takes only splits that fit it, and a forced plan needing more returns
 * W4A8_ESCRATCH. The array is zero-initialised static storage and the split kernels reset the
 * counters they use, so nothing is cleared at set-up. The first call on a device looks up the
 * array's address (a runtime call) and must be made outside HIP graph capture: under capture it
 * returns W4A8_EINVAL; later calls may be captured. Every call on a device shares the array: calls
 * that overlap on one device race and must be ordered by the caller (one stream, or events); a
 * captured call shares it with eager ones too. Same kernels, plans and results as
 * w4a8_gemm_planned with enough registered scratch. */
int w4a8_gemm_noalloc(const void* a, const float* a_scale, const void* wq, const void* sq, void* c,
                      int M, int N, int K, int kernel, int variant, int split_k, void* stream);

/* Number of instantiated variants of a kernel family, and their parameters:
 * skinny: p = {MT (16-token fragments), NT (n-tiles per workgroup), waves, unroll};
 * tile:   p = {WM, WN (MFMA tiles per wave), BM, BN (workgroup tile)};
 * stream: p = {NT (n-tiles per workgroup at most), KPW (k-tiles per wave at most), waves,
 *         NT * KPW (granules per wave at most)}. A stream variant serves (M, N, K) only when
 *         M <= 16, K % 512 == 0 and the shape's n-tiles per workgroup and k-tiles per wave fit it;
 *         forcing one that does not returns W4A8_EINVAL.
 * ring:   p = {MF (16-token fragments), NT (n-tiles per workgroup at most), D (k-tile stages in
 *         flight per wave), waves}. A ring variant serves (M, N, K) when M <= 16 * MF, the
 *         shape's n-tiles per workgroup fit NT and every wave owns a k-tile.
 * band:   p = {MF (16-token fragments), NT (n-tiles per workgroup at most), SG (scale dwords per
 *         n-tile a weight wave holds), R (granule k-tiles in flight per weight wave)}. Four weight
 *         waves and four activation waves per workgroup. A band variant serves (M, N, K, split_k)
 *         when M <= 16 * MF, K % 128 == 0, the shape's n-tiles per workgroup fit NT, every weight
 *         wave owns a k-tile and its k-range spans at most SG k-groups; split_k > 1 splits K over
 *         grid rows (fp32 partials in registered scratch, split_k * M * N * 4 bytes, N % 16 == 0)
 *         and adds a reducing launch. */
int w4a8_variant_count(int kernel);
int w4a8_variant_info(int kernel, int variant, int* p0, int* p1, int* p2, int* p3);

/* 1 when w4a8_gemm_planned(kernel, variant, split_k) serves an M x N x K GEMM (the shape checks it
 * makes before launching; registered scratch for a split is checked at the call), 0 when it
 * would refuse the shape, -1 for an unknown kernel. For sweeps and tests; no counterpart in the
 * reference. */
int w4a8_variant_serves(int kernel, int variant, int M, int N, int K, int split_k);

/* Diagnostic: the macro-tile variant's workgroup tile (bm tokens x bn columns), LDS pipeline
 * depth, waves per workgroup and static LDS bytes. No counterpart in the reference, whose tile
 * shapes are compile-time constants of its kernels. */
int w4a8_tile_config(int variant, int* bm, int* bn, int* stages, int* waves, int* lds_bytes);

/* Scratch a (skinny variant, split_k) plan needs for N columns: partial bytes and counter bytes. */
int w4a8_scratch_bytes(int variant, int N, int split_k, size_t* partial_bytes,
                       size_t* counter_bytes);

/* Scratch the automatic plan may use for any M <= max_m, N <= max_n and any K, plus what
 * w4a8_silu_mul_quant's split rows use: register at least this much with w4a8_set_scratch and
 * w4a8_gemm never has to give up a split for lack of room. The reference sized its decode
 * scratch from its own band limits (sly/mxfp4/radiance_mxfp4.py:1064-1070). max_n <= 2^22. */
int w4a8_workspace_bytes(int max_m, int max_n, size_t* partial_bytes, size_t* counter_bytes);

/* Quantize + GEMM in one call: the body of radiance::mxfp4_linear (sly/mxfp4/radiance_mxfp4.py:
 * 644-816) minus the output allocation, which stays with the caller (torch.empty at
 * sly/mxfp4/radiance_mxfp4.py:737). Where w4a8_linear_fused says so (M <= 2, and M <= 4 where the
 * plan leaves the quantizing waves little work; x 16-byte aligned, ldx % 8 == 0) it is one launch:
 * waves of the streaming GEMM's workgroups quantize the rows into LDS while the others stream the
 * weights; otherwise the quantizer and the GEMM, two launches on the stream. The output is the
 * same bits either way. q [M, K] and scale [M] are caller workspace (not written by the one-launch form). */
int w4a8_linear(const void* x, long ldx, void* q, float* scale, const void* wq, const void* sq,
                void* c, int M, int N, int K, void* stream);

/* 1 when w4a8_linear runs this shape (with a 16-byte aligned x) as one launch, 0 when as the
 * quantizer and the GEMM, -1 for a bad shape. No counterpart in the reference, whose op always
 * quantizes in a separate launch. */
int w4a8_linear_fused(int M, int N, int K, long ldx);

/* (4) Fused fp8 activation producers. Each writes the (q [M, K] e4m3fn, scale [M] fp32) pair of
 * entry point (1) for its bf16 result, so the pair can feed w4a8_gemm directly (the tuple branch of
 * apply_weights, radiance::mxfp4_linear_pq); q_layout W4A8_Q_TILED writes q fragment-tiled for
 * w4a8_gemm_at instead (the reference's `tiled` argument, sly/mxfp4/radiance_mxfp4_fp8.hip:2020,
 * :2161, :2198), same bytes in another order. One workgroup per row; every floating-point step is
 * fixed (no fused multiply-add, fixed summation order, correctly rounded 1/sqrt, a self-contained
 * exp), so the results are reproducible bit for bit. Rows are contiguous and 16-byte aligned. */

/* Gemma RMSNorm with residual, then quant: v = y + residual (fp32), residual_out = bf16(v),
 * x = bf16(v * rsqrt(mean(v^2) + eps) * (weight + 1)). y, residual, residual_out bf16 [M, K],
 * weight bf16 [K]; K % 8 == 0, K <= 10240. Replaces launch_add_rms_quant
 * (sly/mxfp4/radiance_mxfp4_fp8.hip:2196-2234; kernel :1834-1933), behind the reference's
 * radiance::add_rms_quant op (sly/mxfp4/radiance_fused_norm.py:132-160). */
int w4a8_add_rms_quant(const void* y, const void* residual, const void* weight, void* q,
                       float* scale, void* residual_out, int M, int K, float eps, void* stream,
                       int q_layout);

/* SiLU-and-mul, then quant: gate_up bf16 [M, 2N] (gate = columns 0..N-1, up = N..2N-1) ->
 * x = bf16(bf16(silu(gate)) * up), q [M, N]; N % 8 == 0, N <= 18432. Replaces
 * launch_silu_mul_quant (sly/mxfp4/radiance_mxfp4_fp8.hip:2019-2066; kernel :1935-2010), behind
 * radiance::silu_mul_quant (sly/mxfp4/radiance_fused_norm.py:163-187). At M <= 64 and
 * N > 16384 with scratch registered by w4a8_set_scratch (M * ceil(N / 512) * 4 bytes of
 * partials), rows are split over several workgroups in two launches; the results are the same
 * bits either way. */
int w4a8_silu_mul_quant(const void* gate_up, void* q, float* scale, int M, int N, void* stream,
                        int q_layout);

/* The bf16 stage of w4a8_silu_mul_quant without the quantization: out bf16 [M, N] =
 * bf16(bf16(silu(gate)) * up), the same bits the fused op quantizes; gate_up and out 16-byte
 * aligned, N % 8 == 0, N <= 18432. The reference swaps vLLM's SiluAndMul for the fused op
 * (sly/mxfp4/radiance_fused_norm.py:271) and has no bf16-output kernel of its own; this entry
 * point serves callers that need the bf16 activation and lets the stage be tested bit for bit. */
int w4a8_silu_mul(const void* gate_up, void* out, int M, int N, void* stream);

/* The MLP's SiLU-and-mul and down projection in one call: c bf16 [M, N] = the W4A8 linear of
 * w4a8_silu_mul_quant's (q, scale) for gate_up bf16 [M, 2K] (contiguous rows, 16-byte aligned),
 * K % 512 == 0 for the one-launch form, K <= 18432. No counterpart in the reference, whose MLP runs
 * radiance::silu_mul_quant (sly/mxfp4/radiance_fused_norm.py:163-180) and then the down
 * projection's radiance::mxfp4_linear_pq (sly/mxfp4/radiance_mxfp4.py:825-860); this replaces the
 * pair. Where w4a8_silu_mul_linear_fused says so (M <= 2) it is one launch: the streaming GEMM's
 * quantizing waves form the SiLU-and-mul stage with the producer's own steps and quantize it while
 * the weight waves stream; otherwise the producer and the GEMM, two launches. The output is the
 * same bits either way. q [M, K] and scale [M] are caller workspace (not written by the one-launch
 * form). */
int w4a8_silu_mul_linear(const void* gate_up, void* q, float* scale, const void* wq,
                         const void* sq, void* c, int M, int N, int K, void* stream);

/* 1 when w4a8_silu_mul_linear runs this shape as one launch, 0 when as two, -1 for a bad shape.
 * No counterpart in the reference. */
int w4a8_silu_mul_linear_fused(int M, int N, int K);

/* Per-head gated RMSNorm (heads of 128, norm before the gate, silu gate, weight without +1), then
 * quant: x = bf16(x * rsqrt(mean_head(x^2) + eps) * weight * silu(z)). x bf16 [M, N] contiguous,
 * z bf16 [M, N] with row stride z_stride elements (a column slice of a wider projection; a
 * multiple of 8), weight bf16 [128] shared by the heads; N % 128 == 0, N <= 10240. Replaces
 * launch_gdn_norm_quant (sly/mxfp4/radiance_mxfp4_fp8.hip:2159-2195; kernel :2068-2156), behind
 * radiance::gdn_norm_quant (sly/mxfp4/radiance_fused_norm.py:189-220). */
int w4a8_gdn_norm_quant(const void* x, const void* z, long z_stride, const void* weight, void* q,
                        float* scale, int M, int N, float eps, void* stream, int q_layout);

/* Diagnostic: the producers' fp32 silu, x / (1 + exp(-x)), of n bf16 inputs (n % 8 == 0; x
 * 16-byte aligned) into y fp32 [n], unrounded, through the same device function the gated norm
 * and SiLU-and-mul evaluate (each consecutive 8 inputs are one of their 8-element groups). Lets a
 * test compare the quotient with an exactly dividing restatement over every bf16 input. No
 * counterpart in the reference, whose silu is libm's expf and an fp32 division
 * (sly/mxfp4/radiance_mxfp4_fp8.hip:1962, :2109). */
int w4a8_silu_f32(const void* x, float* y, int n, void* stream);

/* Diagnostic: register-resident throughput probe of the scaled MFMA (fp4 A x fp8 B) the GEMMs
 * issue; shape 0 = 16x16x128, 1 = 32x32x64. Launches `blocks` workgroups of 4 waves that write
 * blocks*4 checksums to out; *flop receives the FLOP performed, the caller times the launch. The
 * counterpart of the reference's register-resident fp8 WMMA measurement, quoted at
 * sly/mxfp4/radiance_mxfp4_fp8.hip:6-10. */
int w4a8_mfma_probe(int shape, float* out, int blocks, int iters, double* flop, void* stream);

/* Diagnostic: streaming read of `bytes` (1 .. 2^31 - 2^20, 16-byte aligned buffer) with the
 * decode GEMM's launch shape (10-wave workgroups, 20 KiB of 128-bit loads in flight per wave,
 * all issued before any is used); out receives nothing unless the data xor to a fixed pattern.
 * The caller times it: the HBM read ceiling the M <= 16 GEMMs are compared against. No
 * counterpart in the reference, which quotes its decode kernel against the GDDR6 specification
 * (autoround-tests/RESULTS.md:404-405). */
int w4a8_read_probe(const void* buf, long bytes, int* out, void* stream);

/* Diagnostic: the read probe over launch shapes, to find the fastest way to stream `bytes` (1 ..
 * 2^31 - 2^20, 16-byte aligned buffer): `blocks` workgroups share the bytes in equal 1 KiB-aligned
 * ranges (the last one shorter; no workgroup may be left without bytes), and each of a variant's
 * `waves` waves reads `units` KiB of its workgroup's range as 64-lane 16-byte loads, `window` of
 * them in flight (window == units: all issued before any is used), non-temporal or not. A variant
 * that cannot cover a workgroup's range at this grid returns W4A8_EINVAL. out receives nothing
 * unless the data xor to a fixed pattern; the caller times the launch. No counterpart in the
 * reference. */
int w4a8_read_probe_variants(void);
int w4a8_read_probe_variant_info(int variant, int* waves, int* units, int* window,
                                 int* nontemporal);
int w4a8_read_probe_shape(const void* buf, long bytes, int* out, int blocks, int variant,
                          void* stream);

/* Diagnostic: the loads of the streaming GEMM that w4a8_gemm runs for (M, N, K) (M 1..8; the plan
 * must be W4A8_KERNEL_STREAM), issued exactly as that kernel issues them (same grid, buffer
 * resources, offsets, cache policies and order, all before any is used), without the MFMAs, the
 * reduction and the stores. parts: 1 the weight granules, 3 and the scale dwords, 7 and the
 * activation fragments with the token scales (every load of the GEMM). The operands are those of
 * w4a8_gemm; out (one int) receives nothing unless the data xor to a fixed pattern. The caller
 * times it, against the GEMM and the read probe. No counterpart in the reference. */
int w4a8_stream_load_probe(const void* a, const float* a_scale, const void* wq, const void* sq,
                           int M, int N, int K, int parts, int* out, void* stream);

/* Diagnostic: `count` independent scaled MFMAs (16x16x128, fp4 e2m1 A x fp8 e4m3 B, the instruction
 * every GEMM here issues) on raw lane operands, one wave per tile: a [count][64][4] dwords (16 fp4
 * bytes per lane), b [count][64][8] dwords (32 fp8 bytes per lane), sa / sb [count][64] scale
 * dwords (byte 0 used), d [count][64][4] fp32 result registers. Pins the host model of the operand
 * layout to the hardware, as the reference confirmed its gfx1201 WMMA fragment layout empirically
 * (sly/mxfp4/radiance_mxfp4_fp8.hip:24-25). */
int w4a8_mfma_tile(const void* a, const void* b, const void* sa, const void* sb, float* d,
                   int count, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A8_MXFP4_H_ */
