// C ABI of libw4a8_mxfp4.so: argument validation, plan selection and dispatch.
// Declarations and the reference interfaces each entry point replaces: include/w4a8_mxfp4.h.
#include <stdarg.h>
#include <atomic>
#include <mutex>
#include <stdio.h>
#include <string.h>

#include "w4a8_internal.h"
#include "w4a8_mxfp4.h"

#define W4A8_API extern "C" __attribute__((visibility("default")))

// ---- scratch of the allocation-free entry point (w4a8_gemm_noalloc) -----------------------------
// One copy per device in the code object's static data, held until the process ends: split-K
// partials first, then the counters. Every call on a device shares it; the counters start at
// zero (the array is zero-initialised static storage, so nothing is cleared at set-up) and each
// split reduction's last workgroup resets the ones it used.
constexpr size_t kStaticPartialBytes = 4u << 20;
constexpr size_t kStaticCounterBytes = 16u << 10;
static __device__ __align__(256) uint8_t scratch[kStaticPartialBytes + kStaticCounterBytes];

namespace {

using namespace w4a8;

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_status(hipError_t e, const char* what) {
  if (e == hipSuccess) return W4A8_OK;
  return fail(W4A8_EHIP, "%s: HIP error %d (%s)", what, (int)e, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Split-K scratch: fp32 partials and int counters. A view names one buffer; the registered one is
// caller-owned (w4a8_set_scratch, once per device at load time), the static one belongs to the
// allocation-free entry point (below).
struct Scratch {
  float* partial = nullptr;
  size_t partial_bytes = 0;
  int* counters = nullptr;
  size_t counter_bytes = 0;
  const char* what = "the scratch registered with w4a8_set_scratch";
};
constexpr int kMaxDevices = 64;
Scratch g_scratch[kMaxDevices];
// A view with unlimited room: plans as if every split fitted (scratch sizing queries only).
constexpr size_t kUnbounded = ~(size_t)0;
// The automatic plan splits K across workgroups only in the decode band, M <= kMaxSplitM.
constexpr int kMaxSplitM = 64;
const Scratch kPlanAnySplit{nullptr, kUnbounded, nullptr, kUnbounded, "unbounded scratch"};

int current_device() {
  int d = 0;
  if (hipGetDevice(&d) != hipSuccess || d < 0 || d >= kMaxDevices) return -1;
  return d;
}

// Compute units and the dynamic LDS a workgroup may use, per device, queried once. Without a
// device (planning on a host) the MI355X figures apply: 256 CUs, 160 KiB of LDS per workgroup.
struct DeviceInfo {
  int cus = 256;
  size_t lds = 160 * 1024;
};
// Filled once per device under a lock; the flag is published after the entry, so a reader that
// sees it set reads a complete entry without taking the lock.
DeviceInfo g_devinfo[kMaxDevices];
std::atomic<bool> g_devinfo_set[kMaxDevices];

DeviceInfo device_info(int dev) {
  if (dev < 0) return DeviceInfo{};
  if (!g_devinfo_set[dev].load(std::memory_order_acquire)) {
    static std::mutex fill;
    std::lock_guard<std::mutex> lock(fill);
    if (g_devinfo_set[dev].load(std::memory_order_relaxed)) return g_devinfo[dev];
    DeviceInfo d;
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        v > 0)
      d.cus = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
        v > 0)
      d.lds = (size_t)v;
    g_devinfo[dev] = d;
    g_devinfo_set[dev].store(true, std::memory_order_release);
  }
  return g_devinfo[dev];
}

int check_gemm_shape(const char* who, int M, int N, int K) {
  if (M < 0 || N <= 0 || K <= 0)
    return fail(W4A8_EINVAL, "%s: need M >= 0, N > 0, K > 0 (got M=%d N=%d K=%d)", who, M, N, K);
  if (K % 32)
    return fail(W4A8_EINVAL, "%s: K=%d is not a multiple of the 32-element MX block", who, K);
  if ((size_t)padded_n(N) * padded_k(K) / 2 > ((size_t)1 << 40))
    return fail(W4A8_EINVAL, "%s: N=%d K=%d is too large", who, N, K);
  return W4A8_OK;
}

int check_gemm_ptrs(const char* who, const void* a, const float* as, const void* wq,
                    const void* sq, const void* c) {
  if (!a || !as || !wq || !sq || !c) return fail(W4A8_EINVAL, "%s: null pointer", who);
  if (!aligned(a, 16) || !aligned(wq, 16) || !aligned(sq, 4) || !aligned(as, 4) || !aligned(c, 2))
    return fail(W4A8_EINVAL,
                "%s: misaligned operand (a and wq need 16 B, sq and a_scale 4 B, c 2 B)", who);
  return W4A8_OK;
}

int find_skinny(int mt, int nt, int waves) {
  for (int v = 0; v < skinny_variant_count(); ++v) {
    const SkinnyCfg c = skinny_variant(v);
    if (c.mt == mt && c.nt == nt && c.waves == waves) return v;
  }
  return -1;
}

// The first tile variant of the shape (WM, WN, NW), or of that shape and NS stages (ns > 0).
int find_tile(int wm, int wn, int nw = 4, int ns = 0) {
  for (int v = 0; v < tile_variant_count(); ++v) {
    const TileCfg c = tile_variant(v);
    if (c.wm == wm && c.wn == wn && c.nw == nw && (ns == 0 || c.ns == ns)) return v;
  }
  return -1;
}

bool scratch_fits(const Scratch& s, int variant, int N, int split_k) {
  if (split_k <= 1) return true;
  const bool room = s.partial_bytes == kUnbounded || (s.partial && s.counters);
  return room && skinny_scratch_bytes(variant, N, split_k) <= s.partial_bytes &&
         (size_t)skinny_counter_count(variant, N) * sizeof(int) <= s.counter_bytes;
}

Scratch registered_scratch(int dev) { return dev >= 0 ? g_scratch[dev] : Scratch{}; }

// The stream variant for (M, N, K). When the workgroups cover at least half the CUs (the weight
// stream is the whole cost), the fewest waves whose loads fit 160 registers (4 per granule, 4 per
// activation k-tile at M <= 8, else 8) and that leave no wave without a k-group of its own, then
// the fewest registers: every wave issues all its loads at once whatever the wave count, so fewer
// waves move the same bytes with fewer partial sums to add and fewer waves to launch. Measured on
// MI355X against the fewest-granules rule below (us, GEMM alone, M = 1 / 8 / 16): qkv
// 6.58 / 6.96 / 8.01 -> 6.30 / 6.86 / 7.58 (3 x 8 x 5 waves),
// o_proj 5.11 / 5.82 -> 4.82 / 5.50 (2 x 12 x 4), 7.01 -> 6.67 at M = 16 (2 x 8 x 6), down
// 6.19 / 7.27 -> 6.13 / 7.14 (2 x 12 x 6; at M = 16 the 2 x 12 x 6 loses, 9.06 against 8.90, and
// the budget keeps 2 x 8 x 9); gate_up keeps 5 x 4 x 10 (5 x 8 x 5 was within 1 %). Otherwise the
// fewest granules on the busiest wave, then the fewest n-tile slots, then the fewest waves.
int find_stream(int M, int N, int K, int dev) {
  const DeviceInfo d = device_info(dev);
  const bool wide = 2 * stream_grid(N, d.cus) >= d.cus;
  int best = -1;
  long best_key = 0;
  for (int v = 0; v < stream_variant_count(); ++v) {
    if (!stream_fits(v, M, N, K, d.cus, d.lds)) continue;
    const StreamCfg c = stream_variant(v);
    const int regs = 4 * c.nt * c.kpw + (M <= 8 ? 4 : 8) * c.kpw;
    const long key =
        wide && regs <= 160 && c.waves <= K / kKAlign
            ? ((long)c.waves * 4096 + regs) * 64 + c.nt
            : (1L << 40) + ((long)stream_granules(v, N, K, d.cus) * 64 + c.nt) * 64 + c.waves;
    if (best < 0 || key < best_key) best = v, best_key = key;
  }
  return best;
}

// Macro-tile candidates above the decode band, each with its measured throughput per CU
// (TFLOP/s) with one workgroup on the CU (r1) and with two workgroups' worth of tiles per CU (r2,
// running together or in two rounds). Measured on MI355X, every variant on the four Qwen3.8-27B
// linear shapes at M = 65, 96, 128, 192, 256, 384, 512, 768 and 1024 (medians over the cases with
// that many tiles per CU).
struct TileRate {
  int wm, wn, nw, ns;
  float r1, r2;
};
constexpr TileRate kMidTiles[] = {
    {2, 2, 4, 5, 3.77f, 4.59f},    // 64 x 64
    {1, 4, 4, 8, 3.79f, 3.74f},    // 32 x 128, 8 stages
    {2, 4, 4, 4, 5.60f, 6.24f},    // 64 x 128
    {2, 4, 8, 4, 8.09f, 7.83f},    // 128 x 128, 8 waves
    {2, 8, 8, 4, 9.77f, 9.51f},    // 128 x 256, 8 waves
    {4, 4, 8, 3, 11.53f, 9.96f},   // 256 x 128, 8 waves
    {4, 5, 8, 3, 12.28f, 10.09f},  // 256 x 160, 8 waves
    {4, 8, 8, 3, 13.65f, 12.41f},  // 256 x 256, 8 waves
};

// 64 < M <= 1024: the candidate with the least predicted time, tiles per CU x tile area / rate
// (r2 when the tiles come two per CU). Against the fastest variant measured at each of the 36
// points above, the pick is 0.5 % slower on average and 5.7 % at worst (gate_up M = 384); the
// first-fit rule it replaces was up to 33 % slower (qkv M = 384: 35.7 against 23.7 us).
int mid_tile(int M, int N, int cus) {
  double best = 0;
  int pick = -1;
  for (const TileRate& t : kMidTiles) {
    const int v = find_tile(t.wm, t.wn, t.nw, t.ns);
    if (v < 0) continue;
    const TileCfg c = tile_variant(v);
    const long per = ceil_div((long)ceil_div(M, c.bm) * ceil_div(N, c.bn), (long)cus);
    const double area = (double)c.bm * c.bn;
    const double cost = per == 2 ? 2 * area / t.r2 : per * area / t.r1;
    if (pick < 0 || cost < best) best = cost, pick = v;
  }
  return pick;
}

// Prefill candidates (M > 1024), each with its measured throughput per CU (TFLOP/s) over one or
// more full rounds of one workgroup per CU, and that of the 128 x 128 tiles the automatic path
// gives the columns of a ragged last round (tile_split). Measured on MI355X, every candidate on
// the four Qwen3.8-27B linear shapes at M = 1280, 1536, 2048, 2560, 3072 and 4096 with warm
// clocks (medians).
constexpr TileRate kBigTiles[] = {
    {4, 4, 8, 3, 9.75f, 0.f},   // 256 x 128
    {4, 5, 8, 3, 10.36f, 0.f},  // 256 x 160
    {4, 8, 8, 3, 12.11f, 0.f},  // 256 x 256
    {2, 8, 8, 4, 9.14f, 0.f},   // 128 x 256
};
constexpr float kSplitTailRate = 8.3f;

int tile_split(int M, int N, int variant, int dev, int* tail_variant);

// Rounds of one-per-CU workgroups for an M x N GEMM on tile c, times area / rate.
double round_cost(int M, int N, const TileCfg& c, float rate, int cus) {
  const long per = ceil_div((long)ceil_div(M, c.bm) * ceil_div(N, c.bn), (long)cus);
  return per * ((double)c.bm * c.bn) / rate;
}

// M > 1024: the candidate with the least predicted time as the automatic path would run it (its
// ragged last round split off to 128 x 128 tiles where tile_split does so). Rounds are what
// matter here: at M = 1280 .. 3072 the best tile is the one whose tiles fill whole rounds (qkv
// M = 1280: 256 x 256 in one round of 200 tiles, 56.9 us, against 80 us for 256 x 160 in 320
// tiles; o_proj and down M = 2560, 3072: 256 x 256 at 66.5-92.9 us against 90.6-122 us). Over the
// 21 measured points whose pick runs as one launch or whose split was timed, the pick is 0.1 %
// slower than the fastest candidate on average and 1.7 % at worst.
int big_tile(int M, int N, int dev) {
  const int cus = device_info(dev).cus;
  double best = 0;
  int pick = -1;
  for (const TileRate& t : kBigTiles) {
    const int v = find_tile(t.wm, t.wn, t.nw, t.ns);
    if (v < 0) continue;
    const TileCfg c = tile_variant(v);
    double cost = round_cost(M, N, c, t.r1, cus);
    int tail = -1;
    const int n_main = tile_split(M, N, v, dev, &tail);
    if (n_main > 0 && n_main < N && n_main % kNTile == 0)
      cost = round_cost(M, n_main, c, t.r1, cus) +
             round_cost(M, N - n_main, tile_variant(tail), kSplitTailRate, cus);
    if (pick < 0 || cost < best) best = cost, pick = v;
  }
  return pick;
}

// Decode / verify band: M <= 16 takes the streaming family when a variant fits (whole-K
// workgroups, every weight load in flight at once), else the skinny family, whose workgroup count
// should cover the 256 CUs several times over (for small N the K dimension is split across
// workgroups too). Above 16 tokens the macro tiles (plan_tile). The ring kernel is not in the
// automatic plan: the 8-stage narrow tiles beat it at every M from 17 to 64 on the four
// Qwen3.8-27B shapes (it stays available to a forced plan).
int plan_tile(int M, int N, int dev);

// Decode band, K split across workgroup rows (the tile kernel writes fp32 partials, a second launch
// adds them in split order). At these M every workgroup streams the whole M x K activation panel
// whatever its share of N, so a grid that leaves most CUs idle is bound by the panel each of its
// CUs fetches; splitting K three ways cuts that panel to a third at the cost of the reducing
// launch (~1.5-2 us). Measured on MI355X (graph replays over rotating weights, us, plan before ->
// split): down N=5120 K=8704 at M = 17 / 32 / 48 / 64: 11.2 -> 9.0, 11.2 -> 9.9, 12.8 -> 11.5,
// 13.0 -> 12.4 (within the spread between boxes at 64); o_proj K=6144 (12 k-groups) 8.25 -> 7.67
// at M = 17 and 8.25 -> 7.92 at 20, 2 % at 24 and nothing above; the shapes whose unsplit grid
// covers most CUs (qkv, gate_up) lose at every split. So: three splits of at least 5 k-groups
// each up to 48 tokens, or of 4 k-groups up to 20, when the unsplit grid would leave at least half
// of the CUs idle and three times it fits one round, with 32 x 64 tiles (8 stages) up to 32
// tokens and 64 x 64 (5 stages) above, and only when the scratch holds the partials. Returns the
// split (1: none).
constexpr int kBandSplit = 3, kBandSplitMaxM = 48, kBandSplitShortK = 20;

int band_split(int M, int N, int K, int cus, const Scratch& sc, int* variant) {
  if (M <= 16 || M > kBandSplitMaxM || N % kNTile) return 1;
  const int v = M <= 32 ? find_tile(1, 2, 4, 8) : find_tile(2, 2, 4, 5);
  if (v < 0) return 1;
  const TileCfg c = tile_variant(v);
  const long grid = (long)ceil_div(M, c.bm) * ceil_div(N, c.bn);
  const int kg = padded_k(K) / (kKTile * kKGroup);
  const int kg_min = (M <= kBandSplitShortK ? 4 : 5) * kBandSplit;
  if (2 * grid > cus || grid * kBandSplit > cus || kg < kg_min ||
      tile_split_bytes(M, N, kBandSplit) > sc.partial_bytes || !tile_fits(M, N, K))
    return 1;
  *variant = v;
  return kBandSplit;
}

void plan_impl(int M, int N, int K, int dev, const Scratch& sc, int* kernel, int* variant,
               int* split_k) {
  if (M <= 16) {
    const int v = find_stream(M, N, K, dev);
    if (v >= 0) {
      *kernel = W4A8_KERNEL_STREAM;
      *variant = v;
      *split_k = 1;
      return;
    }
    const int ntiles = padded_n(N) / kNTile;
    int waves = ntiles >= 512 ? 4 : ntiles >= 128 ? 8 : 16;
    int v2 = find_skinny(1, 1, waves);
    int ks = 1;
    const int kte = ceil_div(K, kKTile);
    if (ntiles < 128) {
      for (int c = 2; c <= 16 && ntiles * ks < 256; c *= 2)
        if (c <= kte / 2 && scratch_fits(sc, v2, N, c)) ks = c;
    }
    *kernel = W4A8_KERNEL_SKINNY;
    *variant = v2;
    *split_k = ks;
    return;
  }
  const DeviceInfo d = device_info(dev);
  if (M > 32 && M <= 48 && N >= 8192) {
    // 33 .. 48 tokens on the wide shapes: the band kernel (weight waves and activation waves),
    // measured on MI355X against the plan's tiles, graph replays over rotating weights: qkv
    // (10240 x 5120) 10.95 against 11.67 us at M = 48, gate_up (17408 x 5120) 14.15 against
    // 14.58 us; on the narrow shapes and at M <= 32 or 64 the tiles are as fast or faster
    // (the 48-token variant with the fewest n-tiles per workgroup that covers the shape: fewer
    // registers, and qkv on 3 n-tiles measured 10.95 against 11.63 us on 5)
    int best = -1;
    for (int v = 0; v < band_variant_count(); ++v)
      if (band_variant(v).mf == 3 && band_fits(v, M, N, K, d.cus, 1, d.lds) &&
          (best < 0 || band_variant(v).nt < band_variant(best).nt))
        best = v;
    if (best >= 0) {
      *kernel = W4A8_KERNEL_BAND;
      *variant = best;
      *split_k = 1;
      return;
    }
  }
  *kernel = W4A8_KERNEL_TILE;
  *split_k = band_split(M, N, K, d.cus, sc, variant);
  if (*split_k == 1) *variant = plan_tile(M, N, dev);
}

// The macro-tile variant for an M x N GEMM: the decode-band rule for M <= 64, the prefill rule
// below otherwise. Fragment-tiled activations always take this plan.
//
// Decode band (measured on MI355X, every tile variant up to 64 x 96 and every ring variant on the
// four Qwen3.8-27B linear shapes at M = 17 .. 64): the tiles are latency-bound here, so they run 8
// stages deep, and the fastest keep the workgroups within one per CU while staying 32 tokens tall:
//  * M <= 32: 32 tokens tall and as narrow as fits one round (N = 5120: 32 x 32, 160 workgroups;
//    10240: 32 x 64; 17408: 32 x 96): o_proj 8.6, down 10.8-11.0, qkv 8.9-10.0, gate_up 11.6-12.9
//    us, against 10.0-15.2 us for the 4-5 stage tiles and 9.5-12.3 us for the best ring kernel;
//  * M = 33 .. 64: 32 x 64 tiles over both 32-token halves when they fit one round (N = 5120: 160
//    workgroups; o_proj 9.6-9.9, down 12.1-13.2 us against 11.4-15.4 on 64-token tiles), else
//    64 x 64 (qkv, 160 workgroups, 11.8-13.2 us), else 64 x 96 in 8 waves (gate_up, 182
//    workgroups, 14.7-15.9 us).
int plan_tile(int M, int N, int dev) {
  const int cus = device_info(dev).cus;
  auto tiles = [&](int bm, int bn) { return (long)ceil_div(M, bm) * ceil_div(N, bn); };
  if (M <= 32) {
    int wn = 1;
    while (wn < 4 && tiles(32, 32 * wn) > cus) ++wn;
    return wn < 4 ? find_tile(1, wn, 4, 8) : find_tile(1, 4, 4, 4);
  }
  if (M <= 64) {
    if (tiles(32, 64) <= cus) return find_tile(1, 2, 4, 8);
    if (tiles(64, 64) <= cus) return find_tile(2, 2, 4, 5);
    if (tiles(64, 96) <= cus) return find_tile(1, 3, 8, 5);
    return find_tile(2, 4, 4, 4);
  }
  if (M <= 1024) return mid_tile(M, N, cus);
  return big_tile(M, N, dev);
}

// A tile variant whose workgroup fills a CU's LDS runs in rounds of one workgroup per CU. When the
// last round would run at under half occupancy (gate/up at M = 4096 on 256 x 256 tiles: 1088
// tiles = 4.25 rounds), the automatic path gives the variant the columns [0, n_main) that fill
// whole rounds (16384 of 17408) and the rest to 128 x 128 tiles, which fill one more, shorter
// round. Returns n_main, or 0 for no split.
int tile_split(int M, int N, int variant, int dev, int* tail_variant) {
  const TileCfg c = tile_variant(variant);
  const DeviceInfo d = device_info(dev);
  if ((size_t)2 * c.lds <= d.lds) return 0;       // two or more workgroups per CU
  const int mb = ceil_div(M, c.bm), nb = ceil_div(N, c.bn), slots = d.cus;
  const long total = (long)mb * nb;
  if (total < slots || total % slots == 0 || 2 * (total % slots) >= slots) return 0;
  int nbm = nb - 1;
  while (nbm > 0 && ((long)mb * nbm) % slots) --nbm;
  // the tail's 128 x 128 tiles: 4 stages when they fit one round (the plan's rule)
  const long tail_tiles = (long)ceil_div(M, 128) * ceil_div(N - nbm * c.bn, 128);
  const int tv = find_tile(4, 4, 4, tail_tiles <= slots ? 4 : 3);
  if (nbm <= 0 || tv < 0) return 0;
  *tail_variant = tv;
  return nbm * c.bn;
}

// Output columns [n0, n0 + n) of an M x N GEMM on one tile variant: the weights, scales and
// output are offset by n0 / 16 n-tiles; the output keeps its row stride N.
int tile_columns(const void* a, const float* as, const void* wq, const void* sq, void* c, int M,
                 int N, int K, int n0, int n, int variant, bool a_tiled, const char* who,
                 hipStream_t st) {
  const size_t kt = padded_k(K) / kKTile, nt0 = n0 / kNTile;
  const GemmArgs g{(const uint8_t*)a, as, (const uint8_t*)wq + nt0 * kt * kGranuleBytes,
                   (const uint32_t*)sq + nt0 * (kt / kKGroup) * 64, (uint16_t*)c + n0, M, n, K,
                   N};
  return hip_status(launch_tile(g, variant, a_tiled, st), who);
}

int gemm_dispatch(const void* a, const float* as, const void* wq, const void* sq, void* c, int M,
                  int N, int K, int kernel, int variant, int split_k, const Scratch& sc,
                  const char* who, void* stream) {
  const GemmArgs g{(const uint8_t*)a, as, (const uint8_t*)wq, (const uint32_t*)sq, (uint16_t*)c,
                   M, N, K, N};
  const hipStream_t st = (hipStream_t)stream;
  if (kernel == W4A8_KERNEL_SKINNY) {
    if (variant < 0 || variant >= skinny_variant_count())
      return fail(W4A8_EINVAL, "%s: skinny variant %d out of range", who, variant);
    const SkinnyCfg cfg = skinny_variant(variant);
    if (M > 16 * cfg.mt)
      return fail(W4A8_EINVAL, "%s: skinny variant %d covers M <= %d, got M=%d", who, variant,
                  16 * cfg.mt, M);
    if (split_k < 1 || split_k > 64)
      return fail(W4A8_EINVAL, "%s: split_k=%d outside 1..64", who, split_k);
    float* partial = nullptr;
    int* counters = nullptr;
    if (split_k > 1) {
      if (!scratch_fits(sc, variant, N, split_k))
        return fail(W4A8_ESCRATCH,
                    "%s: split_k=%d needs %zu B of partials and %zu B of counters; %s holds "
                    "%zu and %zu B",
                    who, split_k, skinny_scratch_bytes(variant, N, split_k),
                    (size_t)skinny_counter_count(variant, N) * sizeof(int), sc.what,
                    sc.partial_bytes, sc.counter_bytes);
      partial = sc.partial;
      counters = sc.counters;
    }
    return hip_status(launch_skinny(g, variant, split_k, partial, counters, st), who);
  }
  if (kernel == W4A8_KERNEL_TILE || kernel == W4A8_KERNEL_TILE_AT) {
    if (variant < 0 || variant >= tile_variant_count())
      return fail(W4A8_EINVAL, "%s: tile variant %d out of range", who, variant);
    if (!tile_fits(M, N, K))
      return fail(W4A8_EINVAL, "%s: M=%d K=%d exceeds the tile kernel's 32-bit offsets", who,
                  M, K);
    if (split_k > 1) {
      const int kg = padded_k(K) / (kKTile * kKGroup);
      if (!tile_splits(variant))
        return fail(W4A8_EINVAL, "%s: tile variant %d has no K-split form (4-wave tiles up to 64 "
                    "tokens tall have one)", who, variant);
      if (split_k > kg || N % kNTile)
        return fail(W4A8_EINVAL, "%s: a tile K split needs N %% %d == 0 and at most one split per "
                    "k-group (%d), got N=%d split_k=%d", who, kNTile, kg, N, split_k);
      if (tile_split_bytes(M, N, split_k) > sc.partial_bytes)
        return fail(W4A8_ESCRATCH, "%s: tile split_k=%d needs %zu B of partials; %s holds %zu B",
                    who, split_k, tile_split_bytes(M, N, split_k), sc.what, sc.partial_bytes);
      return hip_status(launch_tile(g, variant, kernel == W4A8_KERNEL_TILE_AT, st, sc.partial,
                                    split_k),
                        who);
    }
    return hip_status(launch_tile(g, variant, kernel == W4A8_KERNEL_TILE_AT, st), who);
  }
  if (kernel == W4A8_KERNEL_RING || kernel == W4A8_KERNEL_RING_AT) {
    if (variant < 0 || variant >= ring_variant_count())
      return fail(W4A8_EINVAL, "%s: ring variant %d out of range", who, variant);
    const DeviceInfo d = device_info(current_device());
    if (!ring_fits(variant, M, N, K, d.cus, d.lds))
      return fail(W4A8_EINVAL, "%s: ring variant %d does not serve M=%d N=%d K=%d", who, variant,
                  M, N, K);
    return hip_status(launch_ring(g, variant, d.cus, kernel == W4A8_KERNEL_RING_AT, st), who);
  }
  if (kernel == W4A8_KERNEL_BAND) {
    if (variant < 0 || variant >= band_variant_count())
      return fail(W4A8_EINVAL, "%s: band variant %d out of range", who, variant);
    const DeviceInfo d = device_info(current_device());
    const int splits = split_k > 1 ? split_k : 1;
    if (!band_fits(variant, M, N, K, d.cus, splits, d.lds))
      return fail(W4A8_EINVAL, "%s: band variant %d does not serve M=%d N=%d K=%d split_k=%d", who,
                  variant, M, N, K, split_k);
    if (band_split_bytes(M, N, splits) > sc.partial_bytes)
      return fail(W4A8_ESCRATCH, "%s: band split_k=%d needs %zu B of partials; %s holds %zu B",
                  who, split_k, band_split_bytes(M, N, splits), sc.what, sc.partial_bytes);
    return hip_status(launch_band(g, variant, d.cus, splits, sc.partial, st), who);
  }
  if (kernel == W4A8_KERNEL_STREAM) {
    if (variant < 0 || variant >= stream_variant_count())
      return fail(W4A8_EINVAL, "%s: stream variant %d out of range", who, variant);
    const DeviceInfo d = device_info(current_device());
    if (!stream_fits(variant, M, N, K, d.cus, d.lds))
      return fail(W4A8_EINVAL, "%s: stream variant %d does not serve M=%d N=%d K=%d",
                  who, variant, M, N, K);
    return hip_status(launch_stream(g, variant, d.cus, false, 0, st), who);
  }
  return fail(W4A8_EINVAL, "%s: unknown kernel %d", who, kernel);
}

// The GEMM on one scratch view: validation, the automatic plan (kernel == W4A8_KERNEL_AUTO) or
// the forced one, and the launch(es) on `stream`. a_tiled: the activations are fragment-tiled,
// which the tile kernel alone reads (the automatic plan is then plan_tile's).
int gemm_run(const void* a, const float* as, const void* wq, const void* sq, void* c, int M, int N,
             int K, int kernel, int variant, int split_k, bool a_tiled, const Scratch& sc,
             const char* who, void* stream) {
  if (int e = check_gemm_shape(who, M, N, K)) return e;
  a_tiled = a_tiled || kernel == W4A8_KERNEL_TILE_AT || kernel == W4A8_KERNEL_RING_AT;
  if (a_tiled && kernel != W4A8_KERNEL_AUTO && kernel != W4A8_KERNEL_TILE_AT &&
      kernel != W4A8_KERNEL_RING_AT)
    return fail(W4A8_EINVAL, "%s: fragment-tiled activations are read by the tile and ring "
                "kernels only (kernel %d)", who, kernel);
  if (a_tiled && K % kKTile)
    return fail(W4A8_EINVAL, "%s: fragment-tiled activations need K %% %d == 0, got K=%d", who,
                kKTile, K);
  if (M == 0) return W4A8_OK;
  if (int e = check_gemm_ptrs(who, a, as, wq, sq, c)) return e;
  if (kernel == W4A8_KERNEL_AUTO) {
    const int dev = current_device();
    if (a_tiled) {
      kernel = W4A8_KERNEL_TILE_AT;
      split_k = band_split(M, N, K, device_info(dev).cus, sc, &variant);
      if (split_k == 1) variant = plan_tile(M, N, dev);
    } else {
      plan_impl(M, N, K, dev, sc, &kernel, &variant, &split_k);
    }
    int tail = -1;
    const int n_main = (kernel == W4A8_KERNEL_TILE || kernel == W4A8_KERNEL_TILE_AT) &&
                               tile_fits(M, N, K)
                           ? tile_split(M, N, variant, dev, &tail)
                           : 0;
    if (n_main > 0 && n_main < N && n_main % kNTile == 0) {
      const hipStream_t st = (hipStream_t)stream;
      if (int e = tile_columns(a, as, wq, sq, c, M, N, K, 0, n_main, variant, a_tiled, who, st))
        return e;
      return tile_columns(a, as, wq, sq, c, M, N, K, n_main, N - n_main, tail, a_tiled, who, st);
    }
  }
  return gemm_dispatch(a, as, wq, sq, c, M, N, K, kernel, variant, split_k, sc, who, stream);
}

}  // namespace

W4A8_API int w4a8_abi_version(void) { return W4A8_ABI_VERSION; }

W4A8_API const char* w4a8_last_error(void) { return g_err; }

W4A8_API int w4a8_layout_version(void) { return 1; }

W4A8_API int w4a8_packed_bytes(int N, int K, size_t* wq_bytes, size_t* sq_bytes) {
  if (N <= 0 || K <= 0 || K % 32)
    return fail(W4A8_EINVAL, "w4a8_packed_bytes: need N > 0 and K a positive multiple of 32");
  if (wq_bytes) *wq_bytes = (size_t)padded_n(N) * padded_k(K) / 2;
  if (sq_bytes) *sq_bytes = (size_t)padded_n(N) * padded_k(K) / 32;
  return W4A8_OK;
}

W4A8_API int w4a8_quant_per_token(const void* x, long ldx, void* q, float* scale, int M, int K,
                                  void* stream) {
  if (M < 0 || K < 0) return fail(W4A8_EINVAL, "w4a8_quant_per_token: negative M or K");
  if (M == 0) return W4A8_OK;
  if (!x || !q || !scale) return fail(W4A8_EINVAL, "w4a8_quant_per_token: null pointer");
  if (ldx < K) return fail(W4A8_EINVAL, "w4a8_quant_per_token: ldx=%ld < K=%d", ldx, K);
  if (!aligned(x, 2) || !aligned(scale, 4))
    return fail(W4A8_EINVAL, "w4a8_quant_per_token: misaligned x or scale");
  return hip_status(launch_quant((const uint16_t*)x, ldx, (uint8_t*)q, scale, M, K,
                                 (hipStream_t)stream),
                    "w4a8_quant_per_token");
}

W4A8_API int w4a8_repack(const void* w, const void* ws, void* wq, void* sq, int N, int K,
                         void* stream) {
  if (N <= 0 || K <= 0 || K % 32)
    return fail(W4A8_EINVAL, "w4a8_repack: need N > 0 and K a positive multiple of 32 (N=%d K=%d)",
                N, K);
  if (!w || !ws || !wq || !sq) return fail(W4A8_EINVAL, "w4a8_repack: null pointer");
  if (!aligned(w, 16) || !aligned(wq, 16) || !aligned(sq, 4))
    return fail(W4A8_EINVAL, "w4a8_repack: w and wq need 16-byte alignment, sq 4-byte");
  return hip_status(launch_repack((const uint8_t*)w, (const uint8_t*)ws, (uint8_t*)wq,
                                  (uint32_t*)sq, N, K, (hipStream_t)stream),
                    "w4a8_repack");
}

W4A8_API int w4a8_set_scratch(void* partial, size_t partial_bytes, void* counters,
                              size_t counter_bytes) {
  const int dev = current_device();
  if (dev < 0) return fail(W4A8_EHIP, "w4a8_set_scratch: no current HIP device");
  if ((partial && !aligned(partial, 16)) || (counters && !aligned(counters, 4)))
    return fail(W4A8_EINVAL, "w4a8_set_scratch: partials need 16-byte, counters 4-byte alignment");
  Scratch& s = g_scratch[dev];
  s.partial = (float*)partial;
  s.partial_bytes = partial ? partial_bytes : 0;
  s.counters = (int*)counters;
  s.counter_bytes = counters ? counter_bytes : 0;
  return W4A8_OK;
}

W4A8_API int w4a8_plan(int M, int N, int K, int* kernel, int* variant, int* split_k) {
  if (int e = check_gemm_shape("w4a8_plan", M, N, K)) return e;
  if (!kernel || !variant || !split_k) return fail(W4A8_EINVAL, "w4a8_plan: null output");
  const int dev = current_device();
  plan_impl(M, N, K, dev, registered_scratch(dev), kernel, variant, split_k);
  return W4A8_OK;
}

W4A8_API int w4a8_gemm_planned(const void* a, const float* a_scale, const void* wq,
                               const void* sq, void* c, int M, int N, int K, int kernel,
                               int variant, int split_k, void* stream) {
  return gemm_run(a, a_scale, wq, sq, c, M, N, K, kernel, variant, split_k, false,
                  registered_scratch(current_device()), "w4a8_gemm", stream);
}

W4A8_API int w4a8_gemm(const void* a, const float* a_scale, const void* wq, const void* sq,
                       void* c, int M, int N, int K, void* stream) {
  return w4a8_gemm_planned(a, a_scale, wq, sq, c, M, N, K, W4A8_KERNEL_AUTO, -1, 0, stream);
}

W4A8_API int w4a8_gemm_at(const void* a_tiled, const float* a_scale, const void* wq,
                          const void* sq, void* c, int M, int N, int K, void* stream) {
  return gemm_run(a_tiled, a_scale, wq, sq, c, M, N, K, W4A8_KERNEL_AUTO, -1, 0, true,
                  registered_scratch(current_device()), "w4a8_gemm_at", stream);
}

W4A8_API int w4a8_tiled_bytes(int M, int K, size_t* bytes) {
  if (M < 0 || K <= 0 || K % kKTile || !bytes)
    return fail(W4A8_EINVAL, "w4a8_tiled_bytes: need M >= 0, K a positive multiple of %d and an "
                "output (M=%d K=%d)", kKTile, M, K);
  *bytes = (size_t)ceil_div(M, 16) * 16 * K;
  return W4A8_OK;
}

W4A8_API int w4a8_variant_count(int kernel) {
  if (kernel == W4A8_KERNEL_SKINNY) return skinny_variant_count();
  if (kernel == W4A8_KERNEL_TILE || kernel == W4A8_KERNEL_TILE_AT) return tile_variant_count();
  if (kernel == W4A8_KERNEL_STREAM) return stream_variant_count();
  if (kernel == W4A8_KERNEL_RING || kernel == W4A8_KERNEL_RING_AT) return ring_variant_count();
  if (kernel == W4A8_KERNEL_BAND) return band_variant_count();
  fail(W4A8_EINVAL, "w4a8_variant_count: unknown kernel %d", kernel);
  return -1;
}

W4A8_API int w4a8_variant_serves(int kernel, int variant, int M, int N, int K, int split_k) {
  if (M < 1 || N < 1 || K < 1 || K % 32) return 0;
  const DeviceInfo d = device_info(current_device());
  const int splits = split_k > 1 ? split_k : 1;
  switch (kernel) {
    case W4A8_KERNEL_SKINNY:
      return variant >= 0 && variant < skinny_variant_count() &&
             M <= 16 * skinny_variant(variant).mt && splits <= 64;
    case W4A8_KERNEL_TILE:
    case W4A8_KERNEL_TILE_AT: {
      if (variant < 0 || variant >= tile_variant_count() || !tile_fits(M, N, K)) return 0;
      if (kernel == W4A8_KERNEL_TILE_AT && K % kKTile) return 0;
      if (splits == 1) return 1;
      return tile_splits(variant) && splits <= padded_k(K) / (kKTile * kKGroup) && N % kNTile == 0;
    }
    case W4A8_KERNEL_STREAM:
      return variant >= 0 && variant < stream_variant_count() &&
             stream_fits(variant, M, N, K, d.cus, d.lds);
    case W4A8_KERNEL_RING:
    case W4A8_KERNEL_RING_AT:
      return variant >= 0 && variant < ring_variant_count() &&
             ring_fits(variant, M, N, K, d.cus, d.lds) &&
             (kernel == W4A8_KERNEL_RING || K % kKTile == 0);
    case W4A8_KERNEL_BAND:
      return band_fits(variant, M, N, K, d.cus, splits, d.lds);
    default:
      return fail(W4A8_EINVAL, "w4a8_variant_serves: unknown kernel %d", kernel), -1;
  }
}

W4A8_API int w4a8_tile_config(int variant, int* bm, int* bn, int* stages, int* waves,
                              int* lds_bytes) {
  if (variant < 0 || variant >= tile_variant_count())
    return fail(W4A8_EINVAL, "w4a8_tile_config: tile variant %d out of range", variant);
  const TileCfg c = tile_variant(variant);
  if (bm) *bm = c.bm;
  if (bn) *bn = c.bn;
  if (stages) *stages = c.ns;
  if (waves) *waves = c.nw;
  if (lds_bytes) *lds_bytes = c.lds;
  return W4A8_OK;
}

W4A8_API int w4a8_variant_info(int kernel, int variant, int* p0, int* p1, int* p2, int* p3) {
  int v[4];
  if (kernel == W4A8_KERNEL_SKINNY && variant >= 0 && variant < skinny_variant_count()) {
    const SkinnyCfg c = skinny_variant(variant);
    v[0] = c.mt; v[1] = c.nt; v[2] = c.waves; v[3] = c.unroll;
  } else if ((kernel == W4A8_KERNEL_TILE || kernel == W4A8_KERNEL_TILE_AT) && variant >= 0 &&
             variant < tile_variant_count()) {
    const TileCfg c = tile_variant(variant);
    v[0] = c.wm; v[1] = c.wn; v[2] = c.bm; v[3] = c.bn;
  } else if (kernel == W4A8_KERNEL_STREAM && variant >= 0 && variant < stream_variant_count()) {
    const StreamCfg c = stream_variant(variant);
    v[0] = c.nt; v[1] = c.kpw; v[2] = c.waves; v[3] = c.u;
  } else if ((kernel == W4A8_KERNEL_RING || kernel == W4A8_KERNEL_RING_AT) && variant >= 0 &&
             variant < ring_variant_count()) {
    const RingCfg c = ring_variant(variant);
    v[0] = c.mf; v[1] = c.nt; v[2] = c.d; v[3] = c.waves;
  } else if (kernel == W4A8_KERNEL_BAND && variant >= 0 && variant < band_variant_count()) {
    const BandCfg c = band_variant(variant);
    v[0] = c.mf; v[1] = c.nt; v[2] = c.sg; v[3] = c.r;
  } else {
    return fail(W4A8_EINVAL, "w4a8_variant_info: no variant %d of kernel %d", variant, kernel);
  }
  if (p0) *p0 = v[0];
  if (p1) *p1 = v[1];
  if (p2) *p2 = v[2];
  if (p3) *p3 = v[3];
  return W4A8_OK;
}

W4A8_API int w4a8_scratch_bytes(int variant, int N, int split_k, size_t* partial_bytes,
                                size_t* counter_bytes) {
  if (variant < 0 || variant >= skinny_variant_count() || N <= 0 || split_k < 1)
    return fail(W4A8_EINVAL, "w4a8_scratch_bytes: bad variant, N or split_k");
  if (partial_bytes) *partial_bytes = skinny_scratch_bytes(variant, N, split_k);
  if (counter_bytes)
    *counter_bytes = split_k > 1 ? (size_t)skinny_counter_count(variant, N) * sizeof(int) : 0;
  return W4A8_OK;
}

namespace {

// The device address of this device's static scratch, found once per device (with the device
// current) by hipGetSymbolAddress; the host-side name `scratch` is not a device address. The
// lookup is a runtime call outside any stream, so the first call on a device must not be made
// while `st` is being captured into a HIP graph: it is refused then (W4A8_EINVAL), and every later
// call, captured or not, uses the address found.
std::mutex g_static_fill;
uint8_t* g_static_addr[kMaxDevices];
std::atomic<bool> g_static_set[kMaxDevices];

int static_scratch(int dev, hipStream_t st, Scratch* out) {
  if (dev < 0) return fail(W4A8_EHIP, "w4a8_gemm_noalloc: no current HIP device");
  if (!g_static_set[dev].load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lock(g_static_fill);
    if (!g_static_set[dev].load(std::memory_order_relaxed)) {
      hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
      if (int e = hip_status(hipStreamIsCapturing(st, &cap),
                             "w4a8_gemm_noalloc: hipStreamIsCapturing"))
        return e;
      if (cap != hipStreamCaptureStatusNone)
        return fail(W4A8_EINVAL, "w4a8_gemm_noalloc: the first call on device %d is being "
                    "captured into a HIP graph; make one call outside capture first (it looks "
                    "up the static scratch's address)", dev);
      void* p = nullptr;
      if (int e = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                             "w4a8_gemm_noalloc: hipGetSymbolAddress(scratch)"))
        return e;
      if (!p || !aligned(p, 256))
        return fail(W4A8_EHIP, "w4a8_gemm_noalloc: static scratch has no usable address");
      g_static_addr[dev] = (uint8_t*)p;
      g_static_set[dev].store(true, std::memory_order_release);
    }
  }
  uint8_t* base = g_static_addr[dev];
  *out = Scratch{(float*)base, kStaticPartialBytes, (int*)(base + kStaticPartialBytes),
                 kStaticCounterBytes, "the allocation-free entry point's static scratch"};
  return W4A8_OK;
}

}  // namespace

W4A8_API int w4a8_workspace_bytes(int max_m, int max_n, size_t* partial_bytes,
                                  size_t* counter_bytes) {
  if (max_m < 1 || max_n < 1 || max_n > (1 << 22))
    return fail(W4A8_EINVAL, "w4a8_workspace_bytes: need max_m >= 1 and 1 <= max_n <= 2^22");
  const int dev = current_device();
  // The plan splits K only at M <= kMaxSplitM; a larger K never splits less, so K = 2^16 bounds
  // every K. SiLU-mul's split rows (M <= 64, N <= 18432) keep their partial maxima here too.
  size_t part = producer_split_bytes(max_m < 64 ? max_m : 64, 18432), cnt = 0;
  for (int M = 1; M <= max_m && M <= kMaxSplitM; ++M)
    for (int N = kNTile; N < max_n + kNTile; N += kNTile) {
      const int n = N < max_n ? N : max_n;
      int kernel = 0, variant = 0, split = 1;
      plan_impl(M, n, 1 << 16, dev, kPlanAnySplit, &kernel, &variant, &split);
      if (split <= 1) continue;
      if (kernel == W4A8_KERNEL_TILE) {       // the band's K split: partials only
        if (tile_split_bytes(M, n, split) > part) part = tile_split_bytes(M, n, split);
        continue;
      }
      const size_t p = skinny_scratch_bytes(variant, n, split);
      const size_t c = (size_t)skinny_counter_count(variant, n) * sizeof(int);
      if (p > part) part = p;
      if (c > cnt) cnt = c;
    }
  if (partial_bytes) *partial_bytes = part;
  if (counter_bytes) *counter_bytes = cnt;
  return W4A8_OK;
}

// The stream variant that runs the whole linear in one launch for this shape, or -1: the plan
// takes the streaming family and stream_linear_fits holds (few rows, 16-byte rows, LDS).
static int linear_fused_variant(int M, int N, int K, long ldx, bool x_aligned, int dev) {
  if (!x_aligned || M < 1 || M > 8) return -1;
  int kernel, variant, split_k;
  plan_impl(M, N, K, dev, registered_scratch(dev), &kernel, &variant, &split_k);
  if (kernel != W4A8_KERNEL_STREAM) return -1;
  const DeviceInfo d = device_info(dev);
  return stream_linear_fits(variant, M, N, K, ldx, d.cus, d.lds) ? variant : -1;
}

W4A8_API int w4a8_linear_fused(int M, int N, int K, long ldx) {
  if (check_gemm_shape("w4a8_linear_fused", M, N, K)) return -1;
  return linear_fused_variant(M, N, K, ldx, true, current_device()) >= 0 ? 1 : 0;
}

W4A8_API int w4a8_linear(const void* x, long ldx, void* q, float* scale, const void* wq,
                         const void* sq, void* c, int M, int N, int K, void* stream) {
  if (int e = check_gemm_shape("w4a8_linear", M, N, K)) return e;
  if (M == 0) return W4A8_OK;
  if (int e = check_gemm_ptrs("w4a8_linear", q, scale, wq, sq, c)) return e;
  if (!x) return fail(W4A8_EINVAL, "w4a8_linear: null x");
  if (ldx < K) return fail(W4A8_EINVAL, "w4a8_linear: ldx=%ld < K=%d", ldx, K);
  const int dev = current_device();
  const int v = linear_fused_variant(M, N, K, ldx, aligned(x, 16), dev);
  if (v >= 0) {
    const GemmArgs g{(const uint8_t*)x, nullptr, (const uint8_t*)wq, (const uint32_t*)sq,
                     (uint16_t*)c, M, N, K, N};
    return hip_status(launch_stream(g, v, device_info(dev).cus, true, ldx, (hipStream_t)stream),
                      "w4a8_linear");
  }
  if (int e = w4a8_quant_per_token(x, ldx, q, scale, M, K, stream)) return e;
  return w4a8_gemm(q, scale, wq, sq, c, M, N, K, stream);
}

// q_layout: W4A8_Q_ROWS, or W4A8_Q_TILED when the row length is whole 128-byte k-tiles
static int check_q_layout(const char* who, int q_layout, int K) {
  if (q_layout != W4A8_Q_ROWS && q_layout != W4A8_Q_TILED)
    return fail(W4A8_EINVAL, "%s: unknown q layout %d", who, q_layout);
  if (q_layout == W4A8_Q_TILED && K % kKTile)
    return fail(W4A8_EINVAL, "%s: the fragment-tiled layout needs a row length that is a "
                "multiple of %d, got %d", who, kKTile, K);
  return W4A8_OK;
}

W4A8_API int w4a8_add_rms_quant(const void* y, const void* residual, const void* weight, void* q,
                                float* scale, void* residual_out, int M, int K, float eps,
                                void* stream, int q_layout) {
  if (M < 0 || K <= 0 || K % 8 || K > 10240)
    return fail(W4A8_EINVAL, "w4a8_add_rms_quant: K must be 8-aligned and <= 10240 (M=%d K=%d)",
                M, K);
  if (int e = check_q_layout("w4a8_add_rms_quant", q_layout, K)) return e;
  if (M == 0) return W4A8_OK;
  if (!y || !residual || !weight || !q || !scale || !residual_out)
    return fail(W4A8_EINVAL, "w4a8_add_rms_quant: null pointer");
  if (!aligned(y, 16) || !aligned(residual, 16) || !aligned(weight, 16) ||
      !aligned(residual_out, 16) || !aligned(q, 8) || !aligned(scale, 4))
    return fail(W4A8_EINVAL,
                "w4a8_add_rms_quant: y, residual, weight and residual_out need 16-byte alignment, "
                "q 8-byte, scale 4-byte");
  return hip_status(launch_add_rms_quant(y, residual, weight, (uint8_t*)q, scale, residual_out, M,
                                         K, eps, q_layout == W4A8_Q_TILED, (hipStream_t)stream),
                    "w4a8_add_rms_quant");
}

W4A8_API int w4a8_silu_mul_quant(const void* gate_up, void* q, float* scale, int M, int N,
                                 void* stream, int q_layout) {
  if (M < 0 || N <= 0 || N % 8 || N > 18432)
    return fail(W4A8_EINVAL, "w4a8_silu_mul_quant: N must be 8-aligned and <= 18432 (M=%d N=%d)",
                M, N);
  if (int e = check_q_layout("w4a8_silu_mul_quant", q_layout, N)) return e;
  if (M == 0) return W4A8_OK;
  if (!gate_up || !q || !scale) return fail(W4A8_EINVAL, "w4a8_silu_mul_quant: null pointer");
  if (!aligned(gate_up, 16) || !aligned(q, 8) || !aligned(scale, 4))
    return fail(W4A8_EINVAL,
                "w4a8_silu_mul_quant: gate_up needs 16-byte alignment, q 8-byte, scale 4-byte");
  const Scratch sc = registered_scratch(current_device());
  void* part = sc.partial;
  const size_t part_bytes = sc.partial_bytes;
  return hip_status(launch_silu_mul_quant(gate_up, (uint8_t*)q, scale, nullptr, M, N, part,
                                          part_bytes, q_layout == W4A8_Q_TILED,
                                          (hipStream_t)stream),
                    "w4a8_silu_mul_quant");
}

// The SiLU-mul linear (no counterpart in the reference, whose MLP runs radiance::silu_mul_quant
// and then the down projection): one launch where the streaming GEMM's quantizing waves can take
// the SiLU-and-mul stage too (M <= 2, where w4a8_linear_fused's rule holds for rows of the gate/up
// width), else the producer and the GEMM. The same bits either way.
static int silu_linear_fused_variant(int M, int N, int K, bool gu_aligned, int dev) {
  if (M < 1 || M > 2) return -1;
  return linear_fused_variant(M, N, K, 2L * K, gu_aligned, dev);
}

W4A8_API int w4a8_silu_mul_linear_fused(int M, int N, int K) {
  if (check_gemm_shape("w4a8_silu_mul_linear_fused", M, N, K)) return -1;
  return silu_linear_fused_variant(M, N, K, true, current_device()) >= 0 ? 1 : 0;
}

W4A8_API int w4a8_silu_mul_linear(const void* gate_up, void* q, float* scale, const void* wq,
                                  const void* sq, void* c, int M, int N, int K, void* stream) {
  if (int e = check_gemm_shape("w4a8_silu_mul_linear", M, N, K)) return e;
  if (K % 8 || K > 18432)
    return fail(W4A8_EINVAL, "w4a8_silu_mul_linear: K must be 8-aligned and <= 18432 (K=%d)", K);
  if (M == 0) return W4A8_OK;
  if (int e = check_gemm_ptrs("w4a8_silu_mul_linear", q, scale, wq, sq, c)) return e;
  if (!gate_up) return fail(W4A8_EINVAL, "w4a8_silu_mul_linear: null gate_up");
  const int dev = current_device();
  const int v = silu_linear_fused_variant(M, N, K, aligned(gate_up, 16), dev);
  if (v >= 0) {
    const GemmArgs g{(const uint8_t*)gate_up, nullptr, (const uint8_t*)wq, (const uint32_t*)sq,
                     (uint16_t*)c, M, N, K, N};
    return hip_status(launch_stream(g, v, device_info(dev).cus, true, 2L * K, (hipStream_t)stream,
                                    true),
                      "w4a8_silu_mul_linear");
  }
  if (int e = w4a8_silu_mul_quant(gate_up, q, scale, M, K, stream, W4A8_Q_ROWS)) return e;
  return w4a8_gemm(q, scale, wq, sq, c, M, N, K, stream);
}

W4A8_API int w4a8_silu_mul(const void* gate_up, void* out, int M, int N, void* stream) {
  if (M < 0 || N <= 0 || N % 8 || N > 18432)
    return fail(W4A8_EINVAL, "w4a8_silu_mul: N must be 8-aligned and <= 18432 (M=%d N=%d)", M, N);
  if (M == 0) return W4A8_OK;
  if (!gate_up || !out) return fail(W4A8_EINVAL, "w4a8_silu_mul: null pointer");
  if (!aligned(gate_up, 16) || !aligned(out, 16))
    return fail(W4A8_EINVAL, "w4a8_silu_mul: gate_up and out need 16-byte alignment");
  return hip_status(launch_silu_mul_quant(gate_up, nullptr, nullptr, out, M, N, nullptr, 0,
                                          false, (hipStream_t)stream),
                    "w4a8_silu_mul");
}

W4A8_API int w4a8_gdn_norm_quant(const void* x, const void* z, long z_stride, const void* weight,
                                 void* q, float* scale, int M, int N, float eps, void* stream,
                                 int q_layout) {
  if (M < 0 || N <= 0 || N % 128 || N > 10240)
    return fail(W4A8_EINVAL,
                "w4a8_gdn_norm_quant: N must be a multiple of 128 and <= 10240 (M=%d N=%d)", M, N);
  if (int e = check_q_layout("w4a8_gdn_norm_quant", q_layout, N)) return e;
  if (M == 0) return W4A8_OK;
  if (z_stride % 8 || (M > 1 && z_stride < N))
    return fail(W4A8_EINVAL, "w4a8_gdn_norm_quant: z row stride %ld must be 8-aligned and >= N",
                z_stride);
  if (!x || !z || !weight || !q || !scale)
    return fail(W4A8_EINVAL, "w4a8_gdn_norm_quant: null pointer");
  if (!aligned(x, 16) || !aligned(z, 16) || !aligned(weight, 16) || !aligned(q, 8) ||
      !aligned(scale, 4))
    return fail(W4A8_EINVAL,
                "w4a8_gdn_norm_quant: x, z and weight need 16-byte alignment, q 8-byte, scale "
                "4-byte");
  return hip_status(launch_gdn_norm_quant(x, z, z_stride, weight, (uint8_t*)q, scale, M, N, eps,
                                          q_layout == W4A8_Q_TILED, (hipStream_t)stream),
                    "w4a8_gdn_norm_quant");
}

W4A8_API int w4a8_silu_f32(const void* x, float* y, int n, void* stream) {
  if (n < 0 || n % 8 || n > (1 << 28))
    return fail(W4A8_EINVAL, "w4a8_silu_f32: n=%d must be a multiple of 8 in 0 .. 2^28", n);
  if (n && (!x || !y || !aligned(x, 16) || !aligned(y, 4)))
    return fail(W4A8_EINVAL, "w4a8_silu_f32: x needs 16-byte alignment, y 4-byte");
  return hip_status(launch_silu_probe(x, y, n / 8, (hipStream_t)stream), "w4a8_silu_f32");
}

W4A8_API int w4a8_read_probe(const void* buf, long bytes, int* out, void* stream) {
  if (!buf || !out || bytes <= 0 || bytes > (1L << 31) - (1L << 20) || !aligned(buf, 16))
    return fail(W4A8_EINVAL,
                "w4a8_read_probe: need a 16-byte aligned buffer of 1 .. 2^31 - 2^20 bytes and out");
  return hip_status(launch_read_probe(buf, (int)bytes, out, (hipStream_t)stream),
                    "w4a8_read_probe");
}

W4A8_API int w4a8_read_probe_variants(void) { return read_variant_count(); }

W4A8_API int w4a8_read_probe_variant_info(int variant, int* waves, int* units, int* window,
                                          int* nontemporal) {
  if (!waves || !units || !window || !nontemporal ||
      !read_variant_info(variant, waves, units, window, nontemporal))
    return fail(W4A8_EINVAL, "w4a8_read_probe_variant_info: variant %d outside 0..%d or null "
                "output", variant, read_variant_count() - 1);
  return W4A8_OK;
}

W4A8_API int w4a8_read_probe_shape(const void* buf, long bytes, int* out, int blocks, int variant,
                                   void* stream) {
  if (!buf || !out || bytes <= 0 || bytes > (1L << 31) - (1L << 20) || !aligned(buf, 16))
    return fail(W4A8_EINVAL, "w4a8_read_probe_shape: need a 16-byte aligned buffer of 1 .. "
                "2^31 - 2^20 bytes and out");
  if (read_shape_wg_bytes(variant, bytes, blocks) == 0)
    return fail(W4A8_EINVAL, "w4a8_read_probe_shape: variant %d with %d workgroups cannot cover "
                "%ld bytes (or leaves a workgroup empty)", variant, blocks, bytes);
  return hip_status(launch_read_shape(buf, (int)bytes, out, blocks, variant, (hipStream_t)stream),
                    "w4a8_read_probe_shape");
}

W4A8_API int w4a8_stream_load_probe(const void* a, const float* a_scale, const void* wq,
                                    const void* sq, int M, int N, int K, int parts, int* out,
                                    void* stream) {
  const char* who = "w4a8_stream_load_probe";
  if (int e = check_gemm_shape(who, M, N, K)) return e;
  if (M < 1 || M > 8) return fail(W4A8_EINVAL, "%s: M must be 1..8 (got %d)", who, M);
  if (parts != 1 && parts != 3 && parts != 7)
    return fail(W4A8_EINVAL, "%s: parts must be 1, 3 or 7 (got %d)", who, parts);
  if (int e = check_gemm_ptrs(who, a, a_scale, wq, sq, out)) return e;
  const int dev = current_device();
  int kernel = 0, variant = -1, split_k = 1;
  plan_impl(M, N, K, dev, registered_scratch(dev), &kernel, &variant, &split_k);
  if (kernel != W4A8_KERNEL_STREAM)
    return fail(W4A8_EINVAL, "%s: the plan for M=%d N=%d K=%d is not the streaming GEMM", who, M,
                N, K);
  const GemmArgs g{(const uint8_t*)a, a_scale, (const uint8_t*)wq, (const uint32_t*)sq, nullptr,
                   M, N, K, N};
  return hip_status(
      launch_stream_loads(g, variant, device_info(dev).cus, parts, out, (hipStream_t)stream), who);
}

W4A8_API int w4a8_mfma_probe(int shape, float* out, int blocks, int iters, double* flop,
                             void* stream) {
  if ((shape != 0 && shape != 1) || !out || !flop || blocks <= 0 || iters <= 0)
    return fail(W4A8_EINVAL, "w4a8_mfma_probe: need shape 0/1, out, flop, blocks > 0, iters > 0");
  return hip_status(launch_mfma_probe(shape, out, blocks, iters, flop, (hipStream_t)stream),
                    "w4a8_mfma_probe");
}

W4A8_API int w4a8_mfma_tile(const void* a, const void* b, const void* sa, const void* sb, float* d,
                            int count, void* stream) {
  if (count < 0 || count > (1 << 24))
    return fail(W4A8_EINVAL, "w4a8_mfma_tile: count=%d outside 0..2^24", count);
  if (count == 0) return W4A8_OK;
  if (!a || !b || !sa || !sb || !d) return fail(W4A8_EINVAL, "w4a8_mfma_tile: null pointer");
  if (!aligned(a, 4) || !aligned(b, 4) || !aligned(sa, 4) || !aligned(sb, 4) || !aligned(d, 4))
    return fail(W4A8_EINVAL, "w4a8_mfma_tile: operands need 4-byte alignment");
  return hip_status(launch_mfma_tiles((const int*)a, (const int*)b, (const int*)sa,
                                      (const int*)sb, d, count, (hipStream_t)stream),
                    "w4a8_mfma_tile");
}

W4A8_API int w4a8_gemm_noalloc(const void* a, const float* a_scale, const void* wq,
                               const void* sq, void* c, int M, int N, int K, int kernel,
                               int variant, int split_k, void* stream) {
  if (int e = check_gemm_shape("w4a8_gemm_noalloc", M, N, K)) return e;
  Scratch sc;
  if (int e = static_scratch(current_device(), (hipStream_t)stream, &sc)) return e;
  return gemm_run(a, a_scale, wq, sq, c, M, N, K, kernel, variant, split_k, false, sc,
                  "w4a8_gemm_noalloc", stream);
}
