// Floating-point identities the GPU kernels rely on, checked on the CPU with the same IEEE fp32
// operations (gcc, -ffp-contract=off; fmaf is the correctly rounded fused multiply-add).
//
//   markstein  For every finite per-token scale s = max(fl32(amax * fl32(1/448)), 1/(448*512)),
//              amax any finite bf16 magnitude, and every bf16 x with |x| <= amax (both signs):
//              fma(-fma(s, q0, -x), y, q0) with y = fl32(1/s), q0 = fl32(x*y) equals
//              the IEEE quotient fl32(x/s), or both quotients are below 2^-12 in magnitude with
//              the same sign (where e4m3 rounds both to the same signed zero).
//   exp        The branch-free exp_f32 (a clamp to [-104, 89]) equals the branching form
//              (y > 88.7228394 -> +inf, y < fl32(-150 ln 2) -> +0) bit for bit, over every non-NaN
//              fp32 input (or every `stride`-th one). For a NaN, where the clamp returns a bound,
//              silu's dividing path x / (1 + exp(-x)) gives the bits it gives with the branching
//              form (NaN -> NaN): x's NaN.
//   fma        fmaf of float32 triples read from stdin, for pinning the oracle's fma emulation.
//
// The checks print "ok <count>" and exit 0, or print the first mismatches and exit 1.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static inline float f32(uint32_t b) { float v; memcpy(&v, &b, 4); return v; }
static inline uint32_t bits(float v) { uint32_t b; memcpy(&b, &v, 4); return b; }

static int markstein(void) {
  const float inv448 = 1.0f / 448.0f, min_scale = 1.0f / (448.0f * 512.0f);
  long bad = 0, total = 0;
#pragma omp parallel for reduction(+ : bad, total) schedule(dynamic)
  for (uint32_t am = 0; am < 0x7F80u; ++am) {
    float s = f32(am << 16) * inv448;
    if (s < min_scale) s = min_scale;
    const float y = 1.0f / s;
    for (uint32_t xb = 0; xb <= am; ++xb) {
      for (int neg = 0; neg < 2; ++neg) {
        const float x = f32((xb << 16) | (neg ? 0x80000000u : 0u));
        const float q = x / s;
        const float q0 = x * y;
        const float q1 = fmaf(-fmaf(s, q0, -x), y, q0);
        ++total;
        if (bits(q1) == bits(q)) continue;
        if (fabsf(q) < 0x1p-12f && fabsf(q1) < 0x1p-12f && signbit(q) == signbit(q1)) continue;
        ++bad;
        if (bad < 5) printf("amax=%04x x=%08x ieee=%a markstein=%a\n", am, bits(x), q, q1);
      }
    }
  }
  if (bad) { printf("markstein: %ld of %ld differ\n", bad, total); return 1; }
  printf("ok %ld\n", total);
  return 0;
}

static const float kLog2e = 0x1.715476p+0f, kLn2Hi = 0x1.62e4p-1f, kLn2Lo = 0x1.7f7d1cp-20f;
static const float kExpHi = 0x1.62e43p+6f, kExpLo = -0x1.9fe368p+6f;

static inline float exp_core(float y) {
  const float n = rintf(y * kLog2e);
  const float r = fmaf(-n, kLn2Lo, fmaf(-n, kLn2Hi, y));
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

static inline float exp_branching(float y) {
  if (y != y) return y;
  if (y > kExpHi) return INFINITY;
  if (y < kExpLo) return 0.0f;
  return exp_core(y);
}

static inline float exp_branch_free(float y_in) {
  return exp_core(fminf(fmaxf(y_in, -104.0f), 89.0f));
}

// the producers' silu on the path every group holding a NaN takes: x / (1 + e^-x)
static inline int silu_div_same(float x) {
  return bits(x / (1.0f + exp_branching(-x))) == bits(x / (1.0f + exp_branch_free(-x)));
}

static inline int exp_same(float y) {
  return y != y ? silu_div_same(-y) : bits(exp_branching(y)) == bits(exp_branch_free(y));
}

static int exp_check(long stride) {
  long bad = 0, total = 0;
#pragma omp parallel for reduction(+ : bad, total) schedule(static)
  for (long i = 0; i < (1L << 32); i += stride) {
    const float y = f32((uint32_t)i);
    ++total;
    if (!exp_same(y)) {
      ++bad;
      if (bad < 5) printf("y=%a branching=%a branch-free=%a\n", y, exp_branching(y),
                          exp_branch_free(y));
    }
  }
  // the clamp's edges, every float in [64, 128) and (-128, -64] and the specials
  for (uint32_t b = bits(64.0f); b < bits(128.0f); ++b)
    for (int neg = 0; neg < 2; ++neg) {
      const float y = f32(b | (neg ? 0x80000000u : 0u));
      ++total;
      if (!exp_same(y)) {
        ++bad;
        if (bad < 5) printf("y=%a\n", y);
      }
    }
  if (bad) { printf("exp: %ld of %ld differ\n", bad, total); return 1; }
  printf("ok %ld\n", total);
  return 0;
}

// fma: reads float32 triples (a, b, c) from stdin, writes fmaf(a, b, c) for each to stdout
static int fma_vectors(void) {
  float t[3];
  while (fread(t, sizeof(float), 3, stdin) == 3) {
    const float r = fmaf(t[0], t[1], t[2]);
    if (fwrite(&r, sizeof(float), 1, stdout) != 1) return 1;
  }
  return 0;
}

int main(int argc, char** argv) {
  if (argc >= 2 && !strcmp(argv[1], "markstein")) return markstein();
  if (argc >= 2 && !strcmp(argv[1], "exp")) return exp_check(argc >= 3 ? atol(argv[2]) : 1);
  if (argc >= 2 && !strcmp(argv[1], "fma")) return fma_vectors();
  fprintf(stderr, "usage: %s markstein | exp [stride] | fma < triples\n", argv[0]);
  return 2;
}
