"""CPU oracle for the fused fp8 activation producers. TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the reference their results are compared
with; the product path never does.

The producers sit in front of the W4A8 GEMMs and end in the same per-token e4m3 quantizer as
``mxfp4_oracle.quant_per_token`` (the reference's ``_traced_quant``), so the (q, scale) pair they
emit can go straight to ``radiance::mxfp4_linear_pq``:

  add_rms_quant    Gemma RMSNorm with residual: fp32 add, bf16 residual out, x * rsqrt(mean(x^2) +
                   eps) * (w + 1) rounded to bf16, then quant
                   (sly/mxfp4/radiance_mxfp4_fp8.hip:1834-1933; sly/mxfp4/radiance_fused_norm.py:132-160;
                   the reference's native chain m_add_rms, sly/check_fused_norm.py:119-123)
  silu_mul_quant   silu(gate) rounded to bf16, times up rounded to bf16, then quant
                   (sly/mxfp4/radiance_mxfp4_fp8.hip:1935-2010; m_silu, sly/check_fused_norm.py:126-128)
  gdn_norm_quant   per-128-head RMSNormGated (norm before gate, silu gate, weight without +1):
                   ((x * rsqrt(mean_head(x^2) + eps)) * w) * silu(z) rounded to bf16 once, then quant
                   (sly/mxfp4/radiance_mxfp4_fp8.hip:2068-2156; m_gdn, sly/check_fused_norm.py:131-136)

Everything the reference leaves to the implementation is fixed here, so that the HIP kernels can
be held to bit-exact parity:
  * Sums of squares run in a fixed order: a thread of the 256-thread workgroup that owns a row
    accumulates its 8-element groups g = t, t + 256, ... element by element (separate fp32 multiply
    and add, no fused multiply-add); the 64 lanes of a wave then combine by an xor butterfly
    (distances 32, 16, 8, 4, 2, 1) and the four wave totals add in wave order. A gdn head sums its
    16 groups by a 16-lane xor butterfly (8, 4, 2, 1).
  * 1/sqrt is two correctly rounded fp32 operations, 1 / sqrt(.), where the reference uses the
    hardware rsqrt approximation.
  * exp is exp_f32 below (Cody-Waite reduction by ln 2 and a degree-7 Taylor polynomial by
    Horner, the reduction and every Horner step one fused multiply-add, fma_f32), where the
    reference calls libm's expf.
  * The e4m3 codes divide by the scale (IEEE fp32 division), as _traced_quant does; the
    reference's HIP producers multiply by fl32(1/scale) instead and document a possible 1-code
    difference (sly/mxfp4/radiance_mxfp4.py:383-386). With division the fused op equals
    "producer -> bf16 -> quant_per_token" bit for bit.

Pins (tests/test_oracle_producers.py): fma_f32 against C's fmaf bit for bit on edge-case and
random triples; exp_f32 and silu_f32 against float64 numpy within 2 / 4 fp32 ulp over a dense sweep and at the special values (0, +-inf, NaN, overflow and underflow edges);
the fixed-order sums against float64 sums within their rounding bound and against the same sums
re-associated by plain loops on tiny rows; every producer against the float64 formula of the
reference's native chain within one bf16 rounding, and against quant_per_token of its own bf16
intermediate bit for bit; closed forms (zero rows, weight -1 rows, rows of equal values).
"""
from __future__ import annotations

import numpy as np

from oracle import mxfp4_oracle as O

THREADS = 256                 # workgroup size of the row kernels
WAVE = 64
HEAD = 128                    # gdn head width (16 groups of 8)

F32 = np.float32
LOG2E = F32(1.4426950408889634)          # fl32(log2 e)
LN2_HI = F32(0.693145751953125)          # 0x3F317200: 16 significant bits, n * LN2_HI is exact
LN2_LO = F32(1.428606765330187e-06)      # 0x35BFBE8E: ln 2 - LN2_HI, rounded
EXP_HI = F32(88.72283935546875)          # above: exp overflows fp32
EXP_LO = F32(-103.97207641601562)        # fl32(-150 ln 2): below, exp rounds to +0
# 1/k! for k = 7 .. 0, rounded to fp32 (Horner from the top)
TAYLOR = [F32(1.0 / 5040.0), F32(1.0 / 720.0), F32(1.0 / 120.0), F32(1.0 / 24.0),
          F32(1.0 / 6.0), F32(0.5), F32(1.0), F32(1.0)]


def fma_f32(a, b, c) -> np.ndarray:
    """fl32(a * b + c) with one rounding (IEEE fusedMultiplyAdd in binary32), elementwise.

    a * b is exact in float64 (two 24-bit significands). The float64 sum s = RN64(a*b + c) may
    round; its error e = (a*b + c) - s is exact by Knuth's TwoSum. Round-to-odd repairs the double
    rounding: when e != 0 and s's last bit is even, s moves one float64 ulp towards the exact value,
    and RN32 of a round-to-odd float64 (53 >= 24 + 2 bits) equals RN32 of the exact value
    (Boldo and Melquiond, "Emulation of FMA and correctly rounded sums: proved algorithms using
    rounding to odd", IEEE TC 57(4), 2008). Non-finite results pass through from the float64 sum."""
    a64 = np.asarray(a, dtype=F32).astype(np.float64)
    b64 = np.asarray(b, dtype=F32).astype(np.float64)
    c64 = np.asarray(c, dtype=F32).astype(np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        p = a64 * b64
        s = p + c64
        bv = s - p
        err = (p - (s - bv)) + (c64 - bv)
        bits = np.ascontiguousarray(s).view(np.int64)
        fix = np.isfinite(s) & np.isfinite(err) & (err != 0) & ((bits & 1) == 0)
        step = np.where(np.signbit(s) == (err < 0), 1, -1).astype(np.int64)   # away from / to 0
        s_odd = np.where(fix, bits + step, bits).view(np.float64)
        return s_odd.astype(F32)


def exp_f32(y: np.ndarray) -> np.ndarray:
    """e^y in fp32, every step one correctly rounded fp32 operation or fused multiply-add:
        n = rint(y * log2e);  r = fma(-n, ln2_lo, fma(-n, ln2_hi, y));  p = Taylor_7(r) by Horner
        with fma;  e^y = ldexp(p, n);  y > EXP_HI -> inf, y < EXP_LO -> +0, NaN -> NaN."""
    y = np.asarray(y, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        yc = np.where(np.isfinite(y), y, F32(0)).astype(F32)
        n = np.rint((yc * LOG2E).astype(F32)).astype(F32)
        r = fma_f32(-n, LN2_LO, fma_f32(-n, LN2_HI, yc))
        p = TAYLOR[0]
        for c in TAYLOR[1:]:
            p = fma_f32(p, r, c)
        e = np.ldexp(p, n.astype(np.int32)).astype(F32)
        e = np.where(y > EXP_HI, F32(np.inf), e)
        e = np.where(y < EXP_LO, F32(0), e)
        e = np.where(np.isnan(y), y, e)
    return e.astype(F32)


def silu_f32(x: np.ndarray) -> np.ndarray:
    """x / (1 + exp_f32(-x)) in fp32 (the fp32 silu of sly/mxfp4/radiance_mxfp4_fp8.hip:1962, :2109)."""
    x = np.asarray(x, dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        d = (F32(1) + exp_f32(-x)).astype(F32)
        return (x / d).astype(F32)


def _thread_layout(v: np.ndarray) -> np.ndarray:
    """[M, K] (K % 8 == 0) -> [M, G, THREADS, 8]: group g = i * THREADS + t, zero-padded."""
    M, K = v.shape
    kv = K // 8
    G = -(-kv // THREADS)
    pad = np.zeros((M, G * THREADS * 8), dtype=F32)
    pad[:, :K] = v
    return pad.reshape(M, G, THREADS, 8)


def row_sum_squares(v: np.ndarray) -> np.ndarray:
    """Sum of v^2 over each row in the kernel's fixed order (module docstring)."""
    vt = _thread_layout(np.asarray(v, dtype=F32))
    M, G = vt.shape[0], vt.shape[1]
    part = np.zeros((M, THREADS), dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        for i in range(G):
            for j in range(8):
                part = (part + (vt[:, i, :, j] * vt[:, i, :, j]).astype(F32)).astype(F32)
        p = part.reshape(M, THREADS // WAVE, WAVE)
        lanes = np.arange(WAVE)
        for o in (32, 16, 8, 4, 2, 1):
            p = (p + p[:, :, lanes ^ o]).astype(F32)
        tot = p[:, 0, 0]
        for w in range(1, THREADS // WAVE):
            tot = (tot + p[:, w, 0]).astype(F32)
    return tot.astype(F32)


def head_sum_squares(v: np.ndarray) -> np.ndarray:
    """[M, N] (N % 128 == 0) -> [M, N/128]: per-head sum of v^2, each lane's 8 elements in order,
    then a 16-lane xor butterfly (8, 4, 2, 1)."""
    v = np.asarray(v, dtype=F32)
    M, N = v.shape
    h = v.reshape(M, N // HEAD, 16, 8)
    part = np.zeros((M, N // HEAD, 16), dtype=F32)
    with np.errstate(over="ignore", invalid="ignore"):
        for j in range(8):
            part = (part + (h[..., j] * h[..., j]).astype(F32)).astype(F32)
        lanes = np.arange(16)
        for o in (8, 4, 2, 1):
            part = (part + part[..., lanes ^ o]).astype(F32)
    return part[..., 0].astype(F32)


def inv_rms(ssq: np.ndarray, n: int, eps: float) -> np.ndarray:
    """1 / sqrt(ssq / n + eps), each step correctly rounded fp32."""
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        mean = (np.asarray(ssq, dtype=F32) / F32(n)).astype(F32)
        d = (mean + F32(eps)).astype(F32)
        return (F32(1) / np.sqrt(d).astype(F32)).astype(F32)


def add_rms_norm(y_bits, res_bits, w_bits, eps: float):
    """bf16 y, residual [M, K], weight [K] -> (normalized bf16 [M, K], residual_out bf16 [M, K])."""
    with np.errstate(over="ignore", invalid="ignore"):
        v = (O.bf16_to_f32(y_bits) + O.bf16_to_f32(res_bits)).astype(F32)
        inv = inv_rms(row_sum_squares(v), v.shape[1], eps)
        w1 = (O.bf16_to_f32(w_bits) + F32(1)).astype(F32)
        n = ((v * inv[:, None]).astype(F32) * w1[None, :]).astype(F32)
    return O.f32_to_bf16(n), O.f32_to_bf16(v)


def add_rms_quant(y_bits, res_bits, w_bits, eps: float):
    """-> (q uint8 [M, K], scale f32 [M], residual_out bf16 [M, K])."""
    n, r = add_rms_norm(y_bits, res_bits, w_bits, eps)
    q, s = O.quant_per_token(n)
    return q, s, r


def silu_mul(gu_bits):
    """bf16 [M, 2N] -> bf16 [M, N]: bf16(bf16(silu(gate)) * up)."""
    gu = np.asarray(gu_bits, dtype=np.uint16)
    N = gu.shape[1] // 2
    g, u = O.bf16_to_f32(gu[:, :N]), O.bf16_to_f32(gu[:, N:])
    t = O.bf16_to_f32(O.f32_to_bf16(silu_f32(g)))
    with np.errstate(over="ignore", invalid="ignore"):
        return O.f32_to_bf16((t * u).astype(F32))


def silu_mul_quant(gu_bits):
    """-> (q uint8 [M, N], scale f32 [M])."""
    return O.quant_per_token(silu_mul(gu_bits))


def gdn_norm(x_bits, z_bits, w_bits, eps: float):
    """bf16 x, z [M, N] (N % 128 == 0), weight [128] -> bf16 [M, N]."""
    x = O.bf16_to_f32(x_bits)
    M, N = x.shape
    inv = inv_rms(head_sum_squares(x), HEAD, eps)                  # [M, N/128]
    w = np.tile(O.bf16_to_f32(w_bits), N // HEAD)
    sg = silu_f32(O.bf16_to_f32(z_bits))
    with np.errstate(over="ignore", invalid="ignore"):
        a = (x.reshape(M, N // HEAD, HEAD) * inv[..., None]).astype(F32).reshape(M, N)
        n = (((a * w[None, :]).astype(F32)) * sg).astype(F32)
    return O.f32_to_bf16(n)


def gdn_norm_quant(x_bits, z_bits, w_bits, eps: float):
    """-> (q uint8 [M, N], scale f32 [M])."""
    return O.quant_per_token(gdn_norm(x_bits, z_bits, w_bits, eps))
