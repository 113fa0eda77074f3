"""CPU oracle for the MXFP4 W4A8 linear path. TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import this module, and only as the reference their results are compared with. The product path
(``vllm_sly_radiance_amd``) never imports it and fails loudly when its HIP library is missing.

Everything here is plain numpy on the host. bf16 tensors are carried as their raw ``uint16`` bit
patterns and fp8 e4m3fn / e8m0 / packed e2m1 as ``uint8``, so no array ever depends on a torch
dtype. Each function cites the reference code it restates (paths relative to the reference repo).

Pins (what checks each function against something other than itself; see tests/test_oracle_*):
  e4m3fn_encode     torch's float8_e4m3fn cast (the library routine _traced_quant calls) over every
                    bf16 pattern, every e4m3 rounding midpoint +-1 ulp and 2M random floats;
                    hand-computed known answers (ties, 448 clamp edge, subnormals).
  e4m3fn_decode     closed form (sign, 4-bit exponent bias 7, 3-bit mantissa, 0x7F NaN) for all
                    256 codes; encode(decode(c)) == c.
  quant_per_token   torch restatement of _traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396) run
                    on the same inputs (torch is a library here, not the reference); closed-form
                    special cases (all-zero row -> 1/(448*512), amax 448 -> scale exactly 1.0).
  dequant_weight    the e2m1 value table from the OCP MX spec / sly/tests/test_kvq_reference.py
                    known answers (0x71 -> 0.5, 6.0; 0x0F -> -6.0); e8m0 = 2^(e-127).
  gemm_ref_f32      gemm_exact_f64, an exact integer-domain brute force, on small shapes.
  repack/unrepack   round trip, one-hot bijectivity, and the MFMA fragment model
                    (oracle/mfma_model.py) reproducing gemm_ref_f32 from the repacked bytes.
  tile_q/untile_q   round trip on ragged M; every byte against the fp8 operand lane map of the
  tiled_offset      MFMA model (itself pinned to the layout measured on MI355X); the scalar offset
                    against the array form at every element.
"""
from __future__ import annotations

import numpy as np

# --------------------------------------------------------------------------------------------
# Format tables
# --------------------------------------------------------------------------------------------
# e2m1 code -> value; bit 3 is the sign. Same table as _exact_ref's _E2M1
# (sly/mxfp4/radiance_mxfp4.py:515-516).
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                        -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=np.float32)

FP8_MAX = np.float32(448.0)
# fl32(1/448) and 1/(448*512): the constants of _traced_quant (sly/mxfp4/radiance_mxfp4.py:388-389).
# torch multiplies an fp32 tensor by a Python float in fp32, so the scalar is rounded to fp32 first.
INV_FP8_MAX = np.float32(1.0 / 448.0)
MIN_SCALE = np.float32(1.0 / (448.0 * 512.0))


# --------------------------------------------------------------------------------------------
# bf16 <-> f32 (bit patterns)
# --------------------------------------------------------------------------------------------
def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 patterns -> float32 (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> uint16 bf16 patterns, round to nearest even (torch's .to(torch.bfloat16)).

    NaN maps to a quiet NaN with the input's sign (0x7FC0 | sign)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = (u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16
    r = np.where(nan, ((u >> 16) & np.uint32(0x8000)) | np.uint32(0x7FC0), r)
    return r.astype(np.uint16)


def bf16_ulp(x: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |x| (float64): 2^(floor(log2|x|) - 7), floored at the smallest
    bf16 subnormal 2^-133."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, np.maximum(np.exp2(e - 7.0), 2.0 ** -133), 2.0 ** -133)


# --------------------------------------------------------------------------------------------
# fp8 e4m3fn (OCP, max 448, 0x7F/0xFF NaN, no infinities)
# --------------------------------------------------------------------------------------------
def e4m3fn_decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 (the `x_fp8.float()` of _exact_ref,
    sly/mxfp4/radiance_mxfp4.py:521)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 0x7
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    out = (sign * mag).astype(np.float32)
    return np.where((c & 0x7F) == 0x7F, np.float32(np.nan), out).astype(np.float32)


def e4m3fn_encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 e4m3fn, round to nearest even, with torch's out-of-range rule: anything
    that rounds past 448 (|x| > 464, and 464 < |x| < 480 by rounding) and NaN become the NaN code
    0x7F | sign. This is the `.to(torch.float8_e4m3fn)` of _traced_quant
    (sly/mxfp4/radiance_mxfp4.py:395); callers clamp to +-448 first, as the reference does."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    sign = ((u >> 24) & np.uint32(0x80)).astype(np.uint8)
    a = u & np.uint32(0x7FFFFFFF)
    af = a.view(np.float32)
    # normal range (|x| >= 2^-6): round the 23-bit mantissa to 3 bits, nearest even
    rn = (a + np.uint32(0x7FFFF) + ((a >> 20) & np.uint32(1))) >> 20
    normal = (rn - np.uint32((127 - 7) << 3)).astype(np.int64)
    # subnormal range (|x| < 2^-6): code = round_half_even(|x| * 2^9), exact in float64
    small = af < np.float32(2.0 ** -6)                  # False for NaN
    sub = np.rint(np.where(small, af, 0).astype(np.float64) * 512.0).astype(np.int64)
    mag = np.where(small, sub, normal)
    # rounding up into 0x7F (or beyond) yields NaN, as does a NaN/inf input
    mag = np.where((a >= np.uint32(0x7F800000)) | (mag >= 0x7F), 0x7F, mag)
    return (mag.astype(np.uint8) | sign).astype(np.uint8)


# --------------------------------------------------------------------------------------------
# Activation quantizer: dynamic per-token e4m3
# --------------------------------------------------------------------------------------------
def quant_per_token(x_bits: np.ndarray):
    """bf16 [M, K] (uint16 patterns) -> (q uint8 [M, K] e4m3fn, s float32 [M]).

    Restates _traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396) step for step, in fp32:
        s = max(amax(|x|) * fl32(1/448), 1/(448*512))      (NaN propagates)
        q = e4m3_rne(clamp(x / s, -448, 448))                (IEEE fp32 division)
    An all-zero row therefore gets s = fl32(1/229376) and q = +-0 (sign kept)."""
    xf = bf16_to_f32(x_bits)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        amax = np.max(np.abs(xf), axis=-1)                         # NaN-propagating
        s = (amax.astype(np.float32) * INV_FP8_MAX).astype(np.float32)
        s = np.where(np.isnan(s), s, np.maximum(s, MIN_SCALE)).astype(np.float32)
        v = (xf / s[:, None]).astype(np.float32)
        v = np.where(np.isnan(v), v, np.clip(v, -FP8_MAX, FP8_MAX)).astype(np.float32)
    return e4m3fn_encode(v), s


# --------------------------------------------------------------------------------------------
# MXFP4 weights: packed e2m1 [N, K/2] (low nibble = even k) + e8m0 [N, K/32]
# --------------------------------------------------------------------------------------------
def e8m0_to_f32(e: np.ndarray) -> np.ndarray:
    """e8m0 block exponent -> 2^(e-127) (`torch.pow(2.0, ws - 127)`,
    sly/mxfp4/radiance_mxfp4.py:525). 0xFF is NaN in the OCP MX spec; the reference's pow gives
    inf there. Neither occurs in checkpoints; parity tests keep e in [0, 254]."""
    e = np.asarray(e, dtype=np.float64)
    return np.where(e == 255, np.nan, np.exp2(e - 127.0)).astype(np.float32)


def unpack_e2m1(w: np.ndarray, K: int) -> np.ndarray:
    """[N, K/2] packed bytes -> [N, K] codes, low nibble first
    (`torch.stack([wc & 0x0F, (wc >> 4) & 0x0F], -1)`, sly/mxfp4/radiance_mxfp4.py:522)."""
    w = np.asarray(w, dtype=np.uint8)
    N = w.shape[0]
    return np.stack([w & 0x0F, w >> 4], axis=-1).reshape(N, K)


def dequant_weight(w: np.ndarray, ws: np.ndarray) -> np.ndarray:
    """float32 [N, K] = E2M1[codes] * 2^(ws - 127) repeated over each 32-element K block
    (sly/mxfp4/radiance_mxfp4.py:519-526). ws is the checkpoint's [N, K/32]."""
    N, K = w.shape[0], w.shape[1] * 2
    codes = unpack_e2m1(w, K)
    sc = np.repeat(e8m0_to_f32(ws), 32, axis=1)
    return (E2M1_VALUES[codes] * sc).astype(np.float32)


def gemm_ref_f32(q: np.ndarray, s: np.ndarray, w: np.ndarray, ws: np.ndarray,
                 chunk: int = 2048) -> np.ndarray:
    """float32 [M, N]: _exact_ref (sly/mxfp4/radiance_mxfp4.py:507-527).

        xr = q.float() * s[:, None]          (fp32)
        y  = xr @ Wdeq.T                     (fp32 matmul, chunked over N)

    The reference reads the scale as [K/32, N] after its load-time transpose
    (sly/mxfp4/radiance_mxfp4.py:1083-1084); this takes the checkpoint's [N, K/32] directly."""
    xr = (e4m3fn_decode(q) * np.asarray(s, dtype=np.float32)[:, None]).astype(np.float32)
    N = w.shape[0]
    out = np.empty((q.shape[0], N), dtype=np.float32)
    for a in range(0, N, chunk):
        b = min(a + chunk, N)
        out[:, a:b] = xr @ dequant_weight(w[a:b], ws[a:b]).T
    return out


def gemm_abs_terms(q: np.ndarray, s: np.ndarray, w: np.ndarray, ws: np.ndarray,
                   chunk: int = 2048) -> np.ndarray:
    """float64 [M, N] sum_k |xr[m,k] * Wdeq[n,k]|: the magnitude fp32 accumulation error scales
    with. Used only to size the accumulation-order allowance of the GEMM tolerance."""
    xr = np.abs(e4m3fn_decode(q).astype(np.float64) * np.asarray(s, np.float64)[:, None])
    N = w.shape[0]
    out = np.empty((q.shape[0], N), dtype=np.float64)
    for a in range(0, N, chunk):
        b = min(a + chunk, N)
        out[:, a:b] = xr @ np.abs(dequant_weight(w[a:b], ws[a:b]).astype(np.float64)).T
    return out


def gemm_exact_f64(q: np.ndarray, s: np.ndarray, w: np.ndarray, ws: np.ndarray) -> np.ndarray:
    """float64 [M, N]: s[m] * sum_k q[m,k] * Wdeq[n,k], the inner sum computed EXACTLY.

    Every term is a multiple of 2^-(9+1+(127-e_min)) and bounded by 448*6*2^(e_max-127), so for
    block exponents within [e_max-20, e_max] the sum fits float64's 53 bits and the float64 dot
    product is exact whatever the summation order; this function checks that condition and
    refuses otherwise. Brute force for small shapes only."""
    e = np.asarray(ws, dtype=np.int64)
    if e.size and (e.max() - e.min() > 20 or e.max() > 254):
        raise ValueError("gemm_exact_f64: exponent spread too wide for an exact float64 sum")
    K = w.shape[1] * 2
    if K > (1 << 16):
        raise ValueError("gemm_exact_f64: K too large for an exact float64 sum")
    qa = e4m3fn_decode(q).astype(np.float64)
    wd = dequant_weight(w, ws).astype(np.float64)
    return (qa @ wd.T) * np.asarray(s, np.float64)[:, None]


def linear_ref(x_bits: np.ndarray, w: np.ndarray, ws: np.ndarray):
    """The whole op: bf16 x [M, K] -> (bf16 y [M, N] as uint16, fp32 y, q, s).
    radiance::mxfp4_linear (sly/mxfp4/radiance_mxfp4.py:644-816) with _traced_quant as the
    activation quantizer, output rounded to bf16 (:737)."""
    q, s = quant_per_token(x_bits)
    y = gemm_ref_f32(q, s, w, ws)
    return f32_to_bf16(y), y, q, s


# --------------------------------------------------------------------------------------------
# The MI355X weight layout ("MFMA granules")
# --------------------------------------------------------------------------------------------
# One granule = one B operand of v_mfma_scale_f32_16x16x128_f8f6f4 with fp4 B: 16 output columns
# x 128 k = 64 lanes x 16 bytes. Lane l carries column n0 + (l % 16) and the 32-element MX block
# k0/32 + l/16, i.e. exactly 16 consecutive checkpoint bytes of one row, nibble order unchanged.
# Granules are stored [n-tile][k-tile][lane][16 B]. The e8m0 scale bytes ride in one dword per lane
# per group of four k-tiles: [n-tile][k-group][lane][4 B], byte j = k-tile 4*g + j.
# K is padded to a multiple of 512 (zero nibbles, scale 127) and N to a multiple of 16 (zero rows).
# This layout replaces the reference's load-time permute_w + psw_pack_w_ + psw_fold_ws + scale
# transpose (sly/mxfp4/radiance_mxfp4.py:181-226, :311-316, :1083-1171).
KT_ELEMS = 128          # k per granule
KG_TILES = 4            # k-tiles per scale dword
K_ALIGN = KT_ELEMS * KG_TILES
N_ALIGN = 16


def padded_dims(N: int, K: int):
    return -(-N // N_ALIGN) * N_ALIGN, -(-K // K_ALIGN) * K_ALIGN


def repack(w: np.ndarray, ws: np.ndarray):
    """checkpoint (w [N, K/2] u8, ws [N, K/32] u8) -> (wq [Np*Kp/2] u8, sq [Np*Kp/32] u8)."""
    w = np.asarray(w, dtype=np.uint8)
    ws = np.asarray(ws, dtype=np.uint8)
    N, K = w.shape[0], w.shape[1] * 2
    if K % 32 or ws.shape != (N, K // 32):
        raise ValueError(f"repack: w {w.shape} / ws {ws.shape} are not [N, K/2] / [N, K/32]")
    Np, Kp = padded_dims(N, K)
    wp = np.zeros((Np, Kp // 2), np.uint8)
    wp[:N, :K // 2] = w
    sp = np.full((Np, Kp // 32), 127, np.uint8)
    sp[:N, :K // 32] = ws
    NT, KT, KG = Np // 16, Kp // 128, Kp // 512
    # wp[n, kb*16 + b] with n = nt*16 + r, kb = kt*4 + h  ->  wq[nt, kt, h*16 + r, b]
    wq = wp.reshape(NT, 16, KT, 4, 16).transpose(0, 2, 3, 1, 4)
    # sp[n, kb] with kb = (g*4 + j)*4 + h  ->  sq[nt, g, h*16 + r, j]
    sq = sp.reshape(NT, 16, KG, 4, 4).transpose(0, 2, 4, 1, 3)
    return np.ascontiguousarray(wq).reshape(-1), np.ascontiguousarray(sq).reshape(-1)


def tile_q(q: np.ndarray) -> np.ndarray:
    """Row-major e4m3 codes q [M, K] (K % 128 == 0) -> the fragment-tiled bytes the producers
    write with q_layout 1 and the tile GEMM reads (flat, ceil(M/16)*16*K; padding tokens zero).
    Block b of 16 tokens, k-tile t, half h, lane l: 16 bytes = token 16b + l%16, k-bytes
    128t + 16(4h + l//16) .. +15, i.e. the scaled MFMA's fp8 operand order (mfma_model.b_lane_map)
    laid out lane after lane. The reference's tile() (sly/mxfp4/tile_layout.py:10-18) does the same
    for gfx1201's 16x16x16 WMMA fragments."""
    q = np.asarray(q, np.uint8)
    M, K = q.shape
    if K % 128:
        raise ValueError(f"tile_q: K={K} is not a multiple of 128")
    Mp = -(-M // 16) * 16
    p = np.zeros((Mp, K), np.uint8)
    p[:M] = q
    # p[16b + r, 128t + 64h + 16c + e] -> [b, t, h, c * 16 + r, e]
    t = p.reshape(Mp // 16, 16, K // 128, 2, 4, 16).transpose(0, 2, 3, 4, 1, 5)
    return np.ascontiguousarray(t).reshape(-1)


def untile_q(t: np.ndarray, M: int, K: int) -> np.ndarray:
    """Inverse of tile_q: flat fragment-tiled bytes -> row-major q [M, K] (padding dropped).
    Counterpart of the reference's untile() (sly/mxfp4/tile_layout.py:21-25)."""
    Mp = -(-M // 16) * 16
    r = np.asarray(t, np.uint8).reshape(-1)[:Mp * K].reshape(Mp // 16, K // 128, 2, 4, 16, 16)
    return np.ascontiguousarray(r.transpose(0, 4, 1, 2, 3, 5)).reshape(Mp, K)[:M].copy()


def tiled_offset(row: int, col: int, K: int) -> int:
    """Byte offset of q[row, col] in the fragment-tiled layout: the scalar form of the producers'
    store address (the reference's kernel_offset, sly/mxfp4/tile_layout.py:28-32, for its own
    layout)."""
    b, r, t, h, c, e = row >> 4, row & 15, col >> 7, (col >> 6) & 1, (col >> 4) & 3, col & 15
    return ((b * (K >> 7) + t) * 2 + h) * 1024 + 16 * (r + 16 * c) + e


def unrepack(wq: np.ndarray, sq: np.ndarray, N: int, K: int):
    """Inverse of repack: -> (w [N, K/2], ws [N, K/32]) with the padding dropped."""
    Np, Kp = padded_dims(N, K)
    NT, KT, KG = Np // 16, Kp // 128, Kp // 512
    wp = np.asarray(wq, np.uint8).reshape(NT, KT, 4, 16, 16).transpose(0, 3, 1, 2, 4)
    sp = np.asarray(sq, np.uint8).reshape(NT, KG, 4, 16, 4).transpose(0, 3, 1, 4, 2)
    wp = np.ascontiguousarray(wp).reshape(Np, Kp // 2)
    sp = np.ascontiguousarray(sp).reshape(Np, Kp // 32)
    return wp[:N, :K // 2].copy(), sp[:N, :K // 32].copy()
