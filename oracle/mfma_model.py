"""Host model of the gfx950 scaled MFMA operand layout. TEST INFRASTRUCTURE ONLY.

Models v_mfma_scale_f32_16x16x128_f8f6f4 as the GEMM kernels issue it: the A operand is the fp4
e2m1 weight granule (cbsz 4) with its e8m0 block scales, the B operand is the fp8 e4m3 activation
fragment (blgp 0) with scale byte 127, and the result is D = W_tile . A_tile^T (16 n x 16 m):

  A (16 x 128, fp4): lane l holds row l % 16, k = 32*(l // 16) + j in nibble j of its 16 bytes
                     (low nibble = even j, byte j // 2): one whole 32-element block per lane.
  B (128 x 16, fp8): lane l holds column l % 16 and two 16-element runs of k:
                     byte j < 16 -> k = 16*(l // 16) + j, byte j >= 16 -> k = 64 + 16*(l // 16) + j - 16.
  Scales:            the scale byte of lane l covers row (A) / column (B) l % 16 and the k-block
                     l // 16 (k in [32*(l // 16), 32*(l // 16) + 32)), for both operands; so an fp8
                     B lane's two runs take their scales from two other lanes.
  D (16 x 16):       lane l, register i holds D[4*(l // 16) + i][l % 16].

These maps were measured on MI355X with one-hot operands (every A nibble x every B byte, plus
bit-coded scale patterns) and are re-checked on every GPU test run by
tests/test_gpu_kernels.py::test_mfma_model_matches_hardware_tiles, which runs raw tiles through the
library's w4a8_mfma_tile diagnostic. Used two ways: (1) on the CPU, gemm_via_granules() consumes the
repacked weight bytes through this model and must reproduce the exact GEMM, which pins the repack
to the model; (2) the GPU test pins the model to the hardware. This describes the MI355X
instruction that replaces the reference's gfx1201 WMMA fragment (empirically confirmed there too,
sly/mxfp4/radiance_mxfp4_fp8.hip:24-25) plus its e2m1->e4m3 fold (:44-86).
"""
from __future__ import annotations

import numpy as np

from .mxfp4_oracle import E2M1_VALUES, e4m3fn_decode, padded_dims


def a_lane_map():
    """(row, k) of each (lane, element) of the fp4 A operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    return np.broadcast_to(lane % 16, (64, 32)), 32 * (lane // 16) + j


def b_lane_map():
    """(k, col) of each (lane, byte) of the fp8 B operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    k = 16 * (lane // 16) + np.where(j < 16, j, 64 + j - 16)
    return k, np.broadcast_to(lane % 16, (64, 32))


def d_lane_map():
    """(row, col) of each (lane, register) of the 16x16 result: two int arrays [64, 4]."""
    lane = np.arange(64)[:, None]
    i = np.arange(4)[None, :]
    return 4 * (lane // 16) + i, np.broadcast_to(lane % 16, (64, 4))


def scale_grid(scales):
    """[64] per-lane e8m0 bytes -> [16, 4] float64 factors: [row or column, k-block]."""
    s = np.asarray(scales, np.float64).reshape(4, 16).T         # lane = idx + 16 * block
    return np.exp2(s - 127.0)


def fp4_lane_values(lanes):
    """[64, 16] packed e2m1 bytes -> [64, 32] float64 element values (unscaled)."""
    lanes = np.asarray(lanes, np.uint8)
    nib = np.stack([lanes & 15, lanes >> 4], -1).reshape(64, 32)
    return E2M1_VALUES[nib].astype(np.float64)


def fp8_lane_values(lanes):
    """[64, 32] e4m3 bytes -> [64, 32] float64 element values (unscaled)."""
    return e4m3fn_decode(np.asarray(lanes, np.uint8)).astype(np.float64)


def mfma_tile(a_vals, b_vals, a_scales=None, b_scales=None):
    """One MFMA, exact: D[r, c] = sum_k A[r, k] sa[r, k/32] B[k, c] sb[c, k/32]  ([16, 16]).
    a_vals / b_vals are decoded lane values (float64 [64, 32]); scales are per-lane e8m0 bytes
    (default 127 = 1.0)."""
    A = np.zeros((16, 128))
    B = np.zeros((128, 16))
    ar, ak = a_lane_map()
    A[ar, ak] = a_vals
    bk, bc = b_lane_map()
    B[bk, bc] = b_vals
    if a_scales is not None:
        A = A * np.repeat(scale_grid(a_scales), 32, axis=1)
    if b_scales is not None:
        B = B * np.repeat(scale_grid(b_scales), 32, axis=1).T
    return A @ B


def mfma_tiles_batch(a_bytes, b_bytes, a_scales, b_scales):
    """Batched mfma_tile on raw lane bytes: a_bytes [T, 64, 16] (fp4), b_bytes [T, 64, 32] (fp8),
    scales [T, 64] e8m0 -> (D lanes [T, 64, 4], sum of |terms| lanes [T, 64, 4]), float64."""
    a_bytes = np.asarray(a_bytes, np.uint8)
    T = a_bytes.shape[0]
    nib = np.stack([a_bytes & 15, a_bytes >> 4], -1).reshape(T, 64, 32)
    av = E2M1_VALUES[nib].astype(np.float64)
    bv = e4m3fn_decode(np.asarray(b_bytes, np.uint8)).astype(np.float64)
    A = np.zeros((T, 16, 128))
    B = np.zeros((T, 128, 16))
    ar, ak = a_lane_map()
    bk, bc = b_lane_map()
    A[:, ar, ak] = av
    B[:, bk, bc] = bv
    sa = np.exp2(np.asarray(a_scales, np.float64).reshape(T, 4, 16).transpose(0, 2, 1) - 127.0)
    sb = np.exp2(np.asarray(b_scales, np.float64).reshape(T, 4, 16).transpose(0, 2, 1) - 127.0)
    A = A * np.repeat(sa, 32, axis=2)
    B = B * np.repeat(sb, 32, axis=2).transpose(0, 2, 1)
    r, c = d_lane_map()
    D = (A @ B)[:, r, c]
    Dabs = (np.abs(A) @ np.abs(B))[:, r, c]
    return D, Dabs


def d_to_lanes(D):
    """[16, 16] result -> [64, 4] per-lane registers."""
    r, c = d_lane_map()
    return np.asarray(D)[r, c]


def gemm_via_granules(q, s, wq, sq, M: int, N: int, K: int):
    """float64 [M, N]: the GEMM computed granule by granule from the repacked weight bytes
    (wq, sq), one modeled MFMA per (n-tile, m-tile, k-tile) with D = W_tile . A_tile^T, activation
    rows/k beyond M/K zero-filled and the per-token scale s applied at the end, as the kernels do."""
    Np, Kp = padded_dims(N, K)
    NT, KT, KG = Np // 16, Kp // 128, Kp // 512
    MT = -(-M // 16)
    qa = np.zeros((MT * 16, Kp), np.uint8)
    qa[:M, :K] = q
    wq = np.asarray(wq, np.uint8).reshape(NT, KT, 64, 16)
    sq = np.asarray(sq, np.uint8).reshape(NT, KG, 64, 4)
    bk, bc = b_lane_map()
    out = np.zeros((Np, MT * 16))
    for kt in range(KT):
        for mt in range(MT):
            b_vals = fp8_lane_values(qa[mt * 16 + bc, kt * 128 + bk])
            for nt in range(NT):
                a_vals = fp4_lane_values(wq[nt, kt])
                out[nt * 16:(nt + 1) * 16, mt * 16:(mt + 1) * 16] += mfma_tile(
                    a_vals, b_vals, sq[nt, kt // 4, :, kt % 4])
    return out[:N, :M].T * np.asarray(s, np.float64)[:, None]
