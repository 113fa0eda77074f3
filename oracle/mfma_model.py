"""Host model of the gfx950 scaled MFMA operand layout. TEST INFRASTRUCTURE ONLY.

Models v_mfma_scale_f32_16x16x128_f8f6f4 as the GEMM kernels issue it: the A operand is the fp4
e2m1 weight granule (cbsz 4) with its e8m0 block scales, the B operand is the fp8 e4m3 activation
fragment (blgp 0) with scale byte 127, and the result is D = W_tile . A_tile^T (16 n x 16 m):

  A (16 x 128): lane l holds row l % 16, k = 32*(l // 16) + j in nibble j of its 16 bytes
                (low nibble = even j, byte j // 2); scale byte of lane l covers that 32-block.
  B (128 x 16): lane l holds column l % 16, k = 32*(l // 16) + j in byte j of its 32 bytes;
                scale byte of lane l covers that 32-block.
  D (16 x 16):  lane l, register i holds D[4*(l // 16) + i][l % 16].

Used two ways: (1) on the CPU, gemm_via_granules() consumes the repacked weight bytes through this
model and must reproduce the exact GEMM, which pins the repack to the model; (2) the GPU probe test
builds one-hot operands from the same lane maps and checks the hardware against mfma_tile(), which
pins the model to the hardware. This describes the MI355X instruction that replaces the
reference's gfx1201 WMMA plus e2m1->e4m3 fold (sly/mxfp4/radiance_mxfp4_fp8.hip:24-25, :44-86).
"""
from __future__ import annotations

import numpy as np

from .mxfp4_oracle import E2M1_VALUES, e4m3fn_decode, padded_dims


def a_lane_map():
    """(row, k) of each (lane, element) of the A operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    return np.broadcast_to(lane % 16, (64, 32)), 32 * (lane // 16) + j


def b_lane_map():
    """(k, col) of each (lane, element) of the B operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    return 32 * (lane // 16) + j, np.broadcast_to(lane % 16, (64, 32))


def d_lane_map():
    """(row, col) of each (lane, register) of the 16x16 result: two int arrays [64, 4]."""
    lane = np.arange(64)[:, None]
    i = np.arange(4)[None, :]
    return 4 * (lane // 16) + i, np.broadcast_to(lane % 16, (64, 4))


def fp4_lane_values(lanes, scales):
    """[64, 16] packed e2m1 bytes + [64] e8m0 -> [64, 32] float64 element values."""
    lanes = np.asarray(lanes, np.uint8)
    nib = np.stack([lanes & 15, lanes >> 4], -1).reshape(64, 32)
    return E2M1_VALUES[nib].astype(np.float64) * np.exp2(
        np.asarray(scales, np.float64)[:, None] - 127.0)


def fp8_lane_values(lanes, scales):
    """[64, 32] e4m3 bytes + [64] e8m0 -> [64, 32] float64 element values."""
    return e4m3fn_decode(np.asarray(lanes, np.uint8)).astype(np.float64) * np.exp2(
        np.asarray(scales, np.float64)[:, None] - 127.0)


def mfma_tile(a_vals, b_vals):
    """One MFMA from decoded lane values (float64 [64, 32] each), exact: D = A @ B, [16, 16]."""
    A = np.zeros((16, 128))
    B = np.zeros((128, 16))
    ar, ak = a_lane_map()
    A[ar, ak] = a_vals
    bk, bc = b_lane_map()
    B[bk, bc] = b_vals
    return A @ B


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
    unit = np.full(64, 127, np.uint8)
    out = np.zeros((Np, MT * 16))
    for kt in range(KT):
        for mt in range(MT):
            b_vals = fp8_lane_values(qa[mt * 16 + bc, kt * 128 + bk], unit)
            for nt in range(NT):
                a_vals = fp4_lane_values(wq[nt, kt], sq[nt, kt // 4, :, kt % 4])
                out[nt * 16:(nt + 1) * 16, mt * 16:(mt + 1) * 16] += mfma_tile(a_vals, b_vals)
    return out[:N, :M].T * np.asarray(s, np.float64)[:, None]
