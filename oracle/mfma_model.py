"""Host model of the gfx950 scaled MFMA operand layout. TEST INFRASTRUCTURE ONLY.

Models v_mfma_scale_f32_16x16x128_f8f6f4 with an fp8 e4m3 A operand (cbsz 0) and an fp4 e2m1
B operand (blgp 4), as the GEMM kernels use it:

  A (16 x 128): lane l holds row l % 16, k = 32*(l // 16) + j in byte j of its 32 bytes.
  B (128 x 16): lane l holds column l % 16, k = 32*(l // 16) + j in nibble j of its 16 bytes
                (low nibble = even j, byte j // 2).
  scales:       lane l's e8m0 byte scales A[l % 16, 32*(l//16) : +32] (for A) and
                B[32*(l//16) : +32, l % 16] (for B).
  D (16 x 16):  lane l, register i holds D[4*(l // 16) + i][l % 16].

Used two ways: (1) on the CPU, gemm_via_granules() consumes the repacked weight bytes through this
model and must reproduce the dequant oracle, which pins the repack to the model; (2) the GPU probe
test builds one-hot operands from the same lane map and checks the hardware against mfma_tile(),
which pins the model to the hardware. Nothing here is part of the reference; it describes the
MI355X instruction the reference's gfx1201 WMMA fold (sly/mxfp4/radiance_mxfp4_fp8.hip:24-25,
:44-86) is replaced by.
"""
from __future__ import annotations

import numpy as np

from .mxfp4_oracle import E2M1_VALUES, e4m3fn_decode, padded_dims


def a_lane_map():
    """(row, k) of each (lane, byte) of the A operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    return np.broadcast_to(lane % 16, (64, 32)), 32 * (lane // 16) + j


def b_lane_map():
    """(k, col) of each (lane, nibble) of the B operand: two int arrays [64, 32]."""
    lane = np.arange(64)[:, None]
    j = np.arange(32)[None, :]
    return 32 * (lane // 16) + j, np.broadcast_to(lane % 16, (64, 32))


def d_lane_map():
    """(row, col) of each (lane, register) of the 16x16 result: two int arrays [64, 4]."""
    lane = np.arange(64)[:, None]
    i = np.arange(4)[None, :]
    return 4 * (lane // 16) + i, np.broadcast_to(lane % 16, (64, 4))


def mfma_tile(a_lanes, b_lanes, sa, sb):
    """One scaled MFMA, exact in float64. a_lanes [64, 32] u8 (e4m3), b_lanes [64, 16] u8 (packed
    e2m1), sa/sb [64] u8 (e8m0). Returns D as a [16, 16] float64 matrix."""
    a_lanes = np.asarray(a_lanes, np.uint8)
    b_lanes = np.asarray(b_lanes, np.uint8)
    A = np.zeros((16, 128))
    B = np.zeros((128, 16))
    ar, ak = a_lane_map()
    A[ar, ak] = e4m3fn_decode(a_lanes).astype(np.float64) * np.exp2(
        np.asarray(sa, np.float64)[:, None] - 127.0)
    nib = np.stack([b_lanes & 15, b_lanes >> 4], -1).reshape(64, 32)
    bk, bc = b_lane_map()
    B[bk, bc] = E2M1_VALUES[nib].astype(np.float64) * np.exp2(
        np.asarray(sb, np.float64)[:, None] - 127.0)
    return A @ B


def d_to_lanes(D):
    """[16, 16] result -> [64, 4] per-lane registers."""
    r, c = d_lane_map()
    return np.asarray(D)[r, c]


def gemm_via_granules(q, s, wq, sq, M: int, N: int, K: int):
    """float64 [M, N]: the GEMM computed granule by granule from the repacked weight bytes
    (wq, sq), one modeled MFMA per (m-tile, n-tile, k-tile), A rows/k beyond M/K zero-filled and
    the per-token scale s applied at the end, as the kernels do."""
    Np, Kp = padded_dims(N, K)
    NT, KT, KG = Np // 16, Kp // 128, Kp // 512
    MT = -(-M // 16)
    qa = np.zeros((MT * 16, Kp), np.uint8)
    qa[:M, :K] = q
    wq = np.asarray(wq, np.uint8).reshape(NT, KT, 64, 16)
    sq = np.asarray(sq, np.uint8).reshape(NT, KG, 64, 4)
    ar, ak = a_lane_map()
    out = np.zeros((MT * 16, Np))
    for mt in range(MT):
        for kt in range(KT):
            a_lanes = qa[mt * 16 + ar, kt * 128 + ak]
            for nt in range(NT):
                sb = sq[nt, kt // 4, :, kt % 4]
                out[mt * 16:(mt + 1) * 16, nt * 16:(nt + 1) * 16] += mfma_tile(
                    a_lanes, wq[nt, kt], np.full(64, 127, np.uint8), sb)
    return out[:M, :N] * np.asarray(s, np.float64)[:, None]
