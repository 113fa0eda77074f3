"""The fragment-tiled activation layout of the oracle (tile_q / untile_q / tiled_offset) pinned
against the scaled MFMA's fp8 operand lane map (oracle/mfma_model.py, which
tests/test_oracle_mfma_layout.py pins to the layout measured on MI355X), against its own inverse and
against its scalar offset. CPU only."""
import numpy as np
import pytest

from oracle import mfma_model as MM
from oracle import mxfp4_oracle as O


@pytest.mark.parametrize("M,K", [(1, 128), (16, 256), (17, 384), (45, 1024), (64, 5120)])
def test_round_trip(M, K):
    q = np.random.default_rng(M * 7 + K).integers(0, 256, (M, K), dtype=np.uint8)
    t = O.tile_q(q)
    assert t.size == -(-M // 16) * 16 * K
    assert np.array_equal(O.untile_q(t, M, K), q)


def test_padding_tokens_are_zero():
    q = np.full((18, 256), 0x38, np.uint8)
    t = O.tile_q(q)
    full = O.untile_q(t, 32, 256)
    assert np.all(full[:18] == 0x38) and np.all(full[18:] == 0)


def test_lanes_follow_the_mfma_fp8_operand():
    # block b, k-tile t: the 2 KiB fragment, read as the operand's 64 lanes x 32 bytes (half h of
    # lane l = bytes 16h .. 16h+15 of the lane), must hold q[16b + col, 128t + k] for the (k, col)
    # the MFMA assigns to that lane byte
    M, K = 40, 384
    q = np.random.default_rng(3).integers(0, 256, (M, K), dtype=np.uint8)
    t = O.tile_q(q).reshape(-1, K // 128, 2, 64, 16)
    bk, bc = MM.b_lane_map()
    qp = np.zeros((48, K), np.uint8)
    qp[:M] = q
    for b in range(3):
        for kt in range(K // 128):
            lanes = np.concatenate([t[b, kt, 0], t[b, kt, 1]], axis=1)   # [64, 32]
            want = qp[16 * b + bc, 128 * kt + bk]
            assert np.array_equal(lanes, want), (b, kt)


def test_scalar_offset_matches_array_form():
    M, K = 35, 512
    q = np.random.default_rng(5).integers(0, 256, (M, K), dtype=np.uint8)
    t = O.tile_q(q)
    rows, cols = np.meshgrid(np.arange(M), np.arange(K), indexing="ij")
    off = np.vectorize(lambda r, c: O.tiled_offset(int(r), int(c), K))(rows, cols)
    assert np.array_equal(t[off], q)
    assert len(np.unique(off)) == M * K


def test_k_must_be_whole_tiles():
    with pytest.raises(ValueError):
        O.tile_q(np.zeros((4, 96), np.uint8))
