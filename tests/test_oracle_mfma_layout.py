"""The MFMA operand model (oracle/mfma_model.py) against the lane layout measured on an MI355X
(tests/golden/mfma_16x16x128_f4f8_layout.npz, written by tests/golden/gen_mfma_layout.py through the
library's w4a8_mfma_tile). CPU only: the fixture is data; the model must reproduce every pairing of
an fp8 B element with an fp4 A element, every scale lane and every result position."""
import os

import numpy as np
import pytest

from oracle import mfma_model as MM

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden",
                       "mfma_16x16x128_f4f8_layout.npz")


def model_layout():
    """The fixture's arrays as the model predicts them."""
    dr, dc = MM.d_lane_map()
    pos_row = dr.reshape(-1)                      # D position (lane * 4 + reg) -> row
    pos_col = dc.reshape(-1)
    a_row_pos = np.array([np.flatnonzero(pos_row == la % 16) for la in range(64)])
    b_col_pos = np.array([np.flatnonzero(pos_col == lb % 16) for lb in range(64)])
    bk, bc = MM.b_lane_map()
    meet = np.zeros((64, 32, 16), np.int64)
    sa_lane = np.zeros((64, 32, 16), np.int64)
    sb_lane = np.zeros((64, 32, 16), np.int64)
    ar, ak = MM.a_lane_map()
    for lb in range(64):
        for jb in range(32):
            k, c = bk[lb, jb], bc[lb, jb]
            for i, pos in enumerate(b_col_pos[lb]):
                r = pos_row[pos]
                la, j = np.argwhere((ar == r) & (ak == k))[0]
                meet[lb, jb, i] = 32 * la + j
                sa_lane[lb, jb, i] = 16 * (k // 32) + r
                sb_lane[lb, jb, i] = 16 * (k // 32) + c
    return dict(a_row_pos=a_row_pos, b_col_pos=b_col_pos, meet=meet, sa_lane=sa_lane,
                sb_lane=sb_lane)


@pytest.fixture(scope="module")
def measured():
    z = np.load(FIXTURE, allow_pickle=False)
    assert str(z["device"]).startswith("gfx950")
    return z


@pytest.fixture(scope="module")
def model():
    return model_layout()


@pytest.mark.parametrize("name", ["a_row_pos", "b_col_pos", "meet", "sa_lane", "sb_lane"])
def test_model_reproduces_measured_layout(measured, model, name):
    assert np.array_equal(measured[name].astype(np.int64), model[name].astype(np.int64)), name


def test_fp8_lane_holds_two_runs_of_16(measured):
    # byte 16 of every B lane meets the A element 64 k further than byte 0 (two A lanes on)
    meet = measured["meet"].astype(np.int64)
    a_lane = meet // 32
    assert np.all(a_lane[:, 16] - a_lane[:, 0] == 32)
    assert np.all(meet[:, 1:16] - meet[:, 0:1] == np.arange(1, 16)[None, :, None])
