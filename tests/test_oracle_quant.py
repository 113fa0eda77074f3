"""Pins of the oracle's per-token quantizer (CPU).

quant_per_token restates _traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396) in numpy with its own
e4m3 encoder. It is checked against that expression evaluated by torch's own kernels (amax, fp32
scalar multiply, clamp, IEEE division, float8 cast) and against closed-form special cases."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from vllm_sly_radiance_amd import synthetic


def torch_traced_quant(x_bits: np.ndarray):
    """_traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396) evaluated by torch's CPU kernels."""
    x = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16)
    xf = x.to(torch.float32)
    s = (xf.abs().amax(-1, keepdim=True) * (1.0 / 448.0)).clamp_min(1.0 / (448.0 * 512.0))
    q = (xf / s).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q.view(torch.uint8).numpy(), s.reshape(-1).numpy()


@pytest.mark.parametrize("M,K,seed", [(8, 5120, 0), (1, 128, 1), (37, 1000, 2), (256, 2048, 3)])
def test_quant_matches_torch_expression(M, K, seed):
    x = synthetic.activations(M, K, seed)
    q, s = O.quant_per_token(x)
    tq, ts = torch_traced_quant(x)
    assert np.array_equal(q, tq)
    assert np.array_equal(s.view(np.uint32), ts.view(np.uint32))


def test_quant_special_rows_match_torch():
    K = 256
    rows = np.zeros((8, K), np.float32)
    rows[1, :] = 0.0                                     # all zero
    rows[2, 7] = -0.0
    rows[3, :] = np.linspace(-1e-30, 1e-30, K)           # tiny: min-scale clamp
    rows[4, :] = np.linspace(-3e38, 3e38, K)             # huge amax
    rows[5, 3] = np.inf
    rows[6, 9] = np.nan
    rows[7, :] = 448.0                                   # amax exactly 448
    x = O.f32_to_bf16(rows)
    q, s = O.quant_per_token(x)
    tq, ts = torch_traced_quant(x)
    assert np.array_equal(np.isnan(s), np.isnan(ts))
    fin = ~np.isnan(s)
    assert np.array_equal(s[fin].view(np.uint32), ts[fin].view(np.uint32))
    # NaN codes: the sign of a NaN produced by arithmetic is not specified by IEEE 754
    canon = lambda c: np.where((c & 0x7F) == 0x7F, 0x7F, c)
    assert np.array_equal(canon(q), canon(tq))


def test_zero_row_takes_min_scale():
    q, s = O.quant_per_token(np.zeros((2, 64), np.uint16))
    assert s[0] == np.float32(1.0 / 229376.0) and not q.any()


def test_negative_zero_keeps_sign():
    x = np.zeros((1, 64), np.uint16)
    x[0, 5] = 0x8000
    q, _ = O.quant_per_token(x)
    assert q[0, 5] == 0x80 and q[0, 4] == 0


def test_amax_448_gives_unit_scale_and_identity_codes():
    # fl32(448 * fl32(1/448)) == 1.0, so every bf16 value that is an e4m3 value or a tie between two
    # of them is quantized exactly as the e4m3 cast of itself; ties go to the even code.
    assert np.float32(448.0) * O.INV_FP8_MAX == np.float32(1.0)
    pos = O.e4m3fn_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    vals = np.concatenate([pos, (pos[:-1] + pos[1:]) / 2]).astype(np.float32)
    vals = vals[O.f32_to_bf16(vals).astype(np.uint32) << 16 == vals.view(np.uint32)]  # bf16-exact
    row = np.concatenate([[448.0], vals, -vals]).astype(np.float32)
    q, s = O.quant_per_token(O.f32_to_bf16(row)[None, :])
    assert s[0] == 1.0
    assert np.array_equal(q[0], O.e4m3fn_encode(row))
    # the tie between 0.5 (0x30) and 0.5625 (0x31) goes to the even code 0x30
    assert O.e4m3fn_encode(np.float32([0.53125]))[0] == 0x30


def test_outlier_row_max_maps_to_448():
    x = synthetic.activations(64, 4096, 7)
    q, s = O.quant_per_token(x)
    xf = O.bf16_to_f32(x)
    amax_idx = np.argmax(np.abs(xf), axis=1)
    assert np.all(q[np.arange(64), amax_idx] & 0x7F == 0x7E)
    assert np.all(s == (np.max(np.abs(xf), 1) * O.INV_FP8_MAX).astype(np.float32))


def test_power_of_two_row_scaling_is_exact():
    # Scaling a row by 2^k scales s by exactly 2^k and leaves every code unchanged (no clamps hit).
    x = synthetic.activations(4, 512, 9)
    xf = O.bf16_to_f32(x)
    for k in (-3, 5):
        x2 = O.f32_to_bf16(xf * np.float32(2.0 ** k))
        q1, s1 = O.quant_per_token(x)
        q2, s2 = O.quant_per_token(x2)
        assert np.array_equal(q1, q2) and np.array_equal(s2, s1 * np.float32(2.0 ** k))
