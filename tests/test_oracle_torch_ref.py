"""Pins of the torch CPU baseline (oracle/torch_ref.py) against the numpy oracle: the quantizer's
codes and scales bit for bit (synthetic rows and the special rows), the dequantized weight exactly,
and the fp32 GEMM within fp32 accumulation of the exact (float64) result."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from oracle import torch_ref as T
from vllm_sly_radiance_amd import synthetic


def bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


@pytest.mark.parametrize("M,K", [(8, 5120), (3, 640), (17, 96)])
def test_quant_matches_the_oracle(M, K):
    x = synthetic.activations(M, K, seed=M + K)
    q, s = T.quant_per_token(bf16(x))
    oq, os_ = O.quant_per_token(x)
    assert np.array_equal(q.view(torch.uint8).numpy(), oq)
    assert np.array_equal(s.numpy().view(np.uint32), os_.view(np.uint32))


def test_quant_special_rows():
    K = 64
    rows = np.zeros((5, K), np.float32)
    rows[1, 3] = 448.0                                   # scale exactly 1.0
    rows[2] = np.linspace(-1e4, 1e4, K)
    rows[3, 7] = np.nan
    rows[4, :] = -0.0
    x = O.f32_to_bf16(rows)
    q, s = T.quant_per_token(bf16(x))
    oq, os_ = O.quant_per_token(x)
    qb = q.view(torch.uint8).numpy()
    assert np.array_equal(np.where((qb & 0x7F) == 0x7F, 0x7F, qb), np.where((oq & 0x7F) == 0x7F,
                                                                            0x7F, oq))
    sn = s.numpy()
    assert np.array_equal(np.isnan(sn), np.isnan(os_))
    ok = ~np.isnan(sn)
    assert np.array_equal(sn[ok].view(np.uint32), os_[ok].view(np.uint32))
    assert sn[1] == 1.0 and sn[0] == np.float32(1.0 / 229376.0)


@pytest.mark.parametrize("N,K", [(48, 512), (5, 96)])
def test_dequant_matches_the_oracle(N, K):
    w, ws = synthetic.weights(N, K, seed=N * K)
    got = T.dequant_weight(torch.from_numpy(w), torch.from_numpy(ws)).numpy()
    assert np.array_equal(got, O.dequant_weight(w, ws))


def test_dequant_known_answers():
    # 0x71: low nibble 1 (0.5) at the even k, high nibble 7 (6.0) at the odd k; 0x0F: -6.0
    w = np.zeros((1, 16), np.uint8)
    w[0, 0], w[0, 1] = 0x71, 0x0F
    ws = np.full((1, 1), 126, np.uint8)                  # 2^-1
    got = T.dequant_weight(torch.from_numpy(w), torch.from_numpy(ws)).numpy()[0]
    assert got[0] == 0.25 and got[1] == 3.0 and got[2] == -3.0 and got[3] == 0.0


@pytest.mark.parametrize("M,N,K", [(8, 64, 512), (1, 16, 32), (17, 33, 640)])
def test_gemm_within_fp32_accumulation_of_the_exact_result(M, N, K):
    x = synthetic.activations(M, K, seed=M * 5 + K)
    w, ws = synthetic.weights(N, K, seed=N + K)
    q, s = T.quant_per_token(bf16(x))
    y = T.gemm(q, s, T.dequant_weight(torch.from_numpy(w), torch.from_numpy(ws))).numpy()
    oq, os_ = O.quant_per_token(x)
    exact = O.gemm_exact_f64(oq, os_, w, ws)
    terms = O.gemm_abs_terms(oq, os_, w, ws)
    assert np.all(np.abs(y.astype(np.float64) - exact) <= K * 2.0 ** -24 * terms + 1e-30)
