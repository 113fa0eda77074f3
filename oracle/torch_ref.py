"""Torch (CPU) restatement of the reference's dequant-then-matmul path: the CPU baseline.

TEST INFRASTRUCTURE ONLY, like the rest of ``oracle/``: ``bench.py``'s ``cpu_baseline`` leg times
these functions on the host's cores, ``tests/test_oracle_torch_ref.py`` pins them against the numpy
oracle (``oracle/mxfp4_oracle.py``), and nothing in the product package imports them.

The three steps are timed separately by the bench, so each is its own function:
  quant_per_token  _traced_quant (sly/mxfp4/radiance_mxfp4.py:392-396): s = max(amax * fl32(1/448),
                   1/(448*512)), q = e4m3(clamp(x / s, +-448)); torch's own float8_e4m3fn cast.
  dequant_weight   _exact_ref's weight side (sly/mxfp4/radiance_mxfp4.py:515-526): e2m1 codes, low
                   nibble first, times 2^(e - 127) per 32-element block, fp32 [N, K].
  gemm             _exact_ref's product (sly/mxfp4/radiance_mxfp4.py:521-527): q.float() * s, then
                   one fp32 matmul against the dequantized weight, [M, N].
Tensors are torch CPU tensors: x bf16 [M, K], w uint8 [N, K/2], ws uint8 [N, K/32] (the
checkpoint's layout), q float8_e4m3fn [M, K], s float32 [M].
"""
from __future__ import annotations

import torch

# e2m1 code -> value, bit 3 the sign (_exact_ref's table, sly/mxfp4/radiance_mxfp4.py:515-516)
E2M1 = torch.tensor([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0,
                     -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0], dtype=torch.float32)


def quant_per_token(x: torch.Tensor):
    """bf16 [M, K] -> (float8_e4m3fn [M, K], float32 [M])."""
    xf = x.float()
    s = xf.abs().amax(dim=-1, keepdim=True) * (1.0 / 448.0)
    s = torch.clamp(s, min=1.0 / (448.0 * 512.0))
    q = torch.clamp(xf / s, -448.0, 448.0).to(torch.float8_e4m3fn)
    return q, s.squeeze(-1)


def dequant_weight(w: torch.Tensor, ws: torch.Tensor) -> torch.Tensor:
    """uint8 [N, K/2] codes + uint8 [N, K/32] e8m0 -> float32 [N, K]."""
    N = w.shape[0]
    codes = torch.stack([w & 0x0F, w >> 4], dim=-1).reshape(N, -1).long()
    vals = E2M1[codes].view(N, -1, 32)
    scale = torch.pow(2.0, ws.float() - 127.0).unsqueeze(-1)
    return (vals * scale).reshape(N, -1)


def gemm(q: torch.Tensor, s: torch.Tensor, wdeq: torch.Tensor) -> torch.Tensor:
    """float8 [M, K], float32 [M], float32 [N, K] -> float32 [M, N]."""
    return (q.float() * s[:, None]) @ wdeq.T
