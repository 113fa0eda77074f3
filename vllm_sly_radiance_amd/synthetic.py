"""Seeded synthetic operands with the distributions the MXFP4 W4A8 benchmarks are quoted on.

  activations  bf16 ~ N(0, 1); each entry independently (p = 1e-3) multiplied by 20
  weights      uniform random bytes = uniform e2m1 codes, two per byte, low nibble = even k
  scales       e8m0 exponents uniform in [119, 125] (2^-8 .. 2^-2), checkpoint layout [N, K/32]

The reference draws its random weights with torch.randint over bytes and exponents
(sly/mxfp4/bench_decode_cells.py:77-81); the distributions here are the ones the benchmark
configurations name. Everything is numpy on the host and returned as raw bit patterns
(bf16 as uint16), so the same seed gives the same bytes on any machine.
"""
from __future__ import annotations

import numpy as np

SCALE_LO, SCALE_HI = 119, 125
OUTLIER_P, OUTLIER_MUL = 1e-3, 20.0


def _bf16_bits(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)


def activations(M: int, K: int, seed: int) -> np.ndarray:
    """bf16 [M, K] as uint16 bit patterns."""
    g = np.random.default_rng(seed)
    x = g.standard_normal((M, K), dtype=np.float32)
    x = np.where(g.random((M, K)) < OUTLIER_P, x * np.float32(OUTLIER_MUL), x)
    return _bf16_bits(x)


def weights(N: int, K: int, seed: int):
    """(w uint8 [N, K/2], ws uint8 [N, K/32]) in the checkpoint layout."""
    if K % 32:
        raise ValueError(f"K={K} is not a multiple of the 32-element MX block")
    g = np.random.default_rng(seed)
    w = g.integers(0, 256, (N, K // 2), dtype=np.uint8)
    ws = g.integers(SCALE_LO, SCALE_HI + 1, (N, K // 32), dtype=np.uint8)
    return w, ws
