"""GPU parity of the decode-band kernel (weight waves + activation waves, 16 < M <= 64) against the
oracle, through the C ABI: every variant that serves each shape, unsplit and with K split over
grid rows, at the Qwen3.8-27B linear shapes and ragged ones (N not a multiple of the n-tiles a
workgroup holds, few k-tiles per weight wave, M one past a fragment). The kernel's hand-over
between waves is checked for determinism (the same bits on repeated calls) and for its failure
mark (a NaN anywhere would fail the oracle comparison)."""
import functools

import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from tests._check import assert_gemm_close, host_u16, stream, to_dev
from vllm_sly_radiance_amd import _native, synthetic

pytestmark = pytest.mark.gpu

BAND = _native.KERNEL_BAND


@pytest.fixture(scope="module")
def scratch(gpu_lib):
    """Registered scratch for the split forms (up to 4 splits of M = 64, N = 17408), the plugin's
    own registration put back afterwards."""
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    part = torch.empty(4 * 64 * 17408, dtype=torch.float32, device="cuda")
    cnt = torch.zeros(4096, dtype=torch.int32, device="cuda")
    _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)
    yield part, cnt
    torch.cuda.synchronize()
    p, c = R._scratch
    if p is None:
        _native.set_scratch(None, 0, None, 0)
    else:
        _native.set_scratch(p.data_ptr(), p.numel() * 4, c.data_ptr(), c.numel() * 4)


@functools.lru_cache(maxsize=2)
def layer(N, K):
    w, ws = synthetic.weights(N, K, seed=N + 5 * K)
    wb, sb = _native.packed_bytes(N, K)
    wq = torch.empty(wb, dtype=torch.uint8, device="cuda")
    sq = torch.empty(sb, dtype=torch.uint8, device="cuda")
    wd, sd = to_dev(w), to_dev(ws)
    _native.repack(wd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, stream())
    torch.cuda.synchronize()
    return w, ws, wq, sq


def run(q, s, wq, sq, N, K, variant, split):
    M = q.shape[0]
    qd, sd = to_dev(q), to_dev(s)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream(), BAND, variant, split)
    torch.cuda.synchronize()
    return host_u16(out)


def serving(M, N, K, split):
    """The band variants that serve (M, N, K, split) (the shape checks of a forced plan)."""
    return [v for v in range(_native.lib().w4a8_variant_count(BAND))
            if _native.variant_serves(BAND, v, M, N, K, split)]


SHAPES = [(17408, 5120), (5120, 8704), (10240, 5120), (5120, 6144), (1040, 2560), (528, 640)]


@pytest.mark.parametrize("M", [17, 32, 33, 48, 64])
@pytest.mark.parametrize("N,K", SHAPES)
def test_band_every_variant(scratch, N, K, M):
    w, ws, wq, sq = layer(N, K)
    x = synthetic.activations(M, K, seed=13 * M + K)
    q, s = O.quant_per_token(x)
    ran = 0
    for split in (1, 2, 3):
        for v in serving(M, N, K, split):
            print(f"[band] N={N} K={K} M={M} variant {v} {_native.variants(BAND)[v]} split {split}",
                  flush=True)
            out = run(q, s, wq, sq, N, K, v, split)
            assert_gemm_close(out, q, s, w, ws, f"band v{v} M={M} N={N} K={K} split {split}")
            ran += 1
    assert ran > 0, "no band variant serves this shape"


def test_band_is_deterministic(scratch):
    """Repeated calls give the same bits (the wave hand-over is ordered; the partial sums are
    added in a fixed order), unsplit and split."""
    M = 64
    for N, K, split in ((17408, 5120, 1), (5120, 8704, 3)):
        w, ws, wq, sq = layer(N, K)
        q, s = O.quant_per_token(synthetic.activations(M, K, seed=3))
        v = serving(M, N, K, split)[0]
        first = run(q, s, wq, sq, N, K, v, split)
        for _ in range(3):
            assert np.array_equal(run(q, s, wq, sq, N, K, v, split), first)


def test_band_refuses_what_it_cannot_serve(gpu_lib):
    """M past the variant's fragments, K not a multiple of 128, more splits than k-tiles per
    weight wave allow: refused before any launch."""
    p = 1 << 20
    lib = _native.lib()
    v = [i for i, c in enumerate(_native.variants(BAND)) if c[0] == 2][0]        # MF = 2
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 33, 5120, 5120, BAND, v, 1, None) == 1
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 5120, 5120 + 32, BAND, v, 1, None) == 1
    assert lib.w4a8_gemm_planned(p, p, p, p, p, 32, 5120, 640, BAND, v, 3, None) == 1
