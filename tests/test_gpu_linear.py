"""The whole linear in one launch (w4a8_linear at M <= 2, and M <= 4 on the wider shapes: waves
of the streaming GEMM's workgroups quantize the rows into LDS while the others stream the weights)
against the quantizer and the GEMM run separately, bit for bit, and against the oracle. Covers M
from 1 to 8 (one launch where it pays, two launches above), the four linear shapes of the
benchmark model and smaller ones, strided rows, special rows (zero, NaN, inf, the largest bf16,
subnormals) and the cases that fall back to two launches."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from tests._check import assert_gemm_close, bf16_dev, host_u16, stream, to_dev
from vllm_sly_radiance_amd import _native, synthetic

pytestmark = pytest.mark.gpu


def repacked(w, ws):
    N, K = w.shape[0], w.shape[1] * 2
    wb, sb = _native.packed_bytes(N, K)
    wq = torch.empty(wb, dtype=torch.uint8, device="cuda")
    sq = torch.empty(sb, dtype=torch.uint8, device="cuda")
    wd, sd = to_dev(w), to_dev(ws)
    _native.repack(wd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, stream())
    return wq, sq


def one_launch(x_dev, ldx, M, N, K, wq, sq):
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.linear(x_dev.data_ptr(), ldx, q.data_ptr(), s.data_ptr(), wq.data_ptr(), sq.data_ptr(),
                   out.data_ptr(), M, N, K, stream())
    torch.cuda.synchronize()
    return host_u16(out)


def two_launches(x_dev, ldx, M, N, K, wq, sq):
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.quant_per_token(x_dev.data_ptr(), ldx, q.data_ptr(), s.data_ptr(), M, K, stream())
    _native.gemm(q.data_ptr(), s.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream())
    torch.cuda.synchronize()
    return host_u16(out)


def strided(x_bits, ldx):
    M, K = x_bits.shape
    pad = np.full((M, ldx), 0x7FC0, np.uint16)          # NaN filler past K: must never be read
    pad[:, :K] = x_bits
    return bf16_dev(pad)


@pytest.mark.parametrize("N,K", [(17408, 5120), (10240, 5120), (5120, 6144), (5120, 8704),
                                 (2048, 1024), (1040, 512)])
def test_one_launch_equals_quantizer_then_gemm(gpu_lib, N, K):
    w, ws = synthetic.weights(N, K, seed=N + K)
    wq, sq = repacked(w, ws)
    # one launch at M <= 2, and up to M = 4 with 3 or more n-tiles per workgroup (qkv, gate_up)
    # or at most 4 row chunks per lane of a quantizing wave (o_proj); the small shapes plan
    # variants of 16 waves, with no room for the quantizing waves
    fused_up_to = {(17408, 5120): 4, (10240, 5120): 4, (5120, 6144): 4, (5120, 8704): 2}
    assert [_native.linear_fused(M, N, K, K) for M in range(1, 9)] == \
        [M <= fused_up_to.get((N, K), 0) for M in range(1, 9)]
    for M in range(1, 9):
        x = synthetic.activations(M, K, seed=M * 31 + N)
        xd = bf16_dev(x)
        print(f"[linear] M={M} N={N} K={K}", flush=True)
        fused = one_launch(xd, K, M, N, K, wq, sq)
        ref = two_launches(xd, K, M, N, K, wq, sq)
        bad = np.argwhere(fused != ref)
        assert bad.size == 0, f"M={M}: {len(bad)} outputs differ, first {bad[:3].tolist()}"
        if M in (1, 2, 8):
            q, s = O.quant_per_token(x)
            assert_gemm_close(fused, q, s, w, ws, f"one-launch linear M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1, 2, 5])
def test_strided_rows(gpu_lib, M):
    N, K, ldx = 5120, 5120, 5120 + 72
    w, ws = synthetic.weights(N, K, seed=3)
    wq, sq = repacked(w, ws)
    x = synthetic.activations(M, K, seed=M)
    assert _native.linear_fused(M, N, K, ldx) == (M <= 2)
    xd = strided(x, ldx)
    fused = one_launch(xd, ldx, M, N, K, wq, sq)
    assert np.array_equal(fused, two_launches(xd, ldx, M, N, K, wq, sq))
    assert np.array_equal(fused, two_launches(bf16_dev(x), K, M, N, K, wq, sq))


@pytest.mark.parametrize("M", [1, 2])
def test_special_rows(gpu_lib, M):
    """Zero row, a NaN and an inf in a row (non-finite scale: the per-element path), the largest
    bf16 magnitudes, subnormals, a row of one nonzero value; one row (or two) at a time through
    the one-launch form."""
    N, K = 5120, 5120
    w, ws = synthetic.weights(N, K, seed=7)
    wq, sq = repacked(w, ws)
    assert _native.linear_fused(M, N, K, K)
    base = synthetic.activations(8, K, seed=11)
    rows = [base[0].copy() * 0, base[1].copy(), base[2].copy(), base[3].copy(), base[4].copy(),
            base[5].copy() * 0, base[6].copy()]
    rows[1][77] = 0x7FC0                                # NaN
    rows[2][4000] = 0x7F80                              # +inf
    rows[3][::3] = 0x7F7F                               # largest finite bf16
    rows[3][1::3] = 0xFF7F
    rows[4][:] = np.random.default_rng(0).integers(1, 0x80, K).astype(np.uint16)  # subnormals
    rows[5][5119] = 0x3F80
    rows[6][512] = 0xFF80                               # -inf
    for i in range(len(rows)):
        x = np.stack([rows[(i + j) % len(rows)] for j in range(M)])
        xd = bf16_dev(x)
        fused = one_launch(xd, K, M, N, K, wq, sq)
        ref = two_launches(xd, K, M, N, K, wq, sq)
        same = (fused == ref) | (np.isnan(O.bf16_to_f32(fused)) & np.isnan(O.bf16_to_f32(ref)))
        assert same.all(), (i, np.argwhere(~same)[:5].tolist())


def test_falls_back_where_it_cannot_fuse(gpu_lib):
    """M = 9, a row stride that breaks 16-byte chunks and a misaligned x go through two launches
    and give the same bits as the quantizer and the GEMM."""
    N, K = 2048, 1024
    w, ws = synthetic.weights(N, K, seed=5)
    wq, sq = repacked(w, ws)
    assert not _native.linear_fused(9, N, K, K)
    assert not _native.linear_fused(1, N, K, K + 4)
    x = synthetic.activations(9, K, seed=9)
    xd = bf16_dev(x)
    assert np.array_equal(one_launch(xd, K, 9, N, K, wq, sq), two_launches(xd, K, 9, N, K, wq, sq))
    xs = strided(x[:1], K + 4)
    assert np.array_equal(one_launch(xs, K + 4, 1, N, K, wq, sq),
                          two_launches(xs, K + 4, 1, N, K, wq, sq))
    buf = torch.empty(K + 8, dtype=torch.bfloat16, device="cuda")
    mis = buf[1:1 + K].view(1, K)                       # 2-byte aligned only
    mis.copy_(bf16_dev(x[:1]))
    assert np.array_equal(one_launch(mis, K, 1, N, K, wq, sq),
                          two_launches(bf16_dev(x[:1]), K, 1, N, K, wq, sq))
