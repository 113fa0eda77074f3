"""The MLP's SiLU-and-mul and down projection in one call (w4a8_silu_mul_linear; one launch at
M <= 2, where the streaming GEMM's quantizing waves form the SiLU-and-mul stage themselves) against
the producer followed by the GEMM, bit for bit: the plain rows of the benchmark's down shape and of
smaller ones, every bf16 gate pattern, the special gates (inf, NaN, the exp clamp) and the shapes
that fall back to two launches; and the torch op against radiance::silu_mul_quant +
mxfp4_linear_pq."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P
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


def fused(gu_dev, M, N, K, wq, sq):
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.silu_mul_linear(gu_dev.data_ptr(), q.data_ptr(), s.data_ptr(), wq.data_ptr(),
                            sq.data_ptr(), out.data_ptr(), M, N, K, stream())
    torch.cuda.synchronize()
    return host_u16(out)


def producer_then_gemm(gu_dev, M, N, K, wq, sq):
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.silu_mul_quant(gu_dev.data_ptr(), q.data_ptr(), s.data_ptr(), M, K, stream())
    _native.gemm(q.data_ptr(), s.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream())
    torch.cuda.synchronize()
    return host_u16(out)


def same(a, b, what):
    """Bit for bit, a NaN output equal to any NaN output: a row with a NaN in its bf16 stage has a
    NaN scale and NaN codes, and the sign of the GEMM's NaN products is the hardware's choice
    between the two NaN operands of the epilogue's scaling (as for the one-launch linear)."""
    ok = (a == b) | (np.isnan(O.bf16_to_f32(a)) & np.isnan(O.bf16_to_f32(b)))
    bad = np.argwhere(~ok)
    assert bad.size == 0, f"{what}: {len(bad)} outputs differ, first {bad[:3].tolist()}"


# the benchmark's down projection (one launch at M <= 2), a 5120-wide square one, and shapes whose
# plan has no room for quantizing waves (two launches at every M)
@pytest.mark.parametrize("N,K,one_up_to", [(5120, 8704, 2), (5120, 5120, 2), (2048, 1024, 0),
                                           (1040, 512, 0)])
def test_silu_mul_linear_equals_producer_then_gemm(gpu_lib, N, K, one_up_to):
    w, ws = synthetic.weights(N, K, seed=N + K)
    wq, sq = repacked(w, ws)
    assert [_native.silu_mul_linear_fused(M, N, K) for M in range(1, 6)] == \
        [M <= one_up_to for M in range(1, 6)]
    for M in (1, 2, 3, 5):
        gu = synthetic.activations(M, 2 * K, seed=M * 7 + K)
        gd = bf16_dev(gu)
        print(f"[silu-linear] M={M} N={N} K={K}", flush=True)
        got = fused(gd, M, N, K, wq, sq)
        same(got, producer_then_gemm(gd, M, N, K, wq, sq), f"M={M} N={N} K={K}")
        if M <= 2:
            q, s = P.silu_mul_quant(gu)
            assert_gemm_close(got, q, s, w, ws, f"silu-mul linear M={M} N={N} K={K}")


def gate_rows(M, K, start, rng):
    """[M, 2K] bf16 bits: gates are the bf16 patterns start, start + 1, ... (wrapping), ups finite
    random values."""
    gate = ((np.arange(M * K) + start) % 65536).astype(np.uint16).reshape(M, K)
    up = O.f32_to_bf16((rng.standard_normal((M, K)) * 3).astype(np.float32))
    return np.concatenate([gate, up], axis=1)


def test_silu_mul_linear_every_gate(gpu_lib):
    """Every bf16 gate pattern (zero, subnormal, inf, NaN and the exp clamp's range) through the
    one-launch form at M = 2, against the producer and the GEMM."""
    N, K = 5120, 8704
    w, ws = synthetic.weights(N, K, seed=5)
    wq, sq = repacked(w, ws)
    assert _native.silu_mul_linear_fused(2, N, K)
    rng = np.random.default_rng(3)
    for start in range(0, 65536, 2 * K):
        gu = gate_rows(2, K, start, rng)
        gd = bf16_dev(gu)
        print(f"[silu-linear] every gate from {start}", flush=True)
        same(fused(gd, 2, N, K, wq, sq), producer_then_gemm(gd, 2, N, K, wq, sq),
             f"gates from {start}")


def test_silu_mul_linear_special_rows(gpu_lib):
    """A zero row, a row with a NaN gate, one with an inf up value, the widest gates (-200 ..
    200) and a single nonzero value, one launch per pair of rows."""
    N, K = 5120, 5120
    w, ws = synthetic.weights(N, K, seed=9)
    wq, sq = repacked(w, ws)
    assert _native.silu_mul_linear_fused(2, N, K)
    g = np.linspace(-200.0, 200.0, K).astype(np.float32)
    u = (np.random.default_rng(2).standard_normal(K) * 2).astype(np.float32)
    rows = []
    rows.append((np.zeros(K, np.float32), u))
    gn = g.copy(); gn[17] = np.nan
    rows.append((gn, u))
    ui = u.copy(); ui[33] = np.inf
    rows.append((g, ui))
    rows.append((g, u))
    g1 = np.zeros(K, np.float32); g1[100] = 3.0
    rows.append((g1, np.ones(K, np.float32)))
    rows.append((g * 0.01, u))
    for i in range(0, len(rows), 2):
        pair = rows[i:i + 2]
        gu = np.stack([np.concatenate([O.f32_to_bf16(a), O.f32_to_bf16(b)]) for a, b in pair])
        gd = bf16_dev(gu)
        print(f"[silu-linear] special rows {i}, {i + 1}", flush=True)
        same(fused(gd, len(pair), N, K, wq, sq), producer_then_gemm(gd, len(pair), N, K, wq, sq),
             f"special rows {i}")


def test_silu_mul_linear_op(gpu_lib):
    """radiance::silu_mul_mxfp4_linear (the plugin's MLP tail) equals radiance::silu_mul_quant
    followed by radiance::mxfp4_linear_pq, through a layer prepared by
    process_weights_after_loading; leading dimensions and M = 0 pass through."""
    from vllm_sly_radiance_amd import radiance_fused_norm as F
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    N, K = 5120, 8704
    w, ws = synthetic.weights(N, K, seed=11)
    layer = torch.nn.Module()
    layer.weight = torch.nn.Parameter(to_dev(w), requires_grad=False)
    layer.weight_scale = torch.nn.Parameter(to_dev(ws), requires_grad=False)
    layer.bias = None
    R.kernel_class()().process_weights_after_loading(layer)
    for M in (1, 2, 3, 4):
        gu = bf16_dev(synthetic.activations(M, 2 * K, seed=M))
        y, y_bias = F.silu_mul_down(layer, gu)          # unpacked as RowParallelLinear's output
        assert y_bias is None
        q, s = torch.ops.radiance.silu_mul_quant(gu)
        ref = torch.ops.radiance.mxfp4_linear_pq(q, s, layer.weight, layer.weight_scale,
                                                 layer.radiance_wref)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), f"M={M}"
    gu3 = bf16_dev(synthetic.activations(6, 2 * K, seed=6)).view(2, 3, 2 * K)
    assert F.silu_mul_down(layer, gu3)[0].shape == (2, 3, N)
    empty = torch.empty((0, 2 * K), dtype=torch.bfloat16, device="cuda")
    assert F.silu_mul_down(layer, empty)[0].shape == (0, N)
    # a bias is added unless the layer defers it (skip_bias_add), as RowParallelLinear does
    layer.bias = torch.nn.Parameter(bf16_dev(synthetic.activations(1, N, seed=12)[0]),
                                    requires_grad=False)
    gu = bf16_dev(synthetic.activations(2, 2 * K, seed=13))
    y, y_bias = F.silu_mul_down(layer, gu)
    q, s = torch.ops.radiance.silu_mul_quant(gu)
    ref = torch.ops.radiance.mxfp4_linear_pq(q, s, layer.weight, layer.weight_scale,
                                             layer.radiance_wref)
    assert y_bias is None and torch.equal(y, ref + layer.bias)
    layer.skip_bias_add = True
    y, y_bias = F.silu_mul_down(layer, gu)
    assert y_bias is layer.bias and torch.equal(y.view(torch.int16), ref.view(torch.int16))
