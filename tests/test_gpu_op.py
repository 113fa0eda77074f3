"""The drop-in surface on the GPU: radiance::mxfp4_linear[_pq] and the MxFp4LinearKernel plugin's
process_weights_after_loading + apply_weights, end to end against the oracle."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from tests._check import assert_gemm_close, bf16_dev, host_u16, host_u8, to_dev
from vllm_sly_radiance_amd import _native, radiance_mxfp4 as R
from vllm_sly_radiance_amd import radiance_fused_norm  # noqa: F401  (registers radiance::*_quant)
from vllm_sly_radiance_amd import synthetic

pytestmark = pytest.mark.gpu


class Layer(torch.nn.Module):
    def __init__(self, w, ws):
        super().__init__()
        self.weight = torch.nn.Parameter(to_dev(w), requires_grad=False)
        self.weight_scale = torch.nn.Parameter(to_dev(ws), requires_grad=False)


@pytest.fixture(scope="module")
def kernel(gpu_lib):
    return R.kernel_class()()


@pytest.mark.parametrize("M,N,K", [(8, 5120, 5120), (1, 17408, 5120), (40, 5120, 8704),
                                   (600, 2048, 5120), (7, 20, 96)])
def test_plugin_load_and_apply(kernel, M, N, K):
    w, ws = synthetic.weights(N, K, seed=N)
    x = synthetic.activations(M, K, seed=M)
    layer = Layer(w, ws)
    storage = layer.weight.data_ptr()
    kernel.process_weights_after_loading(layer)
    aligned = N % 16 == 0 and K % 512 == 0
    assert (layer.weight.data_ptr() == storage) == aligned       # repacked in place when aligned
    assert tuple(layer.radiance_wref.shape) == (N, K, 0)
    owq, osq = O.repack(w, ws)
    assert np.array_equal(host_u8(layer.weight).reshape(-1), owq)
    assert np.array_equal(host_u8(layer.weight_scale).reshape(-1), osq)

    y = kernel.apply_weights(layer, bf16_dev(x))
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (M, N)
    q, s = O.quant_per_token(x)
    assert_gemm_close(host_u16(y), q, s, w, ws, f"apply_weights M={M} N={N} K={K}")

    # tuple (pre-quantized) contract and the quant-method name apply() give the same bits
    qd, sd = R.quant_per_token(bf16_dev(x))
    assert np.array_equal(host_u8(qd), q) and np.array_equal(sd.cpu().numpy(), s)
    y_pq = kernel.apply_weights(layer, (qd, sd))
    assert torch.equal(y_pq, y)
    assert torch.equal(kernel.apply(layer, bf16_dev(x)), y)

    bias = torch.randn(N, device="cuda", dtype=torch.bfloat16)
    assert torch.equal(kernel.apply_weights(layer, bf16_dev(x), bias), y + bias)


def test_leading_dims_are_flattened(kernel):
    N, K = 64, 512
    w, ws = synthetic.weights(N, K, seed=5)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    x = synthetic.activations(6, K, seed=6)
    y2 = kernel.apply_weights(layer, bf16_dev(x))
    y3 = kernel.apply_weights(layer, bf16_dev(x).view(2, 3, K))
    assert tuple(y3.shape) == (2, 3, N) and torch.equal(y3.reshape(6, N), y2)


def test_zero_tokens(kernel):
    """An empty batch (vLLM's dummy and padded runs can hand one over): every entry returns
    empty outputs of the right shapes and launches nothing."""
    N, K = 5120, 5120
    w, ws = synthetic.weights(N, K, seed=11)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    x = torch.zeros(0, K, device="cuda", dtype=torch.bfloat16)
    y = kernel.apply_weights(layer, x)
    assert y.dtype == torch.bfloat16 and tuple(y.shape) == (0, N)
    q, s = R.quant_per_token(x)
    assert tuple(q.shape) == (0, K) and tuple(s.shape) == (0,)
    assert tuple(kernel.apply_weights(layer, (q, s)).shape) == (0, N)
    assert tuple(kernel.apply_weights(layer, x.view(0, 1, K)).shape) == (0, 1, N)
    e = torch.zeros(0, K, device="cuda", dtype=torch.bfloat16)
    qa, sa, ra = torch.ops.radiance.add_rms_quant(e, e, torch.zeros(K, device="cuda",
                                                                    dtype=torch.bfloat16), 1e-6)
    assert tuple(qa.shape) == (0, K) and tuple(sa.shape) == (0,) and tuple(ra.shape) == (0, K)
    qg, sg = torch.ops.radiance.gdn_norm_quant(e, e, torch.zeros(128, device="cuda",
                                                                 dtype=torch.bfloat16), 1e-6)
    assert tuple(qg.shape) == (0, K) and tuple(sg.shape) == (0,)
    gu = torch.zeros(0, 2 * K, device="cuda", dtype=torch.bfloat16)
    yd = torch.ops.radiance.silu_mul_mxfp4_linear(gu, layer.weight, layer.weight_scale,
                                                  layer.radiance_wref)
    assert tuple(yd.shape) == (0, N)
    torch.cuda.synchronize()


def test_op_refuses_mismatched_activation(kernel):
    N, K = 64, 512
    w, ws = synthetic.weights(N, K, seed=7)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    x = torch.zeros(4, K + 32, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="does not match K"):
        kernel.apply_weights(layer, x)


def test_op_is_one_opaque_node_under_compile(kernel):
    N, K = 128, 1024
    w, ws = synthetic.weights(N, K, seed=8)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    f = torch.compile(lambda t: kernel.apply_weights(layer, t), fullgraph=True, dynamic=True,
                      backend="eager")
    x = bf16_dev(synthetic.activations(9, K, seed=9))
    assert torch.equal(f(x), kernel.apply_weights(layer, x))


@pytest.mark.parametrize("M", [1, 3, 8])
def test_hip_graph_capture_and_replay(kernel, M):
    """The op allocates nothing natively and launches on the current stream, so it captures into a
    HIP graph; every replay (with eager work and syncs in between) must match the eager result.
    M = 1 and 3 run as one launch (the quantizing waves' LDS counters start from zero in every
    replay), M = 8 as the quantizer and the GEMM."""
    N, K = 17408, 5120
    assert _native.linear_fused(M, N, K, K) == (M <= 4)
    w, ws = synthetic.weights(N, K, seed=10)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    x = bf16_dev(synthetic.activations(M, K, seed=11))
    eager = kernel.apply_weights(layer, x)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            kernel.apply_weights(layer, x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = kernel.apply_weights(layer, x)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"
        _ = (x.float() * 2).sum().item()          # unrelated eager work between replays


def test_hip_graph_capture_of_the_band_k_split(kernel):
    """down (5120 x 8704) at M = 24 runs the quantizer, the tile kernel's K-split launch into the
    registered scratch and the reducing launch: captured into a HIP graph, every replay (with eager
    work and syncs in between, and an eager call of another shape reusing the scratch) matches the
    eager result."""
    M, N, K = 24, 5120, 8704
    w, ws = synthetic.weights(N, K, seed=12)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    assert _native.plan(M, N, K)[2] == 3, "the band's K split is what this test captures"
    x = bf16_dev(synthetic.activations(M, K, seed=13))
    x2 = bf16_dev(synthetic.activations(40, K, seed=14))
    eager = kernel.apply_weights(layer, x)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            kernel.apply_weights(layer, x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = kernel.apply_weights(layer, x)
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager), f"replay {i}"
        kernel.apply_weights(layer, x2)           # another split call between the replays
        torch.cuda.synchronize()
    assert R._scratch[0] is not None


def test_checkpoint_ingestion_end_to_end(kernel, tmp_path):
    """A merged gate/up linear read from a sharded safetensors checkpoint, repacked in place by
    process_weights_after_loading and applied: equal to the oracle on the concatenated tensors."""
    import json
    import os

    from safetensors.torch import save_file

    from vllm_sly_radiance_amd import checkpoint as CK
    K = 1024
    g, gs = synthetic.weights(96, K, 11)
    u, us = synthetic.weights(64, K, 12)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    save_file({"l.gate_proj.weight_packed": t(g), "l.gate_proj.weight_scale": t(gs)},
              os.path.join(tmp_path, "a.safetensors"))
    save_file({"l.up_proj.weight_packed": t(u), "l.up_proj.weight_scale": t(us)},
              os.path.join(tmp_path, "b.safetensors"))
    with open(os.path.join(tmp_path, "model.safetensors.index.json"), "w") as f:
        json.dump({"weight_map": {"l.gate_proj.weight_packed": "a.safetensors",
                                  "l.gate_proj.weight_scale": "a.safetensors",
                                  "l.up_proj.weight_packed": "b.safetensors",
                                  "l.up_proj.weight_scale": "b.safetensors"}}, f)
    layer = torch.nn.Module()
    CK.load_linear(layer, CK.CheckpointIndex(str(tmp_path)), "l", ["gate_proj", "up_proj"])
    storage = layer.weight.data_ptr()
    kernel.process_weights_after_loading(layer)
    assert layer.weight.data_ptr() == storage                    # repacked in the same storage
    M = 8
    x = synthetic.activations(M, K, 13)
    y = kernel.apply_weights(layer, bf16_dev(x))
    w, ws = np.concatenate([g, u], 0), np.concatenate([gs, us], 0)
    q, s = O.quant_per_token(x)
    assert_gemm_close(host_u16(y), q, s, w, ws, "checkpoint gate_up M=8")


def test_in_situ_exact_check_and_shape_log(kernel, monkeypatch, capsys):
    """RADIANCE_MXFP4_CHECKALL and RADIANCE_MXFP4_MHIST on the device: every checked call of the
    listed shape (one-launch and two-launch linears, the pre-quantized op, SiLU-mul + down) agrees
    with the torch fp32 dequant-matmul, and each (N, K, M) is logged once with its plan."""
    from vllm_sly_radiance_amd import diagnostics as D
    N, K = 5120, 8704
    monkeypatch.setattr(D, "CHECK_ALL", {(N, K)})
    monkeypatch.setattr(D, "MHIST", True)
    monkeypatch.setattr(D, "_seen", set())
    w, ws = synthetic.weights(N, K, seed=41)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    before = (R.STATS.get("checked", 0), R.STATS.get("wrong", 0))
    for M in (1, 8, 40):
        x = bf16_dev(synthetic.activations(M, K, seed=M))
        kernel.apply_weights(layer, x)
        kernel.apply_weights(layer, R.quant_per_token(x))
    gu = bf16_dev(synthetic.activations(1, 2 * K, seed=5))
    torch.ops.radiance.silu_mul_mxfp4_linear(gu, layer.weight, layer.weight_scale,
                                             layer.radiance_wref)
    torch.cuda.synchronize()
    err = capsys.readouterr().err
    assert R.STATS["checked"] - before[0] == 7
    assert R.STATS.get("wrong", 0) == before[1], err
    for M in (1, 8, 40):
        assert err.count(f"[radiance.mxfp4.mhist] N={N} K={K} M={M} ") == 1


def test_sanitize_and_sync_switches(kernel, monkeypatch):
    """RADIANCE_MXFP4_SANITIZE zeroes NaN and inf in the bf16 activations before the quantizer: a
    row holding a NaN gives the output of the cleaned row instead of a NaN row (one-launch and
    two-launch forms). RADIANCE_MXFP4_SYNC only synchronizes: the same bits."""
    from vllm_sly_radiance_amd import diagnostics as D
    N, K = 5120, 5120
    w, ws = synthetic.weights(N, K, seed=43)
    layer = Layer(w, ws)
    kernel.process_weights_after_loading(layer)
    for M in (1, 8):
        x = bf16_dev(synthetic.activations(M, K, seed=7 + M))
        bad = x.clone()
        bad[0, 5] = float("nan")
        bad[M - 1, 9] = float("inf")
        clean = bad.clone()
        clean[0, 5] = 0.0
        clean[M - 1, 9] = 0.0
        monkeypatch.setattr(D, "SANITIZE_X", False)
        y_bad = kernel.apply_weights(layer, bad)
        assert torch.isnan(y_bad[0].float()).all()
        y_clean = kernel.apply_weights(layer, clean)
        monkeypatch.setattr(D, "SANITIZE_X", True)
        assert torch.equal(kernel.apply_weights(layer, bad), y_clean)
        assert torch.isnan(bad[0, 5])                        # the caller's tensor is untouched
        monkeypatch.setattr(D, "SANITIZE_X", False)
        for mode in ("1", "2"):
            monkeypatch.setattr(D, "SYNC", mode)
            assert torch.equal(kernel.apply_weights(layer, x), kernel.apply_weights(layer, x))
        monkeypatch.setattr(D, "SYNC", "0")


def test_padded_cloned_output_and_debug_switches(kernel, monkeypatch, capsys):
    """RADIANCE_MXFP4_PADOUT (an output 3 elements into a padded slab, so every kernel's epilogue
    meets a pointer that is only 2-byte aligned), RADIANCE_MXFP4_CLONE and RADIANCE_MXFP4_DEBUG:
    the same bits as the plain output on every path the ops take (one launch, stream, tile K split,
    band kernel, mid tile, the pre-quantized op, SiLU-mul + down in one launch and in two), and one
    exact-check line per shape, all ok."""
    from vllm_sly_radiance_amd import diagnostics as D
    monkeypatch.setattr(D, "_seen", set())
    cases = [((5120, 8704), (1, 8, 40, 600)), ((17408, 5120), (40,))]
    for (N, K), Ms in cases:
        w, ws = synthetic.weights(N, K, seed=47)
        layer = Layer(w, ws)
        kernel.process_weights_after_loading(layer)
        for M in Ms:
            x = bf16_dev(synthetic.activations(M, K, seed=M + 3))
            qx = R.quant_per_token(x)
            gu = bf16_dev(synthetic.activations(M, 2 * K, seed=M + 4)) if N == 5120 and M < 8 else None
            print(f"[op] padded output N={N} K={K} M={M}", flush=True)

            def run():
                ys = [kernel.apply_weights(layer, x), kernel.apply_weights(layer, qx)]
                if gu is not None:
                    ys.append(torch.ops.radiance.silu_mul_mxfp4_linear(
                        gu, layer.weight, layer.weight_scale, layer.radiance_wref))
                torch.cuda.synchronize()
                return ys
            monkeypatch.setattr(D, "PAD_OUT", 0)
            monkeypatch.setattr(D, "CLONE_OUT", False)
            monkeypatch.setattr(D, "DEBUG", False)
            plain = run()
            monkeypatch.setattr(D, "PAD_OUT", 3)
            monkeypatch.setattr(D, "CLONE_OUT", True)
            monkeypatch.setattr(D, "DEBUG", M <= 128)
            padded = run()
            for a, b in zip(plain, padded):
                assert b.shape == a.shape and torch.equal(a.view(torch.int16), b.view(torch.int16))
    monkeypatch.setattr(D, "DEBUG", False)
    err = capsys.readouterr().err
    lines = [ln for ln in err.splitlines() if ln.startswith("[radiance.mxfp4.exact]")]
    assert len(lines) == 4 and all(ln.endswith(" ok") for ln in lines), err
