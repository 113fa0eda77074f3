"""GPU parity of the fragment-tiled activation handoff: the producers writing q fragment-tiled
(q_layout 1), the tile GEMM reading it (w4a8_gemm_at, kernel TILE_AT) and the custom-op handoff
between them. Bar: the tiled bytes of every real token equal the oracle's tile_q of the oracle's
row-major codes, bit for bit, and padding tokens are left as they were; the tiled GEMM equals the
row-major GEMM through the same tile variant bit for bit (only addresses differ), and the oracle
within the tolerance of tests/_check.py."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P
from tests._check import assert_gemm_close, bf16_dev, host_u16, host_u8, stream, to_dev
from vllm_sly_radiance_amd import _native, synthetic
from vllm_sly_radiance_amd import radiance_fused_norm as FN
from vllm_sly_radiance_amd import radiance_mxfp4 as R

pytestmark = pytest.mark.gpu

TILE, TILE_AT = _native.KERNEL_TILE, _native.KERNEL_TILE_AT
SENTINEL = 0xA5


@pytest.fixture(params=["one_workgroup_per_row", "split_rows"])
def producer_path(request, gpu_lib):
    """silu_mul splits rows of small M over one-wave workgroups when scratch for the partial
    maxima is registered; both paths must write the tiled layout."""
    R.ensure_scratch("cuda")
    part, cnt = R._scratch
    if request.param == "one_workgroup_per_row":
        _native.set_scratch(None, 0, cnt.data_ptr(), cnt.numel() * 4)
    yield request.param
    _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)


def tiled_buffer(M, K):
    return torch.full((_native.tiled_bytes(M, K),), SENTINEL, dtype=torch.uint8, device="cuda")


def check_tiled(t_dev, M, K, oq, what):
    """t_dev: the device bytes a producer wrote with q_layout 1; oq: the oracle's row-major codes."""
    t = host_u8(t_dev)
    assert t.size == -(-M // 16) * 16 * K
    canon = lambda c: np.where((c & 0x7F) == 0x7F, 0x7F, c)
    got = O.untile_q(t, M, K)
    bad = np.argwhere(canon(got) != canon(oq))
    assert bad.size == 0, f"{what}: {len(bad)} tiled codes differ, first at {bad[:3].tolist()}"
    written = np.zeros(t.size, bool)
    written[O.tile_q(np.ones((M, K), np.uint8)).astype(bool)] = True
    assert np.all(t[~written] == SENTINEL), f"{what}: padding tokens were written"


@pytest.mark.parametrize("M,K", [(1, 256), (17, 5120), (130, 1024), (64, 10240)])
def test_add_rms_quant_writes_tiled(gpu_lib, M, K):
    y = synthetic.activations(M, K, seed=M)
    res = synthetic.activations(M, K, seed=M + 1)
    w = O.f32_to_bf16((np.random.default_rng(K).standard_normal(K) * 0.1).astype(np.float32))
    t = tiled_buffer(M, K)
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    r = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
    yd, rd, wd = bf16_dev(y), bf16_dev(res), bf16_dev(w)
    print(f"[tiled] add_rms_quant M={M} K={K}", flush=True)
    _native.add_rms_quant(yd.data_ptr(), rd.data_ptr(), wd.data_ptr(), t.data_ptr(), s.data_ptr(),
                          r.data_ptr(), M, K, 1e-6, stream(), _native.Q_TILED)
    torch.cuda.synchronize()
    oq, os_, orr = P.add_rms_quant(y, res, w, 1e-6)
    check_tiled(t, M, K, oq, f"add_rms M={M} K={K}")
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))
    assert np.array_equal(host_u16(r), orr)


@pytest.mark.parametrize("M,N", [(8, 17408), (3, 8704), (64, 8704), (200, 8704), (129, 18432)])
def test_silu_mul_quant_writes_tiled(producer_path, M, N):
    gu = synthetic.activations(M, 2 * N, seed=M * 5 + N)
    t = tiled_buffer(M, N)
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    gd = bf16_dev(gu)
    print(f"[tiled] silu_mul_quant M={M} N={N} {producer_path}", flush=True)
    _native.silu_mul_quant(gd.data_ptr(), t.data_ptr(), s.data_ptr(), M, N, stream(),
                           _native.Q_TILED)
    torch.cuda.synchronize()
    oq, os_ = P.silu_mul_quant(gu)
    check_tiled(t, M, N, oq, f"silu M={M} N={N} {producer_path}")
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


@pytest.mark.parametrize("M,heads", [(9, 48), (130, 80), (1, 1)])
def test_gdn_norm_quant_writes_tiled(gpu_lib, M, heads):
    N = heads * 128
    x = synthetic.activations(M, N, seed=M + heads)
    z = synthetic.activations(M, N, seed=M + heads + 1)
    w = O.f32_to_bf16((1.0 + np.random.default_rng(heads).standard_normal(128) * 0.2)
                      .astype(np.float32))
    t = tiled_buffer(M, N)
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    xd, zd, wd = bf16_dev(x), bf16_dev(z), bf16_dev(w)
    print(f"[tiled] gdn_norm_quant M={M} N={N}", flush=True)
    _native.gdn_norm_quant(xd.data_ptr(), zd.data_ptr(), N, wd.data_ptr(), t.data_ptr(),
                           s.data_ptr(), M, N, 1e-6, stream(), _native.Q_TILED)
    torch.cuda.synchronize()
    oq, os_ = P.gdn_norm_quant(x, z, w, 1e-6)
    check_tiled(t, M, N, oq, f"gdn M={M} N={N}")
    assert np.array_equal(s.cpu().numpy().view(np.uint32), os_.view(np.uint32))


def repacked(w, ws):
    N, K = w.shape[0], w.shape[1] * 2
    wb, sb = _native.packed_bytes(N, K)
    wd, sd = to_dev(w), to_dev(ws)
    wq = torch.empty(wb, dtype=torch.uint8, device="cuda")
    sq = torch.empty(sb, dtype=torch.uint8, device="cuda")
    _native.repack(wd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, stream())
    return wq, sq


def run(a_dev, s_dev, wq, sq, M, N, K, kernel=0, variant=-1, tiled_auto=False):
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    if tiled_auto:
        _native.gemm_at(a_dev.data_ptr(), s_dev.data_ptr(), wq.data_ptr(), sq.data_ptr(),
                        out.data_ptr(), M, N, K, stream())
    else:
        _native.gemm(a_dev.data_ptr(), s_dev.data_ptr(), wq.data_ptr(), sq.data_ptr(),
                     out.data_ptr(), M, N, K, stream(), kernel, variant, 1)
    torch.cuda.synchronize()
    return host_u16(out)


def tiled_dev(q, K):
    """The oracle's tiled bytes of q, padding tokens filled with the sentinel (never read into an
    output)."""
    M = q.shape[0]
    t = O.tile_q(q)
    pad = np.ones(t.size, bool)
    pad[O.tile_q(np.ones((M, K), np.uint8)).astype(bool)] = False
    t[pad] = SENTINEL
    return to_dev(t)


# ragged M (blocks past M), ragged N, K = 384 and 640 end inside a k-group
@pytest.mark.parametrize("M,N,K", [(65, 544, 1024), (300, 1040, 2560), (129, 33, 640),
                                   (513, 5120, 8704), (17, 200, 384)])
def test_gemm_at_every_tile_variant_matches_row_major(gpu_lib, M, N, K):
    x = synthetic.activations(M, K, seed=M + 7)
    w, ws = synthetic.weights(N, K, seed=N + 7)
    q, s = O.quant_per_token(x)
    wq, sq = repacked(w, ws)
    qd, td, sd = to_dev(q), tiled_dev(q, K), to_dev(s.astype(np.float32))
    for v, cfg in enumerate(_native.variants(TILE)):
        print(f"[tiled] gemm M={M} N={N} K={K} tile variant {v} {cfg}", flush=True)
        ref = run(qd, sd, wq, sq, M, N, K, TILE, v)
        out = run(td, sd, wq, sq, M, N, K, TILE_AT, v)
        if v == 0:
            assert_gemm_close(out, q, s, w, ws, f"tiled M={M} N={N} K={K} variant {v}")
        bad = np.argwhere(out != ref)
        assert bad.size == 0, f"variant {v} {cfg}: {len(bad)} outputs differ from row-major"


# the four linear shapes of the benchmark model through w4a8_gemm_at's plan; at M > 64 the
# row-major automatic plan is the same tile plan, so the outputs must agree bit for bit
@pytest.mark.parametrize("M", [1, 20, 64, 65, 512])
@pytest.mark.parametrize("N,K", [(10240, 5120), (5120, 6144), (17408, 5120), (5120, 8704)])
def test_gemm_at_auto_plan(gpu_lib, M, N, K):
    x = synthetic.activations(M, K, seed=M + N)
    w, ws = synthetic.weights(N, K, seed=N)
    q, s = O.quant_per_token(x)
    wq, sq = repacked(w, ws)
    qd, td, sd = to_dev(q), tiled_dev(q, K), to_dev(s.astype(np.float32))
    print(f"[tiled] gemm_at M={M} N={N} K={K}", flush=True)
    out = run(td, sd, wq, sq, M, N, K, tiled_auto=True)
    rows = np.arange(M)
    if M > 64:
        assert np.array_equal(out, run(qd, sd, wq, sq, M, N, K)), "differs from row-major plan"
        rows = np.unique(np.r_[np.random.default_rng(M).choice(M, 62, replace=False), 0, M - 1])
    assert_gemm_close(out[rows], q[rows], s[rows], w, ws, f"gemm_at M={M} N={N} K={K}")


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 8704)])
def test_gemm_at_prefill_4096(gpu_lib, N, K):
    """M = 4096 (gate_up runs as two launches, 256 x 256 tiles and a 128 x 128 column tail):
    bit-identical to the row-major GEMM, 128 sampled rows against the oracle."""
    M = 4096
    x = synthetic.activations(M, K, seed=K + 1)
    w, ws = synthetic.weights(N, K, seed=N + 1)
    q, s = O.quant_per_token(x)
    wq, sq = repacked(w, ws)
    qd, td, sd = to_dev(q), tiled_dev(q, K), to_dev(s.astype(np.float32))
    print(f"[tiled] gemm_at M=4096 N={N} K={K}", flush=True)
    out = run(td, sd, wq, sq, M, N, K, tiled_auto=True)
    assert np.array_equal(out, run(qd, sd, wq, sq, M, N, K)), "differs from row-major plan"
    rows = np.unique(np.r_[np.random.default_rng(2).choice(M, 126, replace=False), 0, M - 1])
    assert_gemm_close(out[rows], q[rows], s[rows], w, ws, f"gemm_at M=4096 N={N} K={K}")


@pytest.fixture
def tiled_on(monkeypatch, gpu_lib):
    """The handoff armed at M >= 65, a clean handoff table, the plugin's scratch registered."""
    R.ensure_scratch("cuda")
    monkeypatch.setattr(R, "A_TILED_MIN_M", 65)
    R.A_TILED.clear()
    yield
    R.A_TILED.clear()


def plugin_weights(N, K, seed):
    w, ws = synthetic.weights(N, K, seed)
    wq, sq = R.repack_weights(to_dev(w), to_dev(ws))
    return wq, sq, R.layout_ref(N, K, "cuda")


@pytest.mark.parametrize("M", [64, 65, 300])
def test_op_handoff_add_rms_to_linear(tiled_on, M):
    """add_rms_quant -> mxfp4_linear_pq (the qkv / gate_up consumers): tiled from M = 65, the
    same bits as the row-major chain either way."""
    K, N = 5120, 10240
    y, res = bf16_dev(synthetic.activations(M, K, 1)), bf16_dev(synthetic.activations(M, K, 2))
    nw = bf16_dev(O.f32_to_bf16((np.random.default_rng(3).standard_normal(K) * 0.1)
                                .astype(np.float32)))
    wq, sq, wref = plugin_weights(N, K, 4)
    before = R.STATS["calls_tiled"]
    q, s, r = torch.ops.radiance.add_rms_quant(y, res, nw, 1e-6)
    assert tuple(q.shape) == (M, K) and q.is_contiguous()
    tiled = M >= 65
    assert R.a_tiled_take(q, M, K) == tiled
    out = torch.ops.radiance.mxfp4_linear_pq(q, s, wq, sq, wref)
    out2 = torch.ops.radiance.mxfp4_linear_pq(q, s, wq, sq, wref)   # a second consumer
    assert R.STATS["calls_tiled"] - before == (2 if tiled else 0)
    R.A_TILED.clear()
    R.A_TILED_MIN_M = 0
    q_rm, s_rm, r_rm = torch.ops.radiance.add_rms_quant(y, res, nw, 1e-6)
    ref = torch.ops.radiance.mxfp4_linear_pq(q_rm, s_rm, wq, sq, wref)
    torch.cuda.synchronize()
    assert torch.equal(s, s_rm) and torch.equal(r, r_rm)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))


def test_op_handoff_silu_to_down(tiled_on):
    """silu_mul_quant -> mxfp4_linear_pq (the down consumer) at M = 256."""
    M, N, Kd = 256, 5120, 8704
    gu = bf16_dev(synthetic.activations(M, 2 * Kd, 5))
    wq, sq, wref = plugin_weights(N, Kd, 6)
    q, s = torch.ops.radiance.silu_mul_quant(gu)
    assert R.a_tiled_take(q, M, Kd)
    out = torch.ops.radiance.mxfp4_linear_pq(q, s, wq, sq, wref)
    R.A_TILED.clear()
    R.A_TILED_MIN_M = 0
    q_rm, s_rm = torch.ops.radiance.silu_mul_quant(gu)
    ref = torch.ops.radiance.mxfp4_linear_pq(q_rm, s_rm, wq, sq, wref)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert np.array_equal(O.untile_q(tiled_bytes_of(q, M, Kd), M, Kd), host_u8(q_rm))


def tiled_bytes_of(q, M, K):
    """The whole tiled storage behind an [M, K] tiled view (whole 16-token blocks), on the host."""
    torch.cuda.synchronize()
    return host_u8(torch.as_strided(q.view(torch.uint8), (_native.tiled_bytes(M, K),), (1,)))


def test_gated_norm_stays_row_major_unless_switched(tiled_on, monkeypatch):
    M, heads = 130, 48
    N = heads * 128
    x = bf16_dev(synthetic.activations(M, N, 7))
    z = bf16_dev(synthetic.activations(M, N, 8))
    w = bf16_dev(O.f32_to_bf16(np.ones(128, np.float32)))
    q, _ = torch.ops.radiance.gdn_norm_quant(x, z, w, 1e-6)
    assert not R.a_tiled_take(q, M, N)
    monkeypatch.setattr(FN, "TILED_OPROJ", True)
    qt, _ = torch.ops.radiance.gdn_norm_quant(x, z, w, 1e-6)
    assert R.a_tiled_take(qt, M, N)
    assert np.array_equal(O.untile_q(tiled_bytes_of(qt, M, N), M, N), host_u8(q))
