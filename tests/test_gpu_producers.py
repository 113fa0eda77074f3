"""GPU parity of the fused fp8 activation producers against the oracle, through the C ABI and the
custom ops. Bar: codes, scales and the bf16 residual output bit-exact (every floating-point step of
the producers is fixed; oracle/producers_oracle.py)."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P
from tests import _orders as ORD
from tests._check import bf16_dev, host_u16, host_u8, to_dev
from vllm_sly_radiance_amd import _native, synthetic
from vllm_sly_radiance_amd import radiance_fused_norm as FN
from vllm_sly_radiance_amd import radiance_mxfp4 as R

pytestmark = pytest.mark.gpu


def stream():
    return torch.cuda.current_stream().cuda_stream


@pytest.fixture(params=["one_workgroup_per_row", "split_rows"])
def producer_path(request, gpu_lib):
    """silu_mul splits rows of small M over one-wave workgroups when scratch for the partial
    maxima is registered; without it, it takes one workgroup per row. Runs a test both ways and
    leaves the scratch registered."""
    R.ensure_scratch("cuda")
    part, cnt = R._scratch
    if request.param == "one_workgroup_per_row":
        _native.set_scratch(None, 0, cnt.data_ptr(), cnt.numel() * 4)
    yield request.param
    _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)


def weight_bits(K, seed, mean=0.0, sd=0.1):
    return O.f32_to_bf16((mean + np.random.default_rng(seed).standard_normal(K) * sd)
                         .astype(np.float32))


def gpu_add_rms(y, res, w, eps):
    M, K = y.shape
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    r = torch.empty((M, K), dtype=torch.bfloat16, device="cuda")
    yd, rd, wd = bf16_dev(y), bf16_dev(res), bf16_dev(w)
    print(f"[producers] add_rms_quant M={M} K={K}", flush=True)
    _native.add_rms_quant(yd.data_ptr(), rd.data_ptr(), wd.data_ptr(), q.data_ptr(), s.data_ptr(),
                          r.data_ptr(), M, K, eps, stream())
    torch.cuda.synchronize()
    return host_u8(q), s.cpu().numpy(), host_u16(r)


def assert_same_qs(q, s, oq, os_, what):
    assert np.array_equal(np.isnan(s), np.isnan(os_)), f"{what}: NaN scales differ"
    fin = ~np.isnan(os_)
    bad_s = np.argwhere(s[fin].view(np.uint32) != os_[fin].view(np.uint32))
    assert bad_s.size == 0, f"{what}: {len(bad_s)} scales differ, first rows {bad_s[:3].ravel()}"
    canon = lambda c: np.where((c & 0x7F) == 0x7F, 0x7F, c)
    bad = np.argwhere(canon(q) != canon(oq))
    assert bad.size == 0, f"{what}: {len(bad)} codes differ, first at {bad[:3].tolist()}"


@pytest.mark.parametrize("M,K", [(1, 5120), (7, 5120), (64, 8704), (3, 8), (5, 2056),
                                 (2, 10240), (300, 5120)])
def test_add_rms_quant_bit_exact(gpu_lib, M, K):
    y = synthetic.activations(M, K, seed=M + K)
    res = synthetic.activations(M, K, seed=M + K + 1)
    w = weight_bits(K, K)
    q, s, r = gpu_add_rms(y, res, w, 1e-6)
    oq, os_, orr = P.add_rms_quant(y, res, w, 1e-6)
    assert np.array_equal(r, orr), "residual_out differs"
    assert_same_qs(q, s, oq, os_, f"add_rms M={M} K={K}")


def test_add_rms_quant_special_rows(gpu_lib):
    K = 512
    rows = np.zeros((6, K), np.float32)
    rows[1, :] = 1e30                                   # huge: sum of squares overflows to inf
    rows[2, 5] = np.inf
    rows[3, 9] = np.nan
    rows[4, :] = np.linspace(-1e-20, 1e-20, K)          # tiny: eps dominates
    rows[5, :] = 448.0
    y = O.f32_to_bf16(rows)
    res = O.f32_to_bf16(np.zeros_like(rows))
    w = weight_bits(K, 1)
    q, s, r = gpu_add_rms(y, res, w, 1e-6)
    oq, os_, orr = P.add_rms_quant(y, res, w, 1e-6)
    assert np.array_equal(r, orr)
    assert_same_qs(q, s, oq, os_, "add_rms special rows")


@pytest.mark.parametrize("M", [1, 130])
def test_add_rms_quant_sum_order_pinned(gpu_lib, M):
    """Rows on which each plausible other order of the sum of squares (sequential, the butterfly
    reversed, the waves or a thread's groups reversed) gives another row scale than the fixed
    order (tests/_orders.py), run as M copies of each row: the kernel matches the oracle."""
    for y, w, tells in ORD.add_rms_cases():
        yy = np.repeat(y, M, axis=0)
        res = np.zeros_like(yy)
        q, s, r = gpu_add_rms(yy, res, w, 1e-6)
        oq, os_, orr = P.add_rms_quant(yy, res, w, 1e-6)
        assert np.array_equal(r, orr)
        assert_same_qs(q, s, oq, os_, f"add_rms M={M}, a row telling the fixed order from {tells}")


def test_add_rms_quant_sampled_rows_at_prefill_size(gpu_lib):
    """M=4096 K=5120: every row on the GPU, 96 sampled rows (and the first and last) against the
    oracle; the kernel is row-independent."""
    M, K = 4096, 5120
    y = synthetic.activations(M, K, seed=11)
    res = synthetic.activations(M, K, seed=12)
    w = weight_bits(K, 13)
    q, s, r = gpu_add_rms(y, res, w, 1e-6)
    rows = np.unique(np.r_[np.random.default_rng(0).choice(M, 96, replace=False), 0, M - 1])
    oq, os_, orr = P.add_rms_quant(y[rows], res[rows], w, 1e-6)
    assert np.array_equal(r[rows], orr)
    assert_same_qs(q[rows], s[rows], oq, os_, "add_rms M=4096")


def gpu_silu(gu):
    M, N2 = gu.shape
    N = N2 // 2
    q = torch.empty((M, N), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    gd = bf16_dev(gu)
    print(f"[producers] silu_mul_quant M={M} N={N}", flush=True)
    _native.silu_mul_quant(gd.data_ptr(), q.data_ptr(), s.data_ptr(), M, N, stream())
    torch.cuda.synchronize()
    return host_u8(q), s.cpu().numpy()


# M <= 64 splits rows of N > 16384 (with scratch) or runs 1024-thread rows, M <= 128 runs
# 1024-thread rows, larger M 256-thread rows: all must give the same bits
@pytest.mark.parametrize("M,N", [(1, 17408), (8, 17408), (33, 1000), (2, 18432), (64, 8704),
                                 (96, 8704), (4, 8), (200, 17408), (129, 18432), (16, 520)])
def test_silu_mul_quant_bit_exact(producer_path, M, N):
    gu = synthetic.activations(M, 2 * N, seed=M * 3 + N)
    q, s = gpu_silu(gu)
    oq, os_ = P.silu_mul_quant(gu)
    assert_same_qs(q, s, oq, os_, f"silu M={M} N={N}")


def test_silu_mul_quant_special_and_wide_range(producer_path):
    """Gate values across the whole range where exp is exercised (-200 .. 200: overflow, the
    subnormal results and the clamp, inf, NaN)."""
    N = 2048
    g = np.linspace(-200.0, 200.0, 3 * N).astype(np.float32).reshape(3, N)
    g[0, 7], g[1, 9], g[2, 11] = np.inf, -np.inf, np.nan
    u = (np.random.default_rng(1).standard_normal((3, N)) * 2).astype(np.float32)
    gu = np.concatenate([O.f32_to_bf16(g), O.f32_to_bf16(u)], axis=1)
    q, s = gpu_silu(gu)
    oq, os_ = P.silu_mul_quant(gu)
    assert_same_qs(q, s, oq, os_, "silu special")


def all_gates(M, N, seed):
    """[M, 2N] bf16 bits whose gate halves hold each of the 65536 bf16 patterns (shuffled; M N >=
    65536, the rest random patterns), with finite random up values."""
    rng = np.random.default_rng(seed)
    extra = rng.integers(0, 65536, M * N - 65536)
    gate = rng.permutation(np.r_[np.arange(65536), extra]).astype(np.uint16).reshape(M, N)
    up = O.f32_to_bf16((rng.standard_normal((M, N)) * 3).astype(np.float32))
    return np.concatenate([gate, up], axis=1)


@pytest.mark.parametrize("M,N", [(4, 17408), (8, 8192), (256, 256)])
def test_silu_mul_bf16_stage_every_gate(gpu_lib, M, N):
    """The bf16 stage over every bf16 gate, bit for bit (exp's overflow, underflow and clamp,
    the subnormal results, zero, inf and NaN gates), at 1024-thread rows of 3 and 1 groups per
    thread and at 256-thread rows."""
    gu = all_gates(M, N, seed=M)
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    gd = bf16_dev(gu)
    print(f"[producers] silu_mul M={M} N={N}", flush=True)
    _native.silu_mul(gd.data_ptr(), out.data_ptr(), M, N, stream())
    torch.cuda.synchronize()
    got = host_u16(out)
    ref = P.silu_mul(gu)
    bad = np.argwhere(got != ref)
    assert bad.size == 0, [(int(r), int(c), hex(int(gu[r, c])), hex(int(got[r, c])),
                            hex(int(ref[r, c]))) for r, c in bad[:6]]


@pytest.mark.parametrize("M,N", [(4, 17408), (32, 2048), (256, 256)])
def test_silu_mul_quant_every_gate(producer_path, M, N):
    """Every gate through the fused op: split rows (M = 4 with scratch), 1024- and 256-thread
    rows."""
    gu = all_gates(M, N, seed=M + 1)
    q, s = gpu_silu(gu)
    oq, os_ = P.silu_mul_quant(gu)
    assert_same_qs(q, s, oq, os_, f"silu every gate M={M}")


def gpu_gdn(x, z_wide, col0, w, eps):
    """z is columns col0 .. col0 + N - 1 of a wider bf16 tensor (row stride = its width)."""
    M, N = x.shape
    q = torch.empty((M, N), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    xd, zd, wd = bf16_dev(x), bf16_dev(z_wide), bf16_dev(w)
    zv = zd[:, col0:col0 + N]
    print(f"[producers] gdn_norm_quant M={M} N={N} z_stride={zv.stride(0)}", flush=True)
    _native.gdn_norm_quant(xd.data_ptr(), zv.data_ptr(), zv.stride(0), wd.data_ptr(),
                           q.data_ptr(), s.data_ptr(), M, N, eps, stream())
    torch.cuda.synchronize()
    return host_u8(q), s.cpu().numpy()


@pytest.mark.parametrize("M,heads,extra", [(1, 24, 0), (9, 48, 2048), (64, 80, 384), (3, 1, 8),
                                           (160, 48, 128), (130, 80, 0), (8, 5, 0)])
def test_gdn_norm_quant_bit_exact(gpu_lib, M, heads, extra):
    N = heads * 128
    x = synthetic.activations(M, N, seed=M + heads)
    zw = synthetic.activations(M, N + extra, seed=M + heads + 1)
    w = weight_bits(128, heads, mean=1.0, sd=0.2)
    q, s = gpu_gdn(x, zw, extra, w, 1e-6)
    oq, os_ = P.gdn_norm_quant(x, zw[:, extra:extra + N], w, 1e-6)
    assert_same_qs(q, s, oq, os_, f"gdn M={M} heads={heads} z offset {extra}")


@pytest.mark.parametrize("M", [1, 130])
def test_gdn_norm_quant_head_sum_order_pinned(gpu_lib, M):
    """Rows on which a sequential head sum or the 16-lane butterfly reversed gives another row
    scale than the fixed order (tests/_orders.py), as M copies (the 1024- and the 256-thread
    rows): the kernel matches the oracle."""
    for x, z, w, tells in ORD.gdn_cases():
        xx, zz = np.repeat(x, M, axis=0), np.repeat(z, M, axis=0)
        q, s = gpu_gdn(xx, zz, 0, w, 1e-6)
        oq, os_ = P.gdn_norm_quant(xx, zz, w, 1e-6)
        assert_same_qs(q, s, oq, os_, f"gdn M={M}, a row telling the fixed order from {tells}")


def _silu_groups(bits):
    """bf16 patterns -> the kernels' fp32 silu through w4a8_silu_f32 (len % 8 == 0)."""
    x = bf16_dev(np.ascontiguousarray(bits, dtype=np.uint16))
    y = torch.empty(len(bits), dtype=torch.float32, device="cuda")
    _native.silu_f32(x.data_ptr(), y.data_ptr(), len(bits), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return y.cpu().numpy()


def _assert_same_f32(got, want, bits, what):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), what
    bad = np.argwhere(got[~nan].view(np.uint32) != want[~nan].view(np.uint32)).ravel()
    assert bad.size == 0, (what, [(hex(int(b)), float(g), float(w)) for b, g, w in
                                  zip(bits[~nan][bad[:6]], got[~nan][bad[:6]], want[~nan][bad[:6]])])


def test_silu_quotient_every_bf16_input(gpu_lib):
    """The unrounded fp32 silu the producers compute (the gated norm multiplies it into its
    output), against the oracle's exact division for every bf16 input, on both of the kernels'
    paths: groups of 8 inputs that all have |x| <= 44 take the hardware reciprocal and one
    Markstein correction, any other group divides; every such input also goes through the
    division path, by sharing its group with one wide value."""
    print("[producers] silu fp32 over every bf16 input", flush=True)
    allb = np.arange(65536, dtype=np.uint16)
    xf = O.bf16_to_f32(allb)
    narrow = allb[np.abs(xf) <= 44.0]                     # NaN compares false: wide
    wide = allb[~(np.abs(xf) <= 44.0)]
    pad = lambda a: np.r_[a, a[:(-len(a)) % 8]]
    for what, bits in (("reciprocal path", pad(narrow)), ("division path", pad(wide))):
        _assert_same_f32(_silu_groups(bits), P.silu_f32(O.bf16_to_f32(bits)), bits, what)
    seven = np.r_[narrow, narrow[:(-len(narrow)) % 7]].reshape(-1, 7)
    forced = np.c_[seven, np.full(len(seven), O.f32_to_bf16(np.float32([100.0]))[0])].ravel()
    _assert_same_f32(_silu_groups(forced), P.silu_f32(O.bf16_to_f32(forced)), forced,
                     "narrow inputs on the division path")


def test_gdn_norm_quant_every_z(gpu_lib):
    """The gated norm over every bf16 gate value z (65536 patterns, shuffled over 11 rows of 48
    heads; the NaN and infinite z in their own rows, since one makes its whole row NaN)."""
    rng = np.random.default_rng(3)
    N = 48 * 128
    allb = np.arange(65536, dtype=np.uint16)
    special = ~np.isfinite(O.bf16_to_f32(allb))
    fin = rng.permutation(allb[~special])
    rows = -(-len(fin) // N)
    z = np.r_[fin, rng.choice(fin, rows * N - len(fin))].reshape(rows, N)
    zs = np.resize(rng.permutation(allb[special]), (2, N))
    zall = np.r_[z, zs].astype(np.uint16)
    M = zall.shape[0]
    x = synthetic.activations(M, N, seed=5)
    w = weight_bits(128, 7, mean=1.0, sd=0.2)
    q, s = gpu_gdn(x, zall, 0, w, 1e-6)
    oq, os_ = P.gdn_norm_quant(x, zall, w, 1e-6)
    assert_same_qs(q, s, oq, os_, "gdn every z")


def test_split_rows_equal_one_workgroup_rows(gpu_lib):
    """The two small-M silu paths on the same device inputs: identical codes and scales, a NaN row
    included (gate values over the whole exp range)."""
    R.ensure_scratch("cuda")
    part, cnt = R._scratch
    M, N = 8, 17408
    gu = synthetic.activations(M, 2 * N, seed=21)
    gu[3, :N] = O.f32_to_bf16(np.linspace(-300, 300, N).astype(np.float32))
    gu[5, 77] = 0x7FC0                                   # NaN gate: a NaN row scale
    runs = {}
    for path in ("split", "one"):
        if path == "one":
            _native.set_scratch(None, 0, cnt.data_ptr(), cnt.numel() * 4)
        try:
            runs[path] = gpu_silu(gu)
        finally:
            _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(),
                                cnt.numel() * 4)
    for a, b in zip(runs["split"], runs["one"]):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
    assert np.isnan(runs["split"][1][5]) and not np.isnan(runs["split"][1][3])


# ---- the custom ops on device tensors, and their hand-off to the GEMM -------------------------
def test_ops_feed_the_gemm_like_the_unfused_chain(gpu_lib):
    """radiance::add_rms_quant -> mxfp4_linear_pq gives the same bits as quantizing the producer's
    bf16 output inside radiance::mxfp4_linear (the unfused chain), and likewise for silu_mul."""
    M, K, N = 16, 5120, 2048
    w, ws = synthetic.weights(N, K, seed=3)
    wq, sq = R.repack_weights(to_dev(w), to_dev(ws))
    wref = R.layout_ref(N, K, wq.device)
    y, res = synthetic.activations(M, K, seed=4), synthetic.activations(M, K, seed=5)
    nw = weight_bits(K, 6)
    q, s, r = torch.ops.radiance.add_rms_quant(bf16_dev(y), bf16_dev(res), bf16_dev(nw), 1e-6)
    fused = torch.ops.radiance.mxfp4_linear_pq(q, s, wq, sq, wref)
    n, orr = P.add_rms_norm(y, res, nw, 1e-6)
    assert np.array_equal(host_u16(r), orr)
    unfused = torch.ops.radiance.mxfp4_linear(bf16_dev(n), wq, sq, wref)
    assert torch.equal(fused, unfused)

    w2, ws2 = synthetic.weights(K, N, seed=7)            # down_proj-like: K_in = N
    wq2, sq2 = R.repack_weights(to_dev(w2), to_dev(ws2))
    wref2 = R.layout_ref(K, N, wq2.device)
    gu = synthetic.activations(M, 2 * N, seed=8)
    q2, s2 = torch.ops.radiance.silu_mul_quant(bf16_dev(gu))
    fused2 = torch.ops.radiance.mxfp4_linear_pq(q2, s2, wq2, sq2, wref2)
    unfused2 = torch.ops.radiance.mxfp4_linear(bf16_dev(P.silu_mul(gu)), wq2, sq2, wref2)
    assert torch.equal(fused2, unfused2)


def test_producer_ops_capture_into_a_hip_graph(gpu_lib):
    """The three ops (silu on its split path: two launches through the registered scratch) in one
    captured graph; every replay, with eager work between, equals the eager results."""
    R.ensure_scratch("cuda")
    M, K, N, heads = 8, 5120, 17408, 48
    y = bf16_dev(synthetic.activations(M, K, seed=31))
    res = bf16_dev(synthetic.activations(M, K, seed=32))
    nw = bf16_dev(weight_bits(K, 33))
    gu = bf16_dev(synthetic.activations(M, 2 * N, seed=34))
    x = bf16_dev(synthetic.activations(M, heads * 128, seed=35))
    z = bf16_dev(synthetic.activations(M, heads * 128, seed=36))
    gw = bf16_dev(weight_bits(128, 37, mean=1.0, sd=0.2))

    def run():
        return (*torch.ops.radiance.add_rms_quant(y, res, nw, 1e-6),
                *torch.ops.radiance.silu_mul_quant(gu),
                *torch.ops.radiance.gdn_norm_quant(x, z, gw, 1e-6))
    eager = [t.clone() for t in run()]
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = run()
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(out, eager):
            assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), f"replay {i}"
        _ = (gu.float() * 2).sum().item()         # unrelated eager work between replays


def test_gdn_op_takes_a_column_slice_of_z(gpu_lib):
    M, heads = 5, 24
    N = heads * 128
    x = synthetic.activations(M, N, seed=1)
    zw = synthetic.activations(M, 3 * N, seed=2)
    w = weight_bits(128, 3, mean=1.0, sd=0.2)
    zd = bf16_dev(zw)
    q, s = torch.ops.radiance.gdn_norm_quant(bf16_dev(x), zd[:, N:2 * N], bf16_dev(w), 1e-6)
    oq, os_ = P.gdn_norm_quant(x, zw[:, N:2 * N], w, 1e-6)
    assert_same_qs(host_u8(q), s.cpu().numpy(), oq, os_, "gdn op on a z slice")


def test_ops_reject_bad_shapes(gpu_lib):
    with pytest.raises(RuntimeError, match="8-aligned"):
        torch.ops.radiance.add_rms_quant(torch.zeros(2, 12, dtype=torch.bfloat16, device="cuda"),
                                         torch.zeros(2, 12, dtype=torch.bfloat16, device="cuda"),
                                         torch.zeros(12, dtype=torch.bfloat16, device="cuda"),
                                         1e-6)
    with pytest.raises(RuntimeError, match="multiple of 128"):
        torch.ops.radiance.gdn_norm_quant(torch.zeros(2, 200, dtype=torch.bfloat16, device="cuda"),
                                          torch.zeros(2, 200, dtype=torch.bfloat16, device="cuda"),
                                          torch.zeros(128, dtype=torch.bfloat16, device="cuda"),
                                          1e-6)
    with pytest.raises(RuntimeError, match="bfloat16"):
        FN.silu_mul_quant(torch.zeros(2, 16, dtype=torch.float32, device="cuda"))
    q, s = FN.silu_mul_quant(torch.zeros(0, 16, dtype=torch.bfloat16, device="cuda"))
    assert q.shape == (0, 8) and s.shape == (0,)
