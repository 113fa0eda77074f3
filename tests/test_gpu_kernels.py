"""GPU parity of the three gfx950 kernels against the oracle, through the C ABI.

Bar: activation codes, per-token scales and repacked bytes bit-exact; bf16 GEMM outputs within the
tolerance in tests/_check.py (rel-L2 <= 1e-3, <= 2 bf16 ulp of the fp32-accumulated reference plus
the fp32 accumulation-order allowance)."""
import functools
import hashlib

import numpy as np
import pytest
import torch

from oracle import mfma_model as MM
from oracle import mxfp4_oracle as O
from tests._check import (HW_ACC_EPS, assert_gemm_close, bf16_dev, gemm_reference, host_u16,
                          host_u8, stream, to_dev)
from vllm_sly_radiance_amd import _native, synthetic

pytestmark = pytest.mark.gpu

SKINNY, TILE, STREAM = _native.KERNEL_SKINNY, _native.KERNEL_TILE, _native.KERNEL_STREAM
RING = _native.KERNEL_RING
RING_AT = _native.KERNEL_RING_AT


@pytest.fixture(scope="module")
def scratch(gpu_lib):
    """Split-K scratch for every plan these tests force (up to 16 splits of 4 M-fragments,
    N <= 36864): far more than the plugin registers, which covers only the automatic plans. The
    plugin's registration, if any, is put back afterwards."""
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    partial = torch.empty(36864 // 16 * 16 * 4 * 64 * 4, dtype=torch.float32, device="cuda")
    counters = torch.zeros(36864 // 16 + 8, dtype=torch.int32, device="cuda")
    _native.set_scratch(partial.data_ptr(), partial.numel() * 4, counters.data_ptr(),
                        counters.numel() * 4)
    yield partial, counters
    torch.cuda.synchronize()
    part, cnt = R._scratch
    if part is None:
        _native.set_scratch(None, 0, None, 0)
    else:
        _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)


@functools.lru_cache(maxsize=4)
def cached_weights(N, K, seed):
    return synthetic.weights(N, K, seed)


def gpu_quant(x_bits, ldx=None):
    M, K = x_bits.shape
    if ldx is None or ldx == K:
        x = bf16_dev(x_bits)
        ldx = K
    else:
        pad = np.zeros((M, ldx), np.uint16)
        pad[:, :K] = x_bits
        x = bf16_dev(pad)
    q = torch.empty((M, K), dtype=torch.uint8, device="cuda")
    s = torch.empty((M,), dtype=torch.float32, device="cuda")
    _native.quant_per_token(x.data_ptr(), ldx, q.data_ptr(), s.data_ptr(), M, K, stream())
    torch.cuda.synchronize()
    return host_u8(q), s.cpu().numpy()


def gpu_repack(w, ws):
    N, K = w.shape[0], w.shape[1] * 2
    wb, sb = _native.packed_bytes(N, K)
    wd, sd = to_dev(w), to_dev(ws)
    wq = torch.empty(wb, dtype=torch.uint8, device="cuda")
    sq = torch.empty(sb, dtype=torch.uint8, device="cuda")
    _native.repack(wd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), N, K, stream())
    return wq, sq


def gpu_gemm(q, s, wq, sq, N, K, kernel=0, variant=-1, split_k=0):
    M = q.shape[0]
    qd, sd = to_dev(q), to_dev(s.astype(np.float32))
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream(), kernel, variant, split_k)
    torch.cuda.synchronize()
    return host_u16(out)


def gpu_gemm_tiled(q, s, wq, sq, N, K, kernel, variant):
    """gpu_gemm on the fragment-tiled bytes of q (oracle tile_q)."""
    M = q.shape[0]
    qd, sd = to_dev(O.tile_q(q)), to_dev(s.astype(np.float32))
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream(), kernel, variant, 1)
    torch.cuda.synchronize()
    return host_u16(out)


def gpu_gemm_tiled_split(q, s, wq, sq, N, K, variant, split):
    M = q.shape[0]
    qd, sd = to_dev(O.tile_q(q)), to_dev(s.astype(np.float32))
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), out.data_ptr(), M, N,
                 K, stream(), _native.KERNEL_TILE_AT, variant, split)
    torch.cuda.synchronize()
    return host_u16(out)


def canon_nan(c):
    return np.where((c & 0x7F) == 0x7F, 0x7F, c)


# ---- (1) quantizer ----------------------------------------------------------------------------
@pytest.mark.parametrize("M,K,ldx", [(1, 5120, None), (8, 5120, None), (17, 1000, None),
                                     (64, 8704, None), (3, 17408, None), (5, 24, None),
                                     (9, 5120, 5128), (7, 640, 641), (1, 40000, None),
                                     (4096, 5120, None), (4096, 8704, None), (300, 5120, None),
                                     (257, 8704, 8712),
                                     (256, 24, None), (261, 10240, None), (256, 10248, None),
                                     (258, 1000, 1001), (16, 16384, None), (100, 12304, None)])
def test_quant_bit_exact(gpu_lib, M, K, ldx):
    x = synthetic.activations(M, K, seed=M * 7 + K)
    q, s = gpu_quant(x, ldx)
    oq, os_ = O.quant_per_token(x)
    assert np.array_equal(s.view(np.uint32), os_.view(np.uint32)), "scales differ"
    bad = np.argwhere(q != oq)
    assert bad.size == 0, f"{len(bad)} codes differ, first at {bad[:3].tolist()}"


def test_quant_special_rows(gpu_lib):
    K = 256
    rows = np.zeros((8, K), np.float32)
    rows[2, 7] = -0.0
    rows[3, :] = np.linspace(-1e-30, 1e-30, K)
    rows[4, :] = np.linspace(-3e38, 3e38, K)
    rows[5, 3] = np.inf
    rows[5, 4] = -2.0
    rows[6, 9] = np.nan
    rows[7, :] = 448.0
    x = O.f32_to_bf16(rows)
    x[2, 7] = 0x8000
    q, s = gpu_quant(x)
    oq, os_ = O.quant_per_token(x)
    assert np.array_equal(np.isnan(s), np.isnan(os_))
    fin = ~np.isnan(os_)
    assert np.array_equal(s[fin].view(np.uint32), os_[fin].view(np.uint32))
    assert np.array_equal(canon_nan(q), canon_nan(oq))
    assert q[2, 7] == 0x80 and q[5, 4] == 0x80       # -0 kept; finite / inf -> -0


def test_quant_special_rows_many(gpu_lib):
    """The special rows again, 33 copies each (264 rows, several workgroups per CU)."""
    K = 256
    rows = np.zeros((8, K), np.float32)
    rows[3, :] = np.linspace(-1e-30, 1e-30, K)
    rows[4, :] = np.linspace(-3e38, 3e38, K)
    rows[5, 3] = np.inf
    rows[5, 4] = -2.0
    rows[6, 9] = np.nan
    rows[7, :] = 448.0
    x = np.tile(O.f32_to_bf16(rows), (33, 1))
    x[2::8, 7] = 0x8000
    q, s = gpu_quant(x)
    oq, os_ = O.quant_per_token(x)
    assert np.array_equal(np.isnan(s), np.isnan(os_)) and np.isnan(s).sum() == 33
    fin = ~np.isnan(os_)
    assert np.array_equal(s[fin].view(np.uint32), os_[fin].view(np.uint32))
    assert np.array_equal(canon_nan(q), canon_nan(oq))
    assert np.all(q[2::8, 7] == 0x80) and np.all(q[5::8, 4] == 0x80)


def test_quant_rounding_ties_and_subnormals(gpu_lib):
    # amax 448 gives scale exactly 1.0, so the codes are the e4m3 rounding of the inputs themselves:
    # every e4m3 value, every tie between neighbours and one bf16 ulp either side of each tie.
    pos = O.e4m3fn_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)
    mb = O.f32_to_bf16(mids).astype(np.uint16)
    vals = np.concatenate([O.f32_to_bf16(pos.astype(np.float32)), mb, mb + 1, mb - 1])
    vals = np.concatenate([vals, vals | 0x8000, [O.f32_to_bf16(np.float32([448.0]))[0]]])
    K = -(-len(vals) // 8) * 8
    row = np.zeros(K, np.uint16)
    row[:len(vals)] = vals
    x = np.stack([row, np.roll(row, 8)]).astype(np.uint16)
    q, s = gpu_quant(x)
    oq, os_ = O.quant_per_token(x)
    assert np.all(s == 1.0) and np.array_equal(s, os_)
    assert np.array_equal(q, oq)


@pytest.mark.parametrize("K", [5120, 8704])
def test_quant_full_size_digest(gpu_lib, K):
    # M=4096 prefill activations of gate_up (K=5120) and down (K=8704): codes and scales hashed
    # and compared with the oracle's
    x = synthetic.activations(4096, K, seed=4096 + (K != 5120))
    q, s = gpu_quant(x)
    oq, os_ = O.quant_per_token(x)
    h = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()
    assert h(q) == h(oq) and h(s) == h(os_)


# ---- (2) repack -------------------------------------------------------------------------------
@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 8704), (48, 5120), (20, 96), (33, 640)])
def test_repack_bit_exact(gpu_lib, N, K):
    w, ws = synthetic.weights(N, K, seed=N + K)
    wq, sq = gpu_repack(w, ws)
    owq, osq = O.repack(w, ws)
    assert np.array_equal(host_u8(wq), owq)
    assert np.array_equal(host_u8(sq), osq)


# ---- (3) GEMM ---------------------------------------------------------------------------------
def one_hot_case(M, N, K, hits):
    """Operands with one nonzero product per hit (m, n, k, code, exp): out[m, n] = value."""
    q = np.zeros((M, K), np.uint8)
    w = np.zeros((N, K // 2), np.uint8)
    ws = np.full((N, K // 32), 127, np.uint8)
    for m, n, k, code, e in hits:
        q[m, k] = 0x38                                  # 1.0
        w[n, k // 2] |= code << (4 * (k & 1))
        ws[n, k // 32] = e
    return q, w, ws


@pytest.mark.parametrize("kernel,variant", [(0, -1), (TILE, 0), (TILE, 2)])
def test_gemm_one_hot_lane_map(gpu_lib, kernel, variant):
    """Single products placed across every lane group, k-block, nibble parity and scale byte: the
    output must light up exactly at (m, n) with E2M1[code] * 2^(e-127). Pins the hardware MFMA
    operand/result layout (oracle/mfma_model.py) and the granule repack on the device."""
    M, N, K = 16, 64, 1024
    rng = np.random.default_rng(5)
    cases = []
    for m in range(16):
        n = (m * 5 + 3) % N
        k = int(rng.integers(0, K))
        cases.append((m, n, k, int(rng.integers(1, 16)), int(rng.integers(120, 134))))
    # distinct rows, columns and k so no two products ever meet in one output
    used_n, used_k, hits = set(), set(), []
    for c in cases:
        if c[1] not in used_n and c[2] not in used_k:
            used_n.add(c[1])
            used_k.add(c[2])
            hits.append(c)
    assert len(hits) >= 12
    q, w, ws = one_hot_case(M, N, K, hits)
    wq, sq = gpu_repack(w, ws)
    out = O.bf16_to_f32(gpu_gemm(q, np.ones(M, np.float32), wq, sq, N, K, kernel, variant))
    expect = np.zeros((M, N), np.float32)
    for m, n, k, code, e in hits:
        expect[m, n] = O.E2M1_VALUES[code] * 2.0 ** (e - 127)
    assert np.array_equal(out, expect), np.argwhere(out != expect)[:5]


def gpu_mfma_tiles(a, b, sa, sb):
    """Raw scaled-MFMA tiles through w4a8_mfma_tile: a [T, 64, 16] fp4 bytes, b [T, 64, 32] fp8
    bytes, sa / sb [T, 64] e8m0 -> [T, 64, 4] fp32 lane registers."""
    T = a.shape[0]
    ad = to_dev(np.ascontiguousarray(a, np.uint8).view(np.int32))
    bd = to_dev(np.ascontiguousarray(b, np.uint8).view(np.int32))
    sad, sbd = to_dev(sa.astype(np.int32)), to_dev(sb.astype(np.int32))
    d = torch.empty((T, 64, 4), dtype=torch.float32, device="cuda")
    assert ad.shape == (T, 64, 4) and bd.shape == (T, 64, 8) and sad.shape == sbd.shape == (T, 64)
    _native.mfma_tile(ad.data_ptr(), bd.data_ptr(), sad.data_ptr(), sbd.data_ptr(), d.data_ptr(), T,
                      stream())
    torch.cuda.synchronize()
    return d.cpu().numpy().astype(np.float64)


def test_mfma_model_matches_hardware_tiles(gpu_lib):
    """The operand/scale/result lane maps of oracle/mfma_model.py against the hardware: random fp4
    and fp8 lanes with random per-lane scales on BOTH operands, so any wrong k pairing, scale-lane
    association or result placement moves outputs by O(their terms); plus exact one-hot tiles for
    the fp8 operand's split runs (k and k + 64) and the scale lanes."""
    rng = np.random.default_rng(17)
    T = 512
    a = rng.integers(0, 256, (T, 64, 16), dtype=np.uint8)
    b = rng.integers(0, 256, (T, 64, 32), dtype=np.uint8)
    b = np.where((b & 0x7F) == 0x7F, 0x38, b).astype(np.uint8)         # no NaN codes
    sa = rng.integers(118, 137, (T, 64))
    sb = rng.integers(118, 137, (T, 64))
    D, Dabs = MM.mfma_tiles_batch(a, b, sa, sb)
    d = gpu_mfma_tiles(a, b, sa, sb)
    # the MFMA truncates inside its accumulation (tests/test_oracle_mfma_precision.py): within
    # HW_ACC_EPS of the sum of |products|, while a wrong pairing or scale moves results by O(1) of it
    err = np.abs(d - D) / np.maximum(Dabs, 1e-300)
    assert np.all(err <= HW_ACC_EPS), f"{int((err > HW_ACC_EPS).sum())} lane results off the model"
    assert np.median(err) < 2.0 ** -14

    # one-hot: B byte (lane lb, byte jb) meets A nibble (row r) at k = model k; scales on both sides
    cases = [(5, 3, 9, 125, 131), (37, 7, 11, 130, 126), (5, 20, 9, 127, 129), (63, 31, 15, 121, 127),
             (16, 16, 0, 128, 120), (47, 0, 4, 133, 127)]
    T1 = len(cases)
    a1 = np.zeros((T1, 64, 16), np.uint8)
    b1 = np.zeros((T1, 64, 32), np.uint8)
    sa1 = np.full((T1, 64), 127)
    sb1 = np.full((T1, 64), 127)
    bk, bc = MM.b_lane_map()
    expect = np.zeros((T1, 16, 16))
    for t, (lb, jb, r, ea, eb) in enumerate(cases):
        k, c = int(bk[lb, jb]), int(bc[lb, jb])
        la, j = (k // 32) * 16 + r, k % 32
        a1[t, la, j // 2] = 0x7 << (4 * (j & 1))                      # 6.0
        b1[t, lb, jb] = 0x40                                          # 2.0
        sa1[t, la] = ea                                               # A scale of (r, k // 32)
        sb1[t, (k // 32) * 16 + c] = eb                               # B scale of (c, k // 32)
        expect[t, r, c] = 12.0 * 2.0 ** (ea - 127) * 2.0 ** (eb - 127)
    d1 = gpu_mfma_tiles(a1, b1, sa1, sb1)
    r_, c_ = MM.d_lane_map()
    assert np.array_equal(d1, expect[:, r_, c_])


def test_mfma_model_matches_device_on_random_granules(gpu_lib):
    """Random codes and scales at one MFMA tile (M=N=16, K=128): the device result equals the
    modeled MFMA (exact float64, then scaled and rounded once)."""
    M, N, K = 16, 16, 128
    rng = np.random.default_rng(9)
    q = rng.integers(0, 256, (M, K), dtype=np.uint8)
    q = np.where((q & 0x7F) == 0x7F, 0x38, q).astype(np.uint8)
    w = rng.integers(0, 256, (N, K // 2), dtype=np.uint8)
    ws = rng.integers(122, 132, (N, K // 32), dtype=np.uint8)
    wq, sq = gpu_repack(w, ws)
    out = gpu_gemm(q, np.ones(M, np.float32), wq, sq, N, K, SKINNY, 0, 1)
    model = MM.gemm_via_granules(q, np.ones(M, np.float32), *O.repack(w, ws), M, N, K)
    assert_gemm_close(out, q, np.ones(M, np.float32), w, ws, "random tile")
    terms = O.gemm_abs_terms(q, np.ones(M, np.float32), w, ws)
    assert np.all(np.abs(O.bf16_to_f32(out) - model) <= 2 * O.bf16_ulp(model) + HW_ACC_EPS * terms)


DECODE_SHAPES = [(5120, 5120), (17408, 5120), (5120, 8704), (10240, 5120), (5120, 6144),
                 (48, 5120), (33, 640), (10240, 96)]


@pytest.mark.parametrize("M", [1, 2, 8, 16, 17, 24, 32, 33, 48, 64])
@pytest.mark.parametrize("N,K", DECODE_SHAPES)
def test_gemm_decode_band_auto_plan(gpu_lib, scratch, M, N, K):
    x = synthetic.activations(M, K, seed=11 * M + K)
    w, ws = cached_weights(N, K, N * 3 + K)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    out = gpu_gemm(q, s, wq, sq, N, K)
    assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} plan={_native.plan(M, N, K)}")


def test_gemm_every_skinny_variant_and_split(gpu_lib, scratch):
    N, K = 1040, 2560                               # 65 n-tiles: ragged against NT=2 and NT=4
    w, ws = synthetic.weights(N, K, seed=77)
    wq, sq = gpu_repack(w, ws)
    for v, (mt, nt, waves, unroll) in enumerate(_native.variants(SKINNY)):
        M = 16 * mt - 3
        x = synthetic.activations(M, K, seed=v)
        q, s = O.quant_per_token(x)
        for ks in (1, 2, 4, 7):
            out = gpu_gemm(q, s, wq, sq, N, K, SKINNY, v, ks)
            assert_gemm_close(out, q, s, w, ws, f"variant {v} {(mt, nt, waves, unroll)} split {ks}")


@pytest.mark.parametrize("N,K", [(17408, 5120), (1040, 2560), (33, 640), (10240, 96), (5120, 6144),
                                 (5120, 8704), (48, 5120)])
def test_gemm_every_stream_variant(gpu_lib, N, K):
    """The streaming family (M <= 16) at every variant that serves (M, N, K), ragged M and N.
    Shapes no variant serves (a run longer than the k-tiles of an n-tile: K=640, K=96) must be
    refused by every variant and planned on another family."""
    w, ws = cached_weights(N, K, N + 7 * K)
    wq, sq = gpu_repack(w, ws)
    served = any(_native.plan(M, N, K)[0] == STREAM for M in (1, 8, 16))
    ran = 0
    for M in (1, 3, 8, 13, 16):
        x = synthetic.activations(M, K, seed=M + K)
        q, s = O.quant_per_token(x)
        for v, cfg in enumerate(_native.variants(STREAM)):
            try:
                out = gpu_gemm(q, s, wq, sq, N, K, STREAM, v, 1)
            except RuntimeError as e:
                assert "does not serve" in str(e)
                continue
            ran += 1
            assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} stream variant {v} {cfg}")
    assert (ran > 0) == served


@pytest.mark.parametrize("N,K", [(17408, 5120), (10240, 5120), (5120, 8704), (1040, 2560)])
def test_stream_eight_rows_equal_the_same_rows_of_sixteen(gpu_lib, N, K):
    """At M <= 8 the streaming kernel loads each k-tile's activation fragment with one load (both
    16-byte runs of the 8 live tokens, the second moved across lanes); above 8 with two. Every
    output column depends on its own token only, with the same sums in the same order, so the
    rows of an M <= 8 call equal the same rows inside an M = 9..16 call bit for bit, at every
    variant that serves the shape."""
    w, ws = cached_weights(N, K, N + 7 * K)
    wq, sq = gpu_repack(w, ws)
    big = synthetic.activations(16, K, seed=N + 1)
    qb, sb = O.quant_per_token(big)
    ran = 0
    for v, cfg in enumerate(_native.variants(STREAM)):
        for M, Mb in [(1, 9), (5, 13), (8, 16)]:
            try:
                ref = gpu_gemm(qb[:Mb], sb[:Mb], wq, sq, N, K, STREAM, v, 1)
            except RuntimeError as e:
                assert "does not serve" in str(e)
                continue
            out = gpu_gemm(qb[:M], sb[:M], wq, sq, N, K, STREAM, v, 1)
            ran += 1
            bad = np.argwhere(out != ref[:M])
            assert bad.size == 0, f"variant {v} {cfg} M={M}: {len(bad)} differ, {bad[:3].tolist()}"
    assert ran > 0


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 8704), (1040, 2560), (33, 640),
                                 (5120, 6144), (10240, 5120), (48, 1056), (2064, 4128)])
def test_gemm_every_ring_variant(gpu_lib, N, K):
    """The pipelined streaming family at every variant that serves (M, N, K): M up to each
    variant's fragments (ragged), N ragged against the n-tile shares, K ending inside a k-tile
    (1056) or a k-group (640, 4128), ranges whose last round is padded. A variant that does not
    serve a shape (n-tiles per workgroup beyond NT, fewer k-tiles than waves) must refuse it.
    Where K % 128 == 0 the same variant on the fragment-tiled codes (kernel RING_AT) must give the
    same bits."""
    w, ws = cached_weights(N, K, N + 5 * K)
    wq, sq = gpu_repack(w, ws)
    ran = 0
    for M in (1, 5, 16, 17, 33, 48, 64):
        x = synthetic.activations(M, K, seed=3 * M + K)
        q, s = O.quant_per_token(x)
        for v, cfg in enumerate(_native.variants(RING)):
            if M > 16 * cfg[0]:
                continue
            print(f"[ring] M={M} N={N} K={K} variant {v} {cfg}", flush=True)
            try:
                out = gpu_gemm(q, s, wq, sq, N, K, RING, v, 1)
            except RuntimeError as e:
                assert "does not serve" in str(e)
                continue
            ran += 1
            assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} ring variant {v} {cfg}")
            if K % 128 == 0:
                out_at = gpu_gemm_tiled(q, s, wq, sq, N, K, RING_AT, v)
                assert np.array_equal(out_at, out), f"M={M} N={N} K={K} ring variant {v} tiled"
    assert ran > 0


# K = 640, 96 and 1056 end inside a k-group: the k-loop runs whole k-groups over zero slabs
@pytest.mark.parametrize("M,N,K", [(65, 544, 1024), (300, 1040, 2560), (1000, 17408 // 8, 5120),
                                   (129, 33, 640), (513, 5120, 8704), (70, 200, 96),
                                   (257, 300, 1056)])
def test_gemm_every_tile_variant(gpu_lib, M, N, K):
    x = synthetic.activations(M, K, seed=M)
    w, ws = synthetic.weights(N, K, seed=N)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    for v, cfg in enumerate(_native.variants(TILE)):
        out = gpu_gemm(q, s, wq, sq, N, K, TILE, v)
        assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} tile variant {v} {cfg}")


@pytest.mark.parametrize("M,N,K", [(4000, 5104, 1024), (2100, 4800, 2048)])
def test_gemm_tile_variants_agree_bitwise(gpu_lib, M, N, K):
    """More tiles than CUs (several rounds of workgroups), with a ragged last row block and, for
    N=5104, a ragged last column block; 270 tiles is not a multiple of the 8-XCD interleave. Every
    tile variant accumulates each output's k-tiles in the same order into one fp32 chain, so all
    of them must agree bit for bit; the first is checked against the oracle."""
    x = synthetic.activations(M, K, seed=M + 1)
    w, ws = synthetic.weights(N, K, seed=N + 1)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    cfgs = _native.variants(TILE)
    first = None
    for v, cfg in enumerate(cfgs):
        print(f"[tile] M={M} N={N} K={K} variant {v} {cfg}", flush=True)
        out = gpu_gemm(q, s, wq, sq, N, K, TILE, v)
        if first is None:
            assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} tile variant {v} {cfg}")
            first = out
        else:
            bad = np.argwhere(out != first)
            assert bad.size == 0, \
                f"tile variant {v} {cfg}: {len(bad)} outputs differ from variant 0, first {bad[:3]}"


@pytest.mark.parametrize("N,K", [(17408, 5120), (5120, 8704)])
def test_gemm_prefill_4096_sampled_rows(gpu_lib, N, K):
    """M=4096 prefill GEMMs (gate_up, down): every output column, 192 sampled token rows checked
    against the oracle (the oracle's full fp32 GEMM is minutes of CPU)."""
    M = 4096
    x = synthetic.activations(M, K, seed=K)
    w, ws = synthetic.weights(N, K, seed=N)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    out = gpu_gemm(q, s, wq, sq, N, K)
    rows = np.unique(np.concatenate([np.random.default_rng(1).choice(M, 190, replace=False),
                                     [0, M - 1]]))
    assert_gemm_close(out[rows], q[rows], s[rows], w, ws, f"M=4096 N={N} K={K}")


def test_gemm_full_size_exact_properties(gpu_lib, scratch):
    """Size-independent checks at the verify-decode and prefill shapes: doubling every token scale
    doubles every output bit-exactly, and permuting tokens permutes output rows bit-exactly."""
    N, K = 17408, 5120
    w, ws = synthetic.weights(N, K, seed=1)
    wq, sq = gpu_repack(w, ws)
    for M in (8, 4096):
        x = synthetic.activations(M, K, seed=M + 1)
        q, s = O.quant_per_token(x)
        y1 = gpu_gemm(q, s, wq, sq, N, K)
        y2 = gpu_gemm(q, s * np.float32(2.0), wq, sq, N, K)
        assert np.array_equal(O.bf16_to_f32(y2), 2 * O.bf16_to_f32(y1))
        perm = np.random.default_rng(M).permutation(M)
        y3 = gpu_gemm(q[perm], s[perm], wq, sq, N, K)
        assert np.array_equal(y3, y1[perm])


def test_split_k_reduction_has_no_race(gpu_lib, scratch):
    """Race detector for the cross-workgroup split-K reduction (the reference's
    sly/mxfp4/check_decode_splitk.py): two inputs alternate back to back with no synchronization,
    so a partial read before its writer's release is a wrong value; every output must equal its
    golden bit for bit."""
    N, K = 1024, 8704
    w, ws = synthetic.weights(N, K, seed=3)
    wq, sq = gpu_repack(w, ws)
    v = [i for i, c in enumerate(_native.variants(SKINNY)) if c[:3] == (1, 1, 16)][0]
    ins = []
    for j in range(2):
        q, s = O.quant_per_token(synthetic.activations(8, K, seed=50 + j))
        ins.append((to_dev(q), to_dev(s)))
    for ks in (2, 4, 8, 16):
        gold = []
        for qd, sd in ins:
            g = torch.empty((8, N), dtype=torch.bfloat16, device="cuda")
            _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(), g.data_ptr(),
                         8, N, K, stream(), SKINNY, v, ks)
            torch.cuda.synchronize()
            gold.append(g)
        outs = [torch.empty((64, 8, N), dtype=torch.bfloat16, device="cuda") for _ in range(2)]
        for b in range(64):
            for j, (qd, sd) in enumerate(ins):
                _native.gemm(qd.data_ptr(), sd.data_ptr(), wq.data_ptr(), sq.data_ptr(),
                             outs[j][b].data_ptr(), 8, N, K, stream(), SKINNY, v, ks)
        torch.cuda.synchronize()
        for j in range(2):
            miss = int((outs[j] != gold[j]).flatten(1).any(1).sum())
            assert miss == 0, f"split {ks}: {miss}/64 launches differ from golden {j}"


@pytest.mark.parametrize("M,N,K", [(17, 5120, 8704), (40, 1040, 2080), (64, 256, 8704),
                                   (33, 48, 1056), (20, 5120, 6144)])
def test_gemm_tile_k_split(gpu_lib, scratch, M, N, K):
    """The tile kernel with K split over workgroup rows (fp32 partials, then the reducing launch)
    at the band's tile shapes and 2..6 splits: K ending inside a k-tile (1056) or a k-group (2080),
    so the last split runs zero slabs; N ragged against the tile (1040, 48). Against the oracle, and
    the row-major and fragment-tiled activations give the same bits."""
    x = synthetic.activations(M, K, seed=M + K)
    w, ws = cached_weights(N, K, N + 7 * K)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    ref = gemm_reference(q, s, w, ws)
    kg = -(-K // 512)
    ran = 0
    for v, (wm, wn, bm, bn) in enumerate(_native.variants(TILE)):
        cfg = _native.tile_config(v)
        if cfg["waves"] != 4 or wm > 2:
            # only the 4-wave band tiles have a K-split form; the others refuse one
            with pytest.raises(RuntimeError, match="no K-split form"):
                gpu_gemm(q, s, wq, sq, N, K, TILE, v, 2)
            continue
        # every split count on the band plan's two tiles, three splits on the others
        full = cfg["stages"] in (5, 8) and bn == 64
        for split in (range(2, min(6, kg) + 1) if full else (min(3, kg),)):
            print(f"[tile split] M={M} N={N} K={K} variant {v} ({bm}x{bn}) split {split}",
                  flush=True)
            out = gpu_gemm(q, s, wq, sq, N, K, TILE, v, split)
            ran += 1
            assert_gemm_close(out, q, s, w, ws, f"M={M} N={N} K={K} tile {v} split {split}", ref)
            if K % 128 == 0 and split == min(3, kg):
                out_at = gpu_gemm_tiled_split(q, s, wq, sq, N, K, v, split)
                assert np.array_equal(out_at, out), f"tiled split {v}"
    assert ran > 0


def test_band_split_plan_for_down(gpu_lib):
    """With the plugin's scratch registered, the automatic plan splits down (5120 x 8704) three
    ways at M = 17..48 on the 32 x 64 (8-stage) / 64 x 64 (5-stage) tiles, not at M = 64; o_proj
    (5120 x 6144, 12 k-groups) at M = 17..20 only; never qkv or gate_up."""
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    R.ensure_scratch("cuda")
    assert _native.plan(64, 5120, 8704)[2] == 1
    for M in (17, 24, 32, 33, 48):
        k, v, sp = _native.plan(M, 5120, 8704)
        want = (32, 64, 8) if M <= 32 else (64, 64, 5)
        c = _native.tile_config(v)
        assert (k, sp, c["bm"], c["bn"], c["stages"]) == (TILE, 3, *want), (M, k, v, sp, c)
        for N, K in ((10240, 5120), (17408, 5120)):
            assert _native.plan(M, N, K)[2] == 1, (M, N, K)
        assert _native.plan(M, 5120, 6144)[2] == (3 if M <= 20 else 1), M
    assert _native.plan(20, 5120, 6144)[2] == 3 and _native.plan(21, 5120, 6144)[2] == 1


# ---- diagnostics --------------------------------------------------------------------------------
MODEL_SHAPES = [(10240, 5120), (5120, 6144), (17408, 5120), (5120, 8704)]


def test_plugin_scratch_covers_every_automatic_plan(gpu_lib):
    """The scratch the plugin registers (w4a8_workspace_bytes for M <= 64, N <= 36864) lets the
    automatic plan take every split it would take with unlimited room: the plans agree on the
    Qwen3.8-27B linear shapes, and on every N up to 2048 at K = 1056 and 4128 (K not a multiple
    of 512: the streaming kernel cannot serve them, so the decode band splits K across workgroups
    when N is small), at every M of the decode band."""
    from vllm_sly_radiance_amd import radiance_mxfp4 as R
    R.ensure_scratch("cuda")
    part, cnt = R._scratch
    assert part.numel() * 4 < 8 << 20, "the plugin scratch should be a few MB at most"
    big_p = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
    big_c = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    shapes = MODEL_SHAPES + [(n, k) for n in range(16, 2049, 16) for k in (1056, 4128)]
    ms = list(range(1, 65))
    try:
        plans = {}
        _native.set_scratch(big_p.data_ptr(), big_p.numel(), big_c.data_ptr(), big_c.numel() * 4)
        for N, K in shapes:
            for M in ms:
                plans[(M, N, K)] = _native.plan(M, N, K)
        _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)
        differ = [(key, plans[key], _native.plan(*key)) for key in plans
                  if _native.plan(*key) != plans[key]]
        assert not differ, differ[:5]
        assert any(p[2] > 1 for p in plans.values()), "no split plan was exercised"
    finally:
        _native.set_scratch(part.data_ptr(), part.numel() * 4, cnt.data_ptr(), cnt.numel() * 4)


def test_read_probe_shapes_read_without_writing(gpu_lib):
    """Every read-probe variant at a grid it covers, over the verify GEMM's byte count and a short
    ragged buffer: it runs, and with data that never xors to its pattern it writes nothing."""
    for nbytes in (47_669_280, 5000):
        buf = torch.full((nbytes + 16,), 3, dtype=torch.uint8, device="cuda")
        out = torch.zeros(2, dtype=torch.int32, device="cuda")
        for v, (waves, units, window, nt) in enumerate(_native.read_probe_variants()):
            blocks = -(-nbytes // (waves * units * 1024))     # the fewest workgroups that cover it
            print(f"[probe] read shape v={v} blocks={blocks} {nbytes} B", flush=True)
            _native.read_probe_shape(buf.data_ptr(), nbytes, out.data_ptr(), blocks, v, stream())
        torch.cuda.synchronize()
        assert out.cpu().tolist() == [0, 0]


@pytest.mark.parametrize("nbytes", [1000, 204800, 47_669_280])
def test_read_probe_reads_without_writing(gpu_lib, nbytes):
    """The HBM read probe over buffers shorter than, equal to and longer than one workgroup's
    share: it runs, and with data that never xors to its pattern it writes nothing."""
    buf = torch.full((nbytes + 16,), 3, dtype=torch.uint8, device="cuda")
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    print(f"[probe] read {nbytes} B", flush=True)
    _native.read_probe(buf.data_ptr(), nbytes, out.data_ptr(), stream())
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [0, 0]


@pytest.mark.parametrize("M,N,K", [(8, 17408, 5120), (1, 10240, 5120), (8, 5120, 8704),
                                   (4, 5120, 6144), (3, 1000, 1024)])
def test_stream_load_probe_runs_without_writing(gpu_lib, M, N, K):
    """The streaming GEMM's loads alone, each load set, on operands of the GEMM's own sizes (zero
    data never xors to the pattern): it runs and writes nothing; a shape the plan does not stream
    is refused."""
    assert _native.plan(M, N, K)[0] == _native.KERNEL_STREAM
    wb, sb = _native.packed_bytes(N, K)
    q = torch.zeros((M, K), dtype=torch.uint8, device="cuda")
    s = torch.ones(M, dtype=torch.float32, device="cuda")
    wq = torch.zeros(wb, dtype=torch.uint8, device="cuda")
    sq = torch.zeros(sb, dtype=torch.uint8, device="cuda")
    out = torch.zeros(2, dtype=torch.int32, device="cuda")
    for parts in (_native.STREAM_LOADS_WEIGHTS, _native.STREAM_LOADS_SCALES,
                  _native.STREAM_LOADS_ALL):
        print(f"[probe] stream loads M={M} N={N} K={K} parts={parts}", flush=True)
        _native.stream_load_probe(q.data_ptr(), s.data_ptr(), wq.data_ptr(), sq.data_ptr(), M, N,
                                  K, parts, out.data_ptr(), stream())
    torch.cuda.synchronize()
    assert out.cpu().tolist() == [0, 0]
    with pytest.raises(RuntimeError, match="not the streaming GEMM"):
        _native.stream_load_probe(q.data_ptr(), s.data_ptr(), wq.data_ptr(), sq.data_ptr(), M, 33,
                                  640, 7, out.data_ptr(), stream())


def random_shapes(count, seed):
    """Seeded (M, N, K): M over the decode, skinny and tile bands, ragged N, K any multiple of 32."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        M = int(rng.choice([rng.integers(1, 17), rng.integers(17, 65), rng.integers(65, 700)]))
        N = int(rng.integers(1, 2600))
        K = int(32 * rng.integers(1, 97))
        out.append((M, N, K))
    return out


@pytest.mark.parametrize("M,N,K", random_shapes(18, 2024) + [
    (17, 5120, 6144), (21, 5120, 8704), (19, 2048, 1024), (20, 4000, 544)])
def test_gemm_random_shapes_planned(gpu_lib, M, N, K):
    """The automatic plan on seeded random shapes, every output against the oracle; the last four
    sit just above the streaming band (M = 17 .. 21, N = 2048 .. 5120), where the plan takes the
    decode-band tiles (with the K split for the down-shaped one)."""
    x = synthetic.activations(M, K, seed=M * 31 + K)
    w, ws = synthetic.weights(N, K, seed=N * 7 + K)
    q, s = O.quant_per_token(x)
    wq, sq = gpu_repack(w, ws)
    plan = _native.plan(M, N, K)
    print(f"[random] M={M} N={N} K={K} plan {plan}", flush=True)
    out = gpu_gemm(q, s, wq, sq, N, K)
    assert_gemm_close(out, q, s, w, ws, f"random M={M} N={N} K={K} plan {plan}")


NAN_SCALES = [0x7FC00000, 0xFFC00000, 0x7FC12345, 0xFFFFFFFF, 0x7F800001]


@pytest.mark.parametrize("M,N,K,kernel,variant,split,path", [
    (8, 512, 1024, 0, -1, 0, "stream"),
    (40, 17408, 5120, 0, -1, 0, "band"),
    (256, 1024, 1024, TILE, 2, 1, "tile, full tiles (staged stores)"),
    (200, 1000, 1024, TILE, 2, 1, "tile, edge tiles (direct stores)"),
    (24, 5120, 8704, 0, -1, 0, "tile K split + reduce"),
])
def test_nan_token_scales_give_canonical_nan_rows(gpu_lib, M, N, K, kernel, variant, split, path):
    """A NaN token scale (any payload, either sign, quiet or signalling) makes its whole output row
    the canonical bf16 NaN 0x7FC0 | sign on every epilogue (the hardware convert plus the packed
    minimum, or the software rounding); the other rows stay finite."""
    w, ws = synthetic.weights(N, K, seed=M + 1)
    wq, sq = gpu_repack(w, ws)
    q, s = O.quant_per_token(synthetic.activations(M, K, seed=M + 2))
    s = s.astype(np.float32).copy()
    rows = [(3 * i + 1) % M for i in range(len(NAN_SCALES))]
    for r, bits in zip(rows, NAN_SCALES):
        s.view(np.uint32)[r] = bits
    print(f"[kernels] NaN token scales, {path}, M={M} N={N} K={K}", flush=True)
    c = gpu_gemm(q, s, wq, sq, N, K, kernel, variant, split)
    if kernel == 0:
        assert _native.plan(M, N, K)[0] == {"stream": STREAM, "band": _native.KERNEL_BAND}.get(
            path, TILE), _native.plan(M, N, K)
    for r, bits in zip(rows, NAN_SCALES):
        want = 0x7FC0 | ((bits >> 16) & 0x8000)
        assert (c[r] == want).all(), (path, r, hex(bits), np.unique(c[r])[:4])
    others = np.setdiff1d(np.arange(M), rows)
    assert not np.isnan(O.bf16_to_f32(c[others])).any()
