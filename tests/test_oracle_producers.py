"""Pins of the fused-producer oracle (CPU).

oracle/producers_oracle.py restates the reference's add_rms_quant, silu_mul_quant and
gdn_norm_quant with every floating-point step fixed. Each piece is checked here against something
other than itself: float64 numpy for exp and silu; float64 sums and plain scalar loops for the
fixed-order sums of squares; the reference's native chains (m_add_rms / m_silu / m_gdn,
sly/check_fused_norm.py:119-136) evaluated by torch's CPU kernels for the producers; closed forms."""
import math
import os

import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P
from vllm_sly_radiance_amd import synthetic

F32 = np.float32


def ulps(a, ref):
    """|a - ref| in units of fp32 spacing at ref (float64 ref)."""
    a = np.asarray(a, dtype=np.float64)
    sp = np.spacing(np.abs(ref).astype(F32)).astype(np.float64)
    return np.abs(a - ref) / sp


def fma_triples(n, seed):
    """Edge cases (signed zeros, subnormals, infinities, NaN, overflow), random triples with c near
    -a*b (cancellation), and double-rounding traps: a = 1 + i 2^-12, b = 1 + j 2^-12 with i j odd
    make a*b an fp32 midpoint exactly, and c = +-2^-e (e = 60..100) moves the exact sum off it by
    less than a float64 ulp, so float64 arithmetic alone rounds such triples the wrong way."""
    rng = np.random.default_rng(seed)
    sp = np.array([0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 1.17549435e-38, 3.4028235e38, -3.4028235e38,
                   np.inf, -np.inf, np.nan, 0.5, 2.0 ** -24, 1.0 + 2.0 ** -23, 3.0, 1.0 / 3.0],
                  np.float32)
    edge = np.stack(np.meshgrid(sp, sp, sp, indexing="ij"), -1).reshape(-1, 3)
    a = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    b = rng.integers(0, 2 ** 32, n, dtype=np.uint64).astype(np.uint32).view(np.float32)
    a = np.ldexp(np.frexp(np.where(np.isfinite(a), a, 1.5))[0], rng.integers(-60, 60, n))
    b = np.ldexp(np.frexp(np.where(np.isfinite(b), b, -0.75))[0], rng.integers(-60, 60, n))
    prod = a.astype(np.float64) * b.astype(np.float64)
    c = -prod * np.ldexp(1.0, rng.integers(-30, 30, n)) * rng.choice([1.0, 1.0 + 2.0 ** -23, 0.5], n)
    with np.errstate(over="ignore"):
        rand = np.stack([a, b, c], 1).astype(np.float32)          # some c overflow to +-inf
    i = 2 * rng.integers(0, 2048, n) + 1
    j = 2 * rng.integers(0, 2048, n) + 1
    e2 = rng.integers(-20, 20, n)
    ta = np.ldexp(1.0 + i * 2.0 ** -12, e2)
    tb = 1.0 + j * 2.0 ** -12
    tc = np.ldexp(rng.choice([1.0, -1.0], n), e2 - rng.integers(60, 100, n))
    traps = np.stack([ta, tb, tc], 1).astype(np.float32)
    return np.concatenate([edge, rand, traps]).astype(np.float32)


def test_fma_emulation_matches_c_fmaf(tmp_path):
    import shutil
    import subprocess
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / "fpid")
    subprocess.run([gcc, "-O2", "-ffp-contract=off", "-fopenmp",
                    os.path.join(os.path.dirname(__file__), "fp_identities.c"), "-o", exe, "-lm"],
                   check=True)
    tr = fma_triples(200_000, 7)
    out = subprocess.run([exe, "fma"], input=tr.tobytes(), capture_output=True, check=True).stdout
    want = np.frombuffer(out, np.float32)
    got = P.fma_f32(tr[:, 0], tr[:, 1], tr[:, 2])
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    bad = np.flatnonzero(~same)
    assert bad.size == 0, f"{bad.size} differ, first {tr[bad[:3]]} -> {got[bad[:3]]} vs {want[bad[:3]]}"
    # the emulation is not plain float64 arithmetic: some triples round differently
    with np.errstate(over="ignore", invalid="ignore"):
        plain = (tr[:, 0].astype(np.float64) * tr[:, 1] + tr[:, 2]).astype(np.float32)
    assert np.count_nonzero(plain.view(np.uint32) != want.view(np.uint32)) > 0


def test_exp_within_two_ulp_of_float64():
    y = np.linspace(-103.0, 88.7, 3_000_001).astype(F32)
    y = np.concatenate([y, (np.random.default_rng(0).standard_normal(1_000_000) * 8).astype(F32)])
    e = P.exp_f32(y)
    ref = np.exp(y.astype(np.float64))
    norm = ref > 1.2e-38
    assert ulps(e[norm], ref[norm]).max() <= 2.0


def test_exp_special_values():
    y = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1.0, -1.0, 88.72284, 88.7229, -103.97208,
                  -104.0, 1e-8], F32)
    e = P.exp_f32(y)
    assert e[0] == 1.0 and e[1] == 1.0
    assert np.isposinf(e[2]) and e[3] == 0.0 and np.isnan(e[4])
    assert abs(float(e[5]) - math.e) <= 2 * np.spacing(F32(math.e))
    assert np.isposinf(e[7]) or e[7] > 3.4e38       # the last finite fp32 neighbourhood
    assert np.isposinf(e[8])
    assert e[9] <= np.float32(2.0 ** -149) and e[10] == 0.0
    assert e[11] == 1.0


def test_exp_exact_at_integer_multiples_of_ln2():
    # y = n ln 2 exactly representable? No; but e^(n * fl32(ln2)) must stay within 1 ulp of 2^n
    n = np.arange(-120, 120)
    y = (n * F32(math.log(2))).astype(F32)
    e = P.exp_f32(y)
    ref = np.exp(y.astype(np.float64))
    assert ulps(e, ref).max() <= 1.0


def test_silu_within_four_ulp_of_float64():
    x = np.linspace(-90.0, 90.0, 2_000_001).astype(F32)
    s = P.silu_f32(x)
    x64 = x.astype(np.float64)
    ref = x64 / (1.0 + np.exp(-x64))
    # below x = -88.72, 1 + e^-x overflows fp32 and the fp32 formula (the reference's too) gives -0
    # for a true value under 1e-36 in magnitude
    m = (x > -88.72) & (np.abs(ref) > 1e-37)
    assert ulps(s[m], ref[m]).max() <= 4.0
    tail = x <= -88.72
    assert np.all(np.abs(s[tail].astype(np.float64) - ref[tail]) <= 1e-36)
    sp = P.silu_f32(np.array([0.0, -0.0, np.inf, np.nan, -200.0, 200.0], F32))
    assert sp[0] == 0.0 and sp[1] == 0.0 and np.signbit(sp[1])
    assert np.isposinf(sp[2]) and np.isnan(sp[3])
    assert sp[4] == 0.0 and np.signbit(sp[4]) and sp[5] == 200.0


def scalar_row_sum(v):
    """The fixed order, written as plain scalar Python loops over fp32 values."""
    K = len(v)
    kv = K // 8
    part = [F32(0)] * P.THREADS
    for t in range(P.THREADS):
        g = t
        while g < kv:
            for j in range(8):
                x = v[g * 8 + j]
                part[t] = F32(part[t] + F32(x * x))
            g += P.THREADS
    waves = []
    for w in range(P.THREADS // 64):
        lane = part[w * 64:(w + 1) * 64]
        for o in (32, 16, 8, 4, 2, 1):
            lane = [F32(lane[i] + lane[i ^ o]) for i in range(64)]
        waves.append(lane[0])
    tot = waves[0]
    for w in waves[1:]:
        tot = F32(tot + w)
    return tot


@pytest.mark.parametrize("K,seed", [(8, 0), (2056, 1), (5120, 2)])
def test_row_sum_squares_fixed_order(K, seed):
    v = (np.random.default_rng(seed).standard_normal((2, K)) * 3).astype(F32)
    got = P.row_sum_squares(v)
    for r in range(2):
        assert got[r] == scalar_row_sum(list(v[r]))
        exact = float(np.sum(v[r].astype(np.float64) ** 2))
        # a sum of K positive terms in fp32: |error| <= (K + log2 K) * 2^-24 * exact
        assert abs(float(got[r]) - exact) <= (K + 16) * 2.0 ** -24 * exact


def test_head_sum_squares_fixed_order():
    v = (np.random.default_rng(3).standard_normal((3, 384)) * 2).astype(F32)
    got = P.head_sum_squares(v)
    for r in range(3):
        for h in range(3):
            seg = v[r, h * 128:(h + 1) * 128]
            part = []
            for lane in range(16):
                p = F32(0)
                for j in range(8):
                    x = seg[lane * 8 + j]
                    p = F32(p + F32(x * x))
                part.append(p)
            for o in (8, 4, 2, 1):
                part = [F32(part[i] + part[i ^ o]) for i in range(16)]
            assert got[r, h] == part[0]
            exact = float(np.sum(seg.astype(np.float64) ** 2))
            assert abs(float(got[r, h]) - exact) <= 160 * 2.0 ** -24 * exact


def torch_bf16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16)


def bits_of(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def within_one_bf16(a_bits, b_bits):
    """Same value, or adjacent bf16 values (one rounding apart); NaN only with NaN."""
    a = O.bf16_to_f32(a_bits).astype(np.float64)
    b = O.bf16_to_f32(b_bits).astype(np.float64)
    both_nan = np.isnan(a) & np.isnan(b)
    ok = both_nan | (a == b) | (np.abs(a - b) <= np.maximum(O.bf16_ulp(a), O.bf16_ulp(b)))
    return bool(ok.all())


@pytest.mark.parametrize("M,K,seed", [(4, 5120, 0), (3, 2048, 1), (2, 8, 2), (5, 10240, 3)])
def test_add_rms_matches_native_chain(M, K, seed):
    y = synthetic.activations(M, K, seed)
    res = synthetic.activations(M, K, seed + 100)
    w = O.f32_to_bf16((np.random.default_rng(seed).standard_normal(K) * 0.1).astype(F32))
    eps = 1e-6
    n, r = P.add_rms_norm(y, res, w, eps)
    # m_add_rms (sly/check_fused_norm.py:119-123) on torch's CPU kernels
    x = torch_bf16(y).float() + torch_bf16(res).float()
    rr = x.to(torch.bfloat16)
    out = (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
           * (torch_bf16(w).float() + 1.0)).to(torch.bfloat16)
    assert np.array_equal(r, bits_of(rr))
    assert within_one_bf16(n, bits_of(out))
    q, s, r2 = P.add_rms_quant(y, res, w, eps)
    oq, os_ = O.quant_per_token(n)
    assert np.array_equal(q, oq) and np.array_equal(s, os_) and np.array_equal(r2, r)


def test_add_rms_closed_forms():
    K = 1024
    y = np.zeros((3, K), np.uint16)
    res = np.zeros((3, K), np.uint16)
    c = O.f32_to_bf16(np.full(K, 0.5, F32))
    y[1] = c                                            # a row of equal values 0.5
    y[2] = c
    w = np.zeros(K, np.uint16)                          # weight 0 -> factor (w + 1) = 1
    n, r = P.add_rms_norm(y, res, w, 0.0)
    assert np.isnan(O.bf16_to_f32(n[0])).all()          # zero row, eps 0: 0 * (1 / sqrt(0)) = NaN,
    assert not np.isnan(O.bf16_to_f32(n[1:])).any()     # as 0 * rsqrt(0) is in the reference
    n, r = P.add_rms_norm(y, res, w, 1e-6)
    assert not O.bf16_to_f32(n[0]).any()
    expect = 0.5 / math.sqrt(0.25 + 1e-6)
    assert np.all(np.abs(O.bf16_to_f32(n[1]) - expect) <= O.bf16_ulp(np.float64(expect)))
    wneg = O.f32_to_bf16(np.full(K, -1.0, F32))         # w = -1 -> every output 0
    n, _ = P.add_rms_norm(y, res, wneg, 1e-6)
    assert not O.bf16_to_f32(n).any()
    q, s, _ = P.add_rms_quant(y[:1], res[:1], w, 1e-6)
    assert s[0] == O.MIN_SCALE and not q.any()


@pytest.mark.parametrize("M,N,seed", [(4, 17408, 0), (3, 1024, 1), (2, 8, 2)])
def test_silu_mul_matches_native_chain(M, N, seed):
    gu = synthetic.activations(M, 2 * N, seed)
    p = P.silu_mul(gu)
    t = torch_bf16(gu)
    ref = torch.nn.functional.silu(t[:, :N]) * t[:, N:]          # m_silu, bf16 in and out
    assert within_one_bf16(p, bits_of(ref))
    q, s = P.silu_mul_quant(gu)
    oq, os_ = O.quant_per_token(p)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)


def test_silu_mul_special_values():
    g = np.array([0.0, -0.0, 100.0, -100.0, np.inf, np.nan, 1.0, -1.0], F32)
    u = np.array([2.0, 2.0, 1.0, 1.0, 1.0, 1.0, 0.0, 3.0], F32)
    gu = np.concatenate([O.f32_to_bf16(g), O.f32_to_bf16(u)])[None, :]
    p = O.bf16_to_f32(P.silu_mul(gu))[0]
    assert p[0] == 0 and p[1] == 0 and p[2] == 100.0 and p[3] == 0
    assert np.isposinf(p[4]) and np.isnan(p[5]) and p[6] == 0
    s1 = 1.0 / (1.0 + math.exp(1.0))                    # silu(-1) = -1 * sigmoid(-1)
    assert abs(p[7] - (-3.0 * s1)) <= 2 * O.bf16_ulp(np.float64(3.0 * s1))


@pytest.mark.parametrize("M,heads,seed", [(3, 24, 0), (2, 1, 1), (4, 80, 2)])
def test_gdn_norm_matches_native_chain(M, heads, seed):
    N = heads * 128
    x = synthetic.activations(M, N, seed)
    z = synthetic.activations(M, N, seed + 7)
    w = O.f32_to_bf16((1.0 + np.random.default_rng(seed).standard_normal(128) * 0.2).astype(F32))
    eps = 1e-6
    n = P.gdn_norm(x, z, w, eps)
    # m_gdn (sly/check_fused_norm.py:131-136)
    xt = torch_bf16(x).reshape(-1, 128).float()
    zt = torch_bf16(z).reshape(-1, 128).float()
    out = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + eps) * torch_bf16(w).float()
    ref = (out * torch.nn.functional.silu(zt)).to(torch.bfloat16).reshape(M, -1)
    assert within_one_bf16(n, bits_of(ref))
    q, s = P.gdn_norm_quant(x, z, w, eps)
    oq, os_ = O.quant_per_token(n)
    assert np.array_equal(q, oq) and np.array_equal(s, os_)


def test_gdn_heads_are_independent():
    """Scaling one head's x leaves the other heads' normalized values unchanged (per-head norm)."""
    M, N = 2, 512
    x = synthetic.activations(M, N, 9)
    z = synthetic.activations(M, N, 10)
    w = O.f32_to_bf16(np.ones(128, F32))
    n0 = P.gdn_norm(x, z, w, 1e-6)
    x2 = x.copy()
    x2[:, 128:256] = O.f32_to_bf16(O.bf16_to_f32(x[:, 128:256]) * 4)    # exact in bf16
    n1 = P.gdn_norm(x2, z, w, 1e-6)
    keep = np.r_[0:128, 256:512]
    assert np.array_equal(n0[:, keep], n1[:, keep])
    # the scaled head: x * 4 / (4 * rms) = the same up to the eps term and rounding
    assert within_one_bf16(n0[:, 128:256], n1[:, 128:256])
