"""Inputs on which the producers' fixed summation orders decide the output.

The fused producers sum squares in one fixed order (the oracle's row_sum_squares and
head_sum_squares): add-RMSNorm per thread over its groups element by element, an xor butterfly over
the 64 lanes of a wave (32, 16, 8, 4, 2, 1), the four waves in order; the gated norm per lane over
its 8 elements, then a 16-lane xor butterfly (8, 4, 2, 1). On random rows another order changes
the sum's last bits only now and then, and the quantized output almost never: the norm scales the
whole row, and the per-token scale divides it out again. So a kernel that paired its lanes
differently would still pass bit-exact tests on random data.

The cases here are built so that it would not. Each row has element magnitudes spread over 13
binades (rounding then depends on which partial sums meet), and one element far above the rest,
which sets the row's maximum and so its scale. The weight (and for the gated norm the gate z) of
that element is then chosen among bf16 values so that its bf16 output rounds one way with the
oracle's sum and the other way with an alternative order's. The row scale, and with it the codes,
then differ between the orders. Every case is checked to tell apart the oracle's order from the
alternatives it names; tests/test_orders_cpu.py checks that on the CPU, and the GPU tests compare
the kernels with the oracle on the cases.
"""
from __future__ import annotations

import numpy as np

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P

F32 = np.float32


def row_sumsq(v, dist=(32, 16, 8, 4, 2, 1), waves=(0, 1, 2, 3), groups_reversed=False,
              sequential=False):
    """Row sums of squares of fp32 [M, K] in the oracle's order, or in a variant of it."""
    v = np.asarray(v, F32)
    if sequential:
        return np.cumsum((v * v).astype(F32), axis=1, dtype=F32)[:, -1]
    vt = P._thread_layout(v)
    M, G = vt.shape[:2]
    part = np.zeros((M, P.THREADS), F32)
    for i in (range(G - 1, -1, -1) if groups_reversed else range(G)):
        for j in range(8):
            part = (part + (vt[:, i, :, j] * vt[:, i, :, j]).astype(F32)).astype(F32)
    p = part.reshape(M, P.THREADS // P.WAVE, P.WAVE)
    lanes = np.arange(P.WAVE)
    for o in dist:
        p = (p + p[:, :, lanes ^ o]).astype(F32)
    tot = p[:, waves[0], 0]
    for w in waves[1:]:
        tot = (tot + p[:, w, 0]).astype(F32)
    return tot


def head_sumsq(v, dist=(8, 4, 2, 1), sequential=False):
    """Per-head (128) sums of squares of fp32 [M, N] -> [M, N / 128], the oracle's order or a
    variant."""
    v = np.asarray(v, F32)
    M, N = v.shape
    h = v.reshape(M, N // P.HEAD, 16, 8)
    if sequential:
        sq = (h * h).astype(F32).reshape(M, N // P.HEAD, P.HEAD)
        return np.cumsum(sq, axis=2, dtype=F32)[..., -1]
    part = np.zeros((M, N // P.HEAD, 16), F32)
    for j in range(8):
        part = (part + (h[..., j] * h[..., j]).astype(F32)).astype(F32)
    lanes = np.arange(16)
    for o in dist:
        part = (part + part[..., lanes ^ o]).astype(F32)
    return part[..., 0]


ROW_ORDERS = {
    "sequential": dict(sequential=True),
    "butterfly 1..32": dict(dist=(1, 2, 4, 8, 16, 32)),
    "waves reversed": dict(waves=(3, 2, 1, 0)),
    "groups reversed": dict(groups_reversed=True),
}
HEAD_ORDERS = {
    "sequential": dict(sequential=True),
    "butterfly 1..8": dict(dist=(1, 2, 4, 8)),
}


def add_rms_quant_with(y_bits, w_bits, eps, **order):
    """add_rms_quant of rows y with a zero residual, the row sums taken in the given order
    (none: the oracle's) -> (q, scale)."""
    v = O.bf16_to_f32(y_bits)
    inv = P.inv_rms(row_sumsq(v, **order), v.shape[1], eps)
    w1 = (O.bf16_to_f32(w_bits) + F32(1)).astype(F32)
    n = ((v * inv[:, None]).astype(F32) * w1[None, :]).astype(F32)
    return O.quant_per_token(O.f32_to_bf16(n))


def gdn_norm_quant_with(x_bits, z_bits, w_bits, eps, **order):
    """gdn_norm_quant with the head sums taken in the given order -> (q, scale)."""
    x = O.bf16_to_f32(x_bits)
    M, N = x.shape
    inv = P.inv_rms(head_sumsq(x, **order), P.HEAD, eps)
    w = np.tile(O.bf16_to_f32(w_bits), N // P.HEAD)
    sg = P.silu_f32(O.bf16_to_f32(z_bits))
    a = (x.reshape(M, N // P.HEAD, P.HEAD) * inv[..., None]).astype(F32).reshape(M, N)
    n = ((a * w[None, :]).astype(F32) * sg).astype(F32)
    return O.quant_per_token(O.f32_to_bf16(n))


def _differs(a, b):
    (qa, sa), (qb, sb) = a, b
    return not (np.array_equal(qa, qb) and np.array_equal(sa.view(np.uint32), sb.view(np.uint32)))


def _bf16_range(lo, hi):
    """Every bf16 value in [lo, hi] (0 < lo < hi), as bits."""
    b = np.arange(O.f32_to_bf16(np.array([lo], F32))[0], O.f32_to_bf16(np.array([hi], F32))[0] + 1)
    return b.astype(np.uint16)


def _spread_rows(rng, rows, k):
    return (rng.standard_normal((rows, k)) * np.exp2(rng.integers(-6, 7, (rows, k)))).astype(F32)


def add_rms_cases(K=5120, eps=1e-6, seed=5, rows=2048):
    """[(y bits [1, K], weight bits [K], names of the ROW_ORDERS it tells apart)], together
    covering every order in ROW_ORDERS."""
    rng = np.random.default_rng(seed)
    x = _spread_rows(rng, rows, K)
    jstar = rng.integers(0, K, rows)
    x[np.arange(rows), jstar] = np.abs(x).max(axis=1) * F32(2.5)
    y = O.f32_to_bf16(x)
    v = O.bf16_to_f32(y)
    inv = P.inv_rms(row_sumsq(v), K, eps)
    wc = np.concatenate([_bf16_range(2.0 ** -8, 0.5), _bf16_range(2.0 ** -8, 0.5) | 0x8000])
    w1 = (O.bf16_to_f32(wc) + F32(1)).astype(F32)
    top = v[np.arange(rows), jstar]

    def top_out(inv_):
        return O.f32_to_bf16(((top * inv_).astype(F32)[:, None] * w1[None, :]).astype(F32))
    base = top_out(inv)
    cases, covered = [], set()
    for name, order in ROW_ORDERS.items():
        if name in covered:
            continue
        hits = np.argwhere(top_out(P.inv_rms(row_sumsq(v, **order), K, eps)) != base)
        for r, c in hits:
            w = np.zeros(K, np.uint16)
            w[jstar[r]] = wc[c]
            ref = add_rms_quant_with(y[r:r + 1], w, eps)
            tells = {n for n, o in ROW_ORDERS.items()
                     if _differs(ref, add_rms_quant_with(y[r:r + 1], w, eps, **o))}
            if name in tells:
                cases.append((y[r:r + 1].copy(), w, sorted(tells)))
                covered |= tells
                break
    return cases


def gdn_cases(heads=4, eps=1e-6, seed=7, rows=256):
    """[(x bits [1, N], z bits [1, N], weight bits [128], names of the HEAD_ORDERS it tells
    apart)], together covering every order in HEAD_ORDERS."""
    N = heads * P.HEAD
    rng = np.random.default_rng(seed)
    x = _spread_rows(rng, rows, N)
    p = rng.integers(0, P.HEAD, rows)
    hstar = rng.integers(0, heads, rows)
    xr = x.reshape(rows, heads, P.HEAD)
    xr[np.arange(rows), :, p] = 0.0                     # position p: zero in every head ...
    xr[np.arange(rows), hstar, p] = np.abs(xr[np.arange(rows), hstar]).max(axis=1) * F32(2.5)
    xb = O.f32_to_bf16(xr.reshape(rows, N))             # ... but the largest element of head h*
    xf = O.bf16_to_f32(xb)
    inv = P.inv_rms(head_sumsq(xf), P.HEAD, eps)[np.arange(rows), hstar]
    top = xf[np.arange(rows), hstar * P.HEAD + p]
    wc = _bf16_range(0.5, 2.0)
    zc = _bf16_range(1.0, 4.0)
    sg = P.silu_f32(O.bf16_to_f32(zc))

    def top_out(inv_):
        a = (top * inv_).astype(F32)
        return O.f32_to_bf16(((a[:, None, None] * O.bf16_to_f32(wc)[None, :, None]).astype(F32)
                              * sg[None, None, :]).astype(F32))
    base = top_out(inv)
    cases, covered = [], set()
    for name, order in HEAD_ORDERS.items():
        if name in covered:
            continue
        inv_a = P.inv_rms(head_sumsq(xf, **order), P.HEAD, eps)[np.arange(rows), hstar]
        hits = np.argwhere(top_out(inv_a) != base)
        for r, iw, iz in hits:
            w = np.full(P.HEAD, O.f32_to_bf16(np.array([0.25], F32))[0], np.uint16)
            w[p[r]] = wc[iw]
            z = np.full((1, N), O.f32_to_bf16(np.array([1.0], F32))[0], np.uint16)
            z[0, hstar[r] * P.HEAD + p[r]] = zc[iz]
            ref = gdn_norm_quant_with(xb[r:r + 1], z, w, eps)
            tells = {n for n, o in HEAD_ORDERS.items()
                     if _differs(ref, gdn_norm_quant_with(xb[r:r + 1], z, w, eps, **o))}
            if name in tells:
                cases.append((xb[r:r + 1].copy(), z, w, sorted(tells)))
                covered |= tells
                break
    return cases
