"""The order-sensitive producer inputs of tests/_orders.py: the variant sums equal the oracle's
in the oracle's order, and every case tells the oracle's order apart from the alternatives it
names (the GPU tests then hold the kernels to the oracle on them)."""
import numpy as np

from oracle import mxfp4_oracle as O
from oracle import producers_oracle as P
from tests import _orders as ORD
from vllm_sly_radiance_amd import synthetic


def test_default_orders_are_the_oracles():
    v = O.bf16_to_f32(synthetic.activations(6, 5120, seed=3))
    assert np.array_equal(ORD.row_sumsq(v).view(np.uint32), P.row_sum_squares(v).view(np.uint32))
    x = O.bf16_to_f32(synthetic.activations(5, 768, seed=4))
    assert np.array_equal(ORD.head_sumsq(x).view(np.uint32), P.head_sum_squares(x).view(np.uint32))
    y = synthetic.activations(4, 5120, seed=5)
    w = O.f32_to_bf16(np.random.default_rng(6).standard_normal(5120).astype(np.float32) * 0.1)
    q, s = ORD.add_rms_quant_with(y, w, 1e-6)
    oq, os_, _ = P.add_rms_quant(y, np.zeros_like(y), w, 1e-6)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))
    xb = synthetic.activations(3, 512, seed=7)
    zb = synthetic.activations(3, 512, seed=8)
    wg = O.f32_to_bf16(1.0 + np.random.default_rng(9).standard_normal(128).astype(np.float32) * 0.2)
    q, s = ORD.gdn_norm_quant_with(xb, zb, wg, 1e-6)
    oq, os_ = P.gdn_norm_quant(xb, zb, wg, 1e-6)
    assert np.array_equal(q, oq) and np.array_equal(s.view(np.uint32), os_.view(np.uint32))


def test_variant_orders_differ_from_the_oracles():
    """Each variant is a different order: on rows of widely spread magnitudes its sums differ
    from the oracle's on some rows (and equal them on others: rounding, not a wrong formula)."""
    rng = np.random.default_rng(1)
    v = (rng.standard_normal((256, 5120)) * np.exp2(rng.integers(-6, 7, (256, 5120)))).astype(np.float32)
    ref = P.row_sum_squares(v)
    for name, order in ORD.ROW_ORDERS.items():
        alt = ORD.row_sumsq(v, **order)
        diff = np.count_nonzero(alt != ref)
        assert 0 < diff, name
        assert np.allclose(alt, ref, rtol=1e-5), name
    x = (rng.standard_normal((256, 512)) * np.exp2(rng.integers(-6, 7, (256, 512)))).astype(np.float32)
    href = P.head_sum_squares(x)
    for name, order in ORD.HEAD_ORDERS.items():
        alt = ORD.head_sumsq(x, **order)
        assert 0 < np.count_nonzero(alt != href), name
        assert np.allclose(alt, href, rtol=1e-5), name


def test_add_rms_cases_tell_every_order_apart():
    cases = ORD.add_rms_cases()
    covered = set()
    for y, w, tells in cases:
        ref = ORD.add_rms_quant_with(y, w, 1e-6)
        for name in tells:
            assert ORD._differs(ref, ORD.add_rms_quant_with(y, w, 1e-6, **ORD.ROW_ORDERS[name]))
        covered |= set(tells)
    assert covered == set(ORD.ROW_ORDERS)


def test_gdn_cases_tell_every_order_apart():
    cases = ORD.gdn_cases()
    covered = set()
    for x, z, w, tells in cases:
        ref = ORD.gdn_norm_quant_with(x, z, w, 1e-6)
        for name in tells:
            assert ORD._differs(ref, ORD.gdn_norm_quant_with(x, z, w, 1e-6, **ORD.HEAD_ORDERS[name]))
        covered |= set(tells)
    assert covered == set(ORD.HEAD_ORDERS)
