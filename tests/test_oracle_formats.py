"""Pins of the oracle's number formats (CPU): e4m3fn encode/decode against torch's float8_e4m3fn
cast and the closed form, e2m1/e8m0 against the reference's own known answers, bf16 rounding
against torch."""
import numpy as np
import pytest
import torch

from oracle import mxfp4_oracle as O


def torch_e4m3(x_f32: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x_f32, np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_e4m3_decode_closed_form_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    d = O.e4m3fn_decode(codes)
    for c in range(256):
        s, e, m = (c >> 7), (c >> 3) & 15, c & 7
        if (c & 0x7F) == 0x7F:
            assert np.isnan(d[c])
            continue
        v = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        assert d[c] == (-v if s else v), c
    assert d[0x7E] == 448.0 and d[0x08] == 2.0 ** -6 and d[0x01] == 2.0 ** -9


def test_e4m3_decode_matches_torch():
    codes = np.arange(256, dtype=np.uint8)
    t = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    d = O.e4m3fn_decode(codes)
    assert np.array_equal(np.isnan(t), np.isnan(d))
    ok = ~np.isnan(t)
    assert np.array_equal(t[ok].view(np.uint32), d[ok].view(np.uint32))   # incl. -0.0


def test_e4m3_encode_roundtrip_all_codes():
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    assert np.array_equal(O.e4m3fn_encode(O.e4m3fn_decode(codes)), codes)


def test_e4m3_encode_matches_torch_every_bf16_pattern():
    x = O.bf16_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))
    assert np.array_equal(O.e4m3fn_encode(x), torch_e4m3(x))


def test_e4m3_encode_matches_torch_at_every_midpoint():
    pos = O.e4m3fn_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = ((pos[:-1] + pos[1:]) / 2).astype(np.float32)       # exact in fp32
    xs = [mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
          pos.astype(np.float32), np.float32([464.0, 479.99, 480.0, 1e30, 2.0 ** -10])]
    x = np.concatenate(xs).astype(np.float32)
    x = np.concatenate([x, -x])
    assert np.array_equal(O.e4m3fn_encode(x), torch_e4m3(x))


def test_e4m3_encode_matches_torch_random():
    g = np.random.default_rng(1)
    x = (np.exp2(g.uniform(-14, 9.5, 2_000_000)) * g.choice([-1, 1], 2_000_000)).astype(np.float32)
    assert np.array_equal(O.e4m3fn_encode(x), torch_e4m3(x))


def test_e4m3_encode_known_answers():
    x = np.float32([448, 464, -0.0, 2.0 ** -10, 3 * 2.0 ** -10, 0.3, np.nan, 500])
    assert O.e4m3fn_encode(x).tolist() == [0x7E, 0x7E, 0x80, 0x00, 0x02, 0x2A, 0x7F, 0x7F]


def test_e2m1_pack_low_nibble_is_even_index():
    # sly/tests/test_kvq_reference.py:42-45: codes 1 (0.5) and 7 (6.0) pack as 0x71
    w = np.array([[0x71]], np.uint8)
    ws = np.array([[127]], np.uint8)
    codes = O.unpack_e2m1(w, 2)
    assert codes.tolist() == [[1, 7]]
    d = O.dequant_weight(np.tile(w, (1, 16)), ws)
    assert d[0, :2].tolist() == [0.5, 6.0]


def test_e2m1_negative_code_sets_bit3():
    # sly/tests/test_kvq_reference.py:48-49: -6.0 is code 0xF
    assert O.E2M1_VALUES[0xF] == -6.0 and O.E2M1_VALUES[0x7] == 6.0
    assert np.all(O.E2M1_VALUES[8:] == -O.E2M1_VALUES[:8])
    assert O.E2M1_VALUES[:8].tolist() == [0, 0.5, 1, 1.5, 2, 3, 4, 6]


def test_e8m0_scale():
    assert O.e8m0_to_f32(np.uint8([127, 119, 125, 0, 254])).tolist() == [
        1.0, 2.0 ** -8, 2.0 ** -2, 2.0 ** -127, 2.0 ** 127]
    assert np.isnan(O.e8m0_to_f32(np.uint8([255]))[0])


def test_dequant_weight_block_scale_applies_per_32():
    w = np.full((1, 32), 0x77, np.uint8)           # 64 codes of 6.0
    ws = np.array([[126, 120]], np.uint8)
    d = O.dequant_weight(w, ws)
    assert np.all(d[0, :32] == 3.0) and np.all(d[0, 32:] == 6.0 * 2.0 ** -7)


def test_bf16_rounding_matches_torch():
    g = np.random.default_rng(2)
    x = (g.standard_normal(1_000_000) * np.exp2(g.uniform(-30, 30, 1_000_000))).astype(np.float32)
    ties = (np.arange(1, 1000, dtype=np.uint32) << 16 | np.uint32(0x8000)).view(np.float32)
    x = np.concatenate([x, ties, -ties, np.float32([0.0, -0.0, np.inf, -np.inf])])
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(O.f32_to_bf16(x), t)


@pytest.mark.parametrize("v,ulp", [(1.0, 2.0 ** -7), (1.99, 2.0 ** -7), (-3.0, 2.0 ** -6),
                                   (0.0, 2.0 ** -133), (2.0 ** -20, 2.0 ** -27)])
def test_bf16_ulp(v, ulp):
    assert O.bf16_ulp(np.array([v]))[0] == ulp
