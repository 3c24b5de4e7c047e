"""Pins the NumPy oracle's encoder / decoder against checks that do not retype it.

* closed-form known answers (axis-aligned angles, 3-4-5 radius, fp16 x*x
  overflow, V floor scale, group max -> +-127, half-even ties);
* an independent exact-rational restatement (tests/exact_f16.py) on random,
  heavy-tailed and edge inputs, for fp16 and fp32 inputs and every bit width;
* the packed shapes asserted by the reference's own tests
  (tests/benchmarks/test_turbo_polar_offline.py:27-34 of the reference);
* invariants: pack/unpack round trips, |decoded pair| == radius within fp16
  rounding, decode->encode idempotence of the angle codes.
"""

import math

import numpy as np
import pytest

import oracle
from exact_f16 import (
    log_radius_f16,
    pair_codes_f16,
    pair_codes_f32,
    r16,
    r32,
    v_group_f16,
    v_group_f32,
)
from fractions import Fraction

F16 = np.float16


def _page_from_pairs(pairs, dtype=np.float16):
    k = np.zeros((1, 1, 64, 128), dtype=np.float32)
    for i, (x, y) in enumerate(pairs):
        t, j = divmod(i, 64)
        k[0, 0, t, 2 * j] = x
        k[0, 0, t, 2 * j + 1] = y
    return k.astype(dtype)


def _codes(enc, which="deep", bits=4, n=64):
    c = enc["angle_codes_" + which][0, 0]
    if bits == 4:
        return oracle.unpack_4bit(c, n)
    if bits == 2:
        return oracle.unpack_2bit(c, n)
    return c


# ---------------------------------------------------------------- known answers

KNOWN = [  # (x, y) -> (4-bit code, 8-bit code), worked out by hand from encoder.py:46-55
    ((0.0, 0.0), (8, 128)),
    ((1.0, 0.0), (8, 128)),
    ((-1.0, 0.0), (15, 255)),
    ((-1.0, -0.0), (0, 0)),
    ((0.0, 1.0), (11, 191)),
    ((0.0, -1.0), (4, 64)),
    ((1.0, 1.0), (9, 159)),
    ((-1.0, 1.0), (13, 223)),
]


@pytest.mark.parametrize("bits,col", [(4, 0), (8, 1)])
def test_known_angle_codes(bits, col):
    k = _page_from_pairs([p for p, _ in KNOWN])
    enc = oracle.encode_block(k, l1_bits=8, deep_bits=bits, split_dim=0)
    got = _codes(enc, "deep", bits)[0][: len(KNOWN)]
    assert list(got) == [c[col] for _, c in KNOWN]


def test_known_angle_code_fp32_wrap():
    """For fp32 inputs the near-one wrap (encoder.py:50-51) fires: (-1, +0) -> 0,
    while fp16 inputs give 15 (fp16(1 - 1e-6) == 1.0)."""
    k32 = _page_from_pairs([(-1.0, 0.0)], np.float32)
    k16 = _page_from_pairs([(-1.0, 0.0)], np.float16)
    c32 = _codes(oracle.encode_block(k32, l1_bits=8, deep_bits=4, split_dim=0))[0][0]
    c16 = _codes(oracle.encode_block(k16, l1_bits=8, deep_bits=4, split_dim=0))[0][0]
    assert (c32, c16) == (0, 15)


def test_known_radii():
    k = _page_from_pairs([(3, 4), (256, 0), (255, 10), (0, 0), (-3, -4)])
    r = oracle.encode_block(k)["radii"][0, 0, 0, :5].view(np.uint16)
    assert list(r) == [0x4500, 0x7C00, 0x5BF9, 0x0000, 0x4500]


def test_fp16_constants():
    assert F16(np.pi).view(np.uint16) == 0x4248
    assert F16(2 * np.pi).view(np.uint16) == 0x4648
    assert F16(1e-6).view(np.uint16) == 0x0011
    assert F16(1e-4).view(np.uint16) == 0x068E
    assert oracle.fp16_scale(1 / math.sqrt(128)) == 0.08837890625


def test_v_known_answers():
    v = np.zeros((1, 1, 1, 1, 128), np.float16)
    v[..., 32:64] = np.arange(32) * 0.5 - 8  # scale 1 after the 127 below: exact ties at +-x.5
    v[..., 32] = 127
    v[..., 64:96] = np.linspace(-3, 3, 32)
    codes, scales = oracle.quantize_block(v)
    s = scales[0, 0, 0, 0].view(np.uint16)
    assert s[0] == 0x068E and np.all(codes[..., :32] == 0)  # zero group -> floor scale, codes 0
    assert float(scales[0, 0, 0, 0, 1]) == 1.0
    ties = codes[0, 0, 0, 0, 33:64]
    expect = [int(np.rint(x)) for x in (np.arange(1, 32) * 0.5 - 8)]  # half-even
    assert list(ties) == expect
    g2 = codes[0, 0, 0, 0, 64:96]
    assert g2.min() == -127 and g2.max() == 127  # group max maps to +-127


# ------------------------------------------------ exact-rational restatement

def _random_pairs(rng, n):
    xs = np.concatenate([
        rng.standard_normal(n // 2) * 3,
        rng.standard_t(3, n // 4) * 20,
        rng.choice([-0.0, 0.0, 1e-7, -1e-7, 65504, 255.9, 256, 300], n - n // 2 - n // 4),
    ])
    ys = np.concatenate([rng.standard_normal(n // 2) * 3, rng.standard_normal(n // 4) * 1e-3,
                         rng.choice([0.0, -0.0, 1.0, -1.0, 1e-5], n - n // 2 - n // 4)])
    rng.shuffle(xs)
    return xs, ys


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_encoder_matches_exact_rational_fp16(bits):
    rng = np.random.default_rng(bits)
    xs, ys = _random_pairs(rng, 4096)
    pairs = list(zip(F16(xs).astype(float), F16(ys).astype(float)))
    k = _page_from_pairs(pairs, np.float16)
    enc = oracle.encode_block(k, l1_bits=8, deep_bits=bits, split_dim=0)
    radii = enc["radii"][0, 0].reshape(-1)
    codes = _codes(enc, "deep", bits).reshape(-1)
    for i, (x, y) in enumerate(pairs):
        r, c = pair_codes_f16(x, y, bits)
        assert float(radii[i]) == r or (math.isinf(r) and math.isinf(radii[i])), (x, y, r, radii[i])
        assert codes[i] == c, (x, y, c, codes[i])


@pytest.mark.parametrize("bits", [4, 8])
def test_encoder_matches_exact_rational_fp32(bits):
    rng = np.random.default_rng(100 + bits)
    xs, ys = _random_pairs(rng, 2048)
    pairs = list(zip(np.float32(xs).astype(float), np.float32(ys).astype(float)))
    k = _page_from_pairs(pairs, np.float32)
    enc = oracle.encode_block(k, l1_bits=8, deep_bits=bits, split_dim=0)
    radii = enc["radii"][0, 0].reshape(-1)
    codes = _codes(enc, "deep", bits).reshape(-1)
    for i, (x, y) in enumerate(pairs):
        r, c = pair_codes_f32(x, y, bits)
        assert float(radii[i]) == r or (math.isinf(r) and math.isinf(radii[i])), (x, y)
        assert codes[i] == c, (x, y, c, codes[i])


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_int8_log_radii_match_exact_rational(dtype):
    rng = np.random.default_rng(7)
    k = (rng.standard_normal((1, 1, 64, 128)) * np.exp(rng.uniform(-3, 3, (1, 1, 64, 1)))).astype(dtype)
    k[0, 0, 0, :4] = 0  # zero radii hit the fp16(1e-6) floor
    enc = oracle.encode_block(k, l1_bits=4, deep_bits=8, split_dim=0, use_int8_radii=True)
    r16s = []
    for t in range(64):
        for j in range(64):
            x, y = float(k[0, 0, t, 2 * j]), float(k[0, 0, t, 2 * j + 1])
            r16s.append((pair_codes_f16 if dtype == np.float16 else pair_codes_f32)(x, y, 8)[0])
    lr = [log_radius_f16(r) for r in r16s]
    ls = max(abs(v) for v in lr)
    ls16 = r16(r32(Fraction(ls) / 127))
    assert float(enc["radii_scales"].reshape(())) == ls16
    expect = [int(min(max(round(r32(Fraction(v) / Fraction(ls16))), -128), 127)) for v in lr]
    assert list(enc["radii"].reshape(-1)) == expect


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_v_quantizer_matches_exact_rational(dtype):
    rng = np.random.default_rng(9)
    v = (rng.standard_normal((1, 1, 1, 16, 128)) * np.exp(rng.uniform(-4, 4, (1, 1, 1, 16, 1)))).astype(dtype)
    v[0, 0, 0, 0, :32] = 0
    v[0, 0, 0, 1, 32:64] = np.arange(32) - 16.0
    codes, scales = oracle.quantize_block(v)
    fn = v_group_f16 if dtype == np.float16 else v_group_f32
    for t in range(16):
        for g in range(4):
            s, c = fn([float(x) for x in v[0, 0, 0, t, 32 * g: 32 * g + 32]])
            assert float(scales[0, 0, 0, t, g]) == s
            assert list(codes[0, 0, 0, t, 32 * g: 32 * g + 32]) == c


# ------------------------------------------------ V dequantisation (v_quant/encoder.py:32-38)

def test_dequantize_known_answers():
    """Element by element with exact rationals: dim d of a token takes the scale
    of group d // 32 of that token (the reshape to [..., D // 32, 32] at
    v_quant/encoder.py:35), and the product is rounded once to fp16."""
    rng = np.random.default_rng(21)
    codes = rng.integers(-128, 128, size=(1, 2, 3, 5, 128)).astype(np.int8)
    codes[0, 0, 0, 0, :4] = [-128, 127, 0, 1]
    # four scales of different magnitude per token, so a group read from the
    # wrong token, group or position changes the product
    scales = (np.exp2(rng.integers(-9, 3, size=(1, 2, 3, 5, 4))) *
              rng.uniform(1.0, 2.0, size=(1, 2, 3, 5, 4))).astype(np.float16)
    scales[0, 0, 0, 0] = np.array([0x068E, 0x3C00, 0x7BFF, 0x0001], np.uint16).view(np.float16)
    got = oracle.dequantize_block(codes, scales)
    assert got.dtype == np.float16 and got.shape == codes.shape
    for b, h, s, t in np.ndindex(1, 2, 3, 5):
        for d in range(128):
            want = r16(Fraction(int(codes[b, h, s, t, d])) * Fraction(float(scales[b, h, s, t, d // 32])))
            g = float(got[b, h, s, t, d])
            assert g == want or (math.isinf(want) and g == want), (b, h, s, t, d, g, want)
    # closed forms: -128 * fp16(1e-4) = -0.012817..., 127 * 1.0, 65504 * 0 = 0,
    # 1 * smallest subnormal = smallest subnormal
    row = got[0, 0, 0, 0].view(np.uint16)
    assert float(got[0, 0, 0, 0, 0]) == r16(Fraction(-128) * Fraction(float(np.uint16(0x068E).view(np.float16))))
    assert row[32] == np.float16(float(codes[0, 0, 0, 0, 32])).view(np.uint16)  # scale 1.0 is the identity
    assert row[96] == (np.float16(float(codes[0, 0, 0, 0, 96])) * np.uint16(1).view(np.float16)).view(np.uint16)


def test_dequantize_inverts_exact_quantization():
    """Values that are code x power-of-two with the group max at 127 x scale
    quantise exactly, so dequantize(quantize(v)) returns v bit for bit."""
    rng = np.random.default_rng(22)
    v = np.zeros((1, 1, 2, 64, 128), np.float32)
    for s, t, g in np.ndindex(2, 64, 4):
        scale = np.exp2(float(rng.integers(-12, 4)))
        c = rng.integers(-127, 128, size=32).astype(np.float32)
        c[rng.integers(0, 32)] = rng.choice([-127.0, 127.0])
        v[0, 0, s, t, 32 * g: 32 * g + 32] = c * scale
    for dtype in (np.float16, np.float32):
        x = v.astype(dtype)
        codes, scales = oracle.quantize_block(x)
        back = oracle.dequantize_block(codes, scales)
        assert np.array_equal(back.astype(np.float32), x.astype(np.float16).astype(np.float32))


def test_dequantize_bounds_quantization_error():
    """|v - dequantize(quantize(v))| <= 0.53125 * s + half an fp16 ulp of the
    result, s the group's scale: the fp16 quotient v / s (|v / s| <= 127.5)
    errs by at most 2^-5, rint by 0.5, and the product rounds once.  Groups of
    one token span 2^-8 .. 2^8 in magnitude, so any mix-up of groups breaks it."""
    rng = np.random.default_rng(23)
    mag = np.exp2(rng.integers(-8, 9, size=(1, 2, 4, 64, 4, 1))).astype(np.float32)
    v = (rng.standard_normal((1, 2, 4, 64, 4, 32)).astype(np.float32) * mag).reshape(1, 2, 4, 64, 128)
    v = v.astype(np.float16)
    codes, scales = oracle.quantize_block(v)
    back = oracle.dequantize_block(codes, scales).astype(np.float64)
    s = np.repeat(scales.astype(np.float64), 32, axis=-1)
    half_ulp = np.spacing(np.abs(back).astype(np.float16)).astype(np.float64) / 2
    err = np.abs(back - v.astype(np.float64))
    assert np.all(err <= 0.53125 * s + half_ulp)
    # and the bound is tight enough to matter: the error reaches a third of s somewhere
    assert np.max(err / s) > 0.33


def test_f64_to_f16_rounding_is_direct():
    """atan2_cr / log_cr rely on NumPy's float64 -> float16 cast rounding once;
    checked against the exact rounding on values straddling fp16 midpoints."""
    rng = np.random.default_rng(3)
    h = rng.integers(0x0400, 0x7800, 2000).astype(np.uint16).view(np.float16).astype(np.float64)
    ulp = np.spacing(h.astype(np.float16)).astype(np.float64)
    d = h + ulp / 2 + rng.choice([-1, 1], 2000) * np.ldexp(1.0, -40) * h
    got = d.astype(np.float16).astype(np.float64)
    want = np.array([r16(Fraction(x)) for x in d])
    assert np.array_equal(got, want)


# ------------------------------------------------------------ layout / packing

@pytest.mark.parametrize("l1,deep,split", [(4, 4, 64), (4, 8, 0), (8, 2, 32), (4, 2, 46), (8, 4, 128)])
def test_packed_shapes_follow_reference_rule(l1, deep, split):
    k = np.random.default_rng(1).standard_normal((2, 3, 64, 128)).astype(np.float16)
    enc = oracle.encode_block(k, l1_bits=l1, deep_bits=deep, split_dim=split)
    split_half = split // 2
    deep_half = 64 - split_half
    l1_len = (split_half + 1) // 2 if l1 == 4 else split_half
    cpb = 8 // deep
    deep_len = (deep_half + cpb - 1) // cpb
    assert enc["angle_codes_l1"].shape == (2, 3, 64, l1_len)
    assert enc["angle_codes_deep"].shape == (2, 3, 64, deep_len)
    assert oracle.layout_bytes(l1, deep, split) == (l1_len, deep_len)
    assert enc["radii"].shape == (2, 3, 64, 64)


@pytest.mark.parametrize("n", [1, 2, 7, 31, 32, 46])
def test_pack_unpack_round_trip(n):
    rng = np.random.default_rng(n)
    c4 = rng.integers(0, 16, (3, n)).astype(np.uint8)
    c2 = rng.integers(0, 4, (3, n)).astype(np.uint8)
    assert np.array_equal(oracle.unpack_4bit(oracle.pack_4bit(c4), n), c4)
    assert np.array_equal(oracle.unpack_2bit(oracle.pack_2bit(c2), n), c2)
    # low nibble / low bit pair first (encoder.py:111-112,126-129)
    assert oracle.pack_4bit(np.array([[1, 2]], np.uint8))[0, 0] == 0x21
    assert oracle.pack_2bit(np.array([[1, 2, 3, 0]], np.uint8))[0, 0] == 0b00111001


# ------------------------------------------------------------------ invariants

@pytest.mark.parametrize("layout", [(False, 4, 4, 64), (True, 4, 8, 0), (False, 4, 2, 64)])
def test_decode_radius_invariant(layout):
    int8, l1, deep, split = layout
    k = np.random.default_rng(4).standard_normal((1, 2, 64, 128)).astype(np.float16)
    enc = oracle.encode_block(k, l1_bits=l1, deep_bits=deep, split_dim=split, use_int8_radii=int8)
    kh = oracle.decode_block(enc["radii"], enc["radii_scales"], enc["angle_codes_l1"], enc["angle_codes_deep"],
                             enc["metadata"]).astype(np.float64).reshape(1, 2, 64, 64, 2)
    r_dec = np.sqrt((kh ** 2).sum(-1))
    if int8:
        r_ref = np.exp(enc["radii"].astype(np.float32) * enc["radii_scales"].astype(np.float32))
    else:
        r_ref = enc["radii"].astype(np.float64)
    assert np.allclose(r_dec, r_ref, rtol=2e-3, atol=1e-3)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_decode_then_encode_returns_codes(bits):
    """Decoded pairs sit at the centre of their code's angle bin, so re-encoding
    them returns the same code (away from the +-pi seam of the top code)."""
    rng = np.random.default_rng(bits)
    k = (rng.standard_normal((1, 1, 64, 128)) * 4).astype(np.float16)
    enc = oracle.encode_block(k, l1_bits=8, deep_bits=bits, split_dim=0)
    kh = oracle.decode_block(enc["radii"], None, enc["angle_codes_l1"], enc["angle_codes_deep"], enc["metadata"])
    enc2 = oracle.encode_block(kh.reshape(1, 1, 64, 128), l1_bits=8, deep_bits=bits, split_dim=0)
    c1 = _codes(enc, "deep", bits)
    c2 = _codes(enc2, "deep", bits)
    top = (1 << bits) - 1
    seam = (c1 == top) | (c1 == 0)
    small = enc["radii"][0, 0].astype(np.float32) < 0.05
    ok = (c1 == c2) | seam | small
    assert ok.all(), np.argwhere(~ok)[:5]


def test_angle_code_rule_consistent_with_encoder():
    """oracle.angle_codes_f16 (used for the exhaustive kernel table) agrees with
    encode_block on encoded pairs."""
    rng = np.random.default_rng(11)
    k = rng.standard_normal((1, 1, 64, 128)).astype(np.float16)
    a16 = oracle.atan2_cr(k[..., 1::2], k[..., 0::2], np.float16)
    for bits in (2, 4, 8):
        enc = oracle.encode_block(k, l1_bits=8, deep_bits=bits, split_dim=0)
        assert np.array_equal(oracle.angle_codes_f16(a16, bits)[0, 0], _codes(enc, "deep", bits))


def test_angle_quotient_product_is_exact_for_every_fp16_numerator():
    """The encoder's fast angle code divides the shifted angle s1 = fp16(a16 +
    fp16(pi)) by fp16(2*pi) as one fp32 product with fp32(1 / 6.28125), rounded
    once, then to fp16; its guards skip the quotient on the strength of this
    check.  Over every finite fp16 s1 the product rounds to the same fp16 as
    the oracle's fp16 division (encoder.py:48) and as the correctly rounded
    quotient of the exact rationals."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    s1 = bits.view(F16)
    s1 = s1[np.isfinite(s1)]
    inv = np.float32(0.159203976392745972)
    assert Fraction(float(inv)) - Fraction(1) / Fraction(6.28125) < Fraction(1, 2 ** 26)
    prod = (s1.astype(np.float32) * inv).astype(F16)
    div = (s1 / F16(2 * np.pi)).astype(F16)
    assert np.array_equal(prod.view(np.uint16), div.view(np.uint16))
    two_pi16 = Fraction(6.28125)
    exact = np.array([r16(Fraction(float(x)) / two_pi16) for x in s1], dtype=np.float64).astype(F16)
    assert np.array_equal(prod, exact)  # by value: the rationals carry no -0
