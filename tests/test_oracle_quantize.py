"""Pins oracle/quantize.py (the MLX affine quantizer restatement) without running the oracle's
formula twice: expected values come from exact rational arithmetic on hand-built groups, from
invariants the algorithm fixes, and from the layout the reference kernel reads
(laguna_mlx/q8_attn.py:8-10). Each planted-mistake test shows that a plausible slip in the
restatement (wrong rounding mode, dropped q0 adjustment, swapped nibble order, skipped bf16
rounding) fails at least one of these checks."""
from fractions import Fraction as Fr

import numpy as np
import pytest

from oracle import quantize as Q


def half_away(fr: Fr) -> int:
    """Exact round-half-away-from-zero of a rational."""
    s = -1 if fr < 0 else 1
    a = abs(fr)
    f = a.numerator // a.denominator
    return s * (f + (1 if a - f >= Fr(1, 2) else 0))


def bf16_exact(fr: Fr) -> Fr:
    """Round a rational to bf16 (8 significant bits, nearest even), exactly."""
    if fr == 0:
        return Fr(0)
    s = -1 if fr < 0 else 1
    a = abs(fr)
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    m = a * 128  # 7 fraction bits
    f = m.numerator // m.denominator
    r = m - f
    f = f + (1 if r > Fr(1, 2) or (r == Fr(1, 2) and f % 2 == 1) else 0)
    return s * Fr(f, 128) * Fr(2) ** e


def bf16_bits(v) -> int:
    return int(Q.f32_to_bf16_bits(np.array([v], np.float32))[0])


def fr_to_bits(fr: Fr) -> int:
    return bf16_bits(float(fr))


# ---------------------------------------------------------------------------------------------
# hand-derived known answers
# ---------------------------------------------------------------------------------------------

def test_ramp_8bit_known_answer():
    # x = 0..63: side is False (|min| < |max|), edge = 63, q0 = -255, scale = -63/255, bias = 63,
    # code(x) = round((63 - x) * 255 / 63); fractional parts are k/21, never near 1/2.
    x = np.arange(64, dtype=np.float32)
    codes, s, b = Q.quantize(x[None], 64, 8)
    want = [half_away(Fr(63 - i) * 255 / 63) for i in range(64)]
    assert codes[0].tolist() == want
    assert want[0] == 255 and want[63] == 0
    assert int(s[0, 0]) == fr_to_bits(bf16_exact(Fr(-63, 255)))
    assert float(Q.bf16_bits_to_f32(s)[0, 0]) == -0.2470703125
    assert float(Q.bf16_bits_to_f32(b)[0, 0]) == 63.0


def test_negative_ramp_flips_side():
    # x = -(0..63): |min| > |max| so scale = +63/255 and bias = min = -63.
    x = -np.arange(64, dtype=np.float32)
    codes, s, b = Q.quantize(x[None], 64, 8)
    want = [half_away(Fr(63 - i) * 255 / 63) for i in range(64)]
    assert codes[0].tolist() == want
    assert float(Q.bf16_bits_to_f32(s)[0, 0]) == 0.2470703125
    assert float(Q.bf16_bits_to_f32(b)[0, 0]) == -63.0


def test_ramp_4bit_known_answer():
    # n_bins 15: scale = -63/15 = -4.2, bias = 63, code = round((63 - x) * 5 / 21).
    x = np.arange(64, dtype=np.float32)
    codes, s, b = Q.quantize(x[None], 64, 4)
    want = [half_away(Fr(63 - i) * 5 / 21) for i in range(64)]
    assert codes[0].tolist() == want
    assert int(s[0, 0]) == fr_to_bits(bf16_exact(Fr(-63, 15)))


def test_rounding_is_half_away_from_zero():
    # range [0, 255] -> scale -1, bias 255, code(x) = round(255 - x): x = 0.5 and 2.5 sit on
    # exact halves (254.5, 252.5) -> 255 and 253 away from zero (254 and 252 with ties-to-even).
    x = np.zeros(64, np.float32)
    x[1], x[2], x[3] = 255.0, 0.5, 2.5
    codes, s, b = Q.quantize(x[None], 64, 8)
    assert float(Q.bf16_bits_to_f32(s)[0, 0]) == -1.0
    assert float(Q.bf16_bits_to_f32(b)[0, 0]) == 255.0
    assert codes[0, 2] == 255 and codes[0, 3] == 253
    assert codes[0, 0] == 255 and codes[0, 1] == 0


def test_q0_adjustment_4bit():
    # max 1, min -0.3125: delta = 1.3125/15 = 0.0875, 1/0.0875 = 11.43 -> q0 = -11,
    # scale = 1 / -11 (not -delta), bias = 1. code(min) = round(1.3125 * 11) = round(14.4375) = 14
    # (15 without the adjustment); code(0) = 11 exactly: zero is representable.
    x = np.zeros(64, np.float32)
    x[0], x[1] = 1.0, -0.3125
    codes, s, b = Q.quantize(x[None], 64, 4)
    assert int(s[0, 0]) == fr_to_bits(bf16_exact(Fr(-1, 11)))
    assert float(Q.bf16_bits_to_f32(b)[0, 0]) == 1.0
    assert codes[0, 0] == 0 and codes[0, 1] == 14 and codes[0, 2] == 11


def test_all_zero_group_uses_eps_scale():
    # delta = max(0, 1e-7); side False -> scale = -1e-7, edge 0 -> q0 = 0 -> bias 0, codes 0.
    codes, s, b = Q.quantize(np.zeros((1, 64), np.float32), 64, 8)
    assert (codes == 0).all()
    assert int(b[0, 0]) == 0
    assert int(s[0, 0]) == bf16_bits(np.float32(-1e-7))


def test_constant_group():
    # all 0.5: delta 1e-7, scale -1e-7, q0 = round(-5e6) != 0 -> scale = 0.5/q0, bias 0.5,
    # every code round(0) = 0; dequantizes to exactly 0.5.
    x = np.full((1, 64), 0.5, np.float32)
    codes, s, b = Q.quantize(x, 64, 8)
    assert (codes == 0).all()
    assert float(Q.bf16_bits_to_f32(b)[0, 0]) == 0.5
    assert (Q.dequantize(codes, s, b, 64, 8) == 0.5).all()


def test_group_sizes_are_independent():
    rng = np.random.default_rng(3)
    x = Q.randn_bf16(rng, (4, 128))
    for gs in (32, 64, 128):
        c, s, b = Q.quantize(x, gs, 8)
        for g in range(128 // gs):
            c1, s1, b1 = Q.quantize(x[:, g * gs:(g + 1) * gs], gs, 8)
            assert (c[:, g * gs:(g + 1) * gs] == c1).all()
            assert (s[:, g] == s1[:, 0]).all() and (b[:, g] == b1[:, 0]).all()


# ---------------------------------------------------------------------------------------------
# invariants on random data
# ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("bits", [8, 4])
def test_invariants_random(bits):
    rng = np.random.default_rng(0)
    x = Q.randn_bf16(rng, (512, 128)) * np.float32(3)
    codes, s, b = Q.quantize(x, 64, bits)
    nb = (1 << bits) - 1
    assert codes.max() <= nb
    # each group uses both ends of the code range (min and max map to 0 / n_bins or near)
    cg = codes.reshape(-1, 64)
    assert (cg.min(axis=1) == 0).all()
    assert (cg.max(axis=1) >= nb - 1).all()
    # reconstruction error <= |scale|/2, plus what the clamp at n_bins cuts off when the q0
    # adjustment shrinks |scale| (range - n_bins*|scale|), plus bf16 rounding of scale/bias/output
    y = Q.dequantize(Q.pack_codes(codes, bits), s, b, 64, bits)
    sg = np.abs(Q.bf16_bits_to_f32(s))
    xg = x.reshape(-1, 2, 64)
    clamp = np.maximum(0, (xg.max(-1) - xg.min(-1)) - nb * sg)
    sc = np.repeat(sg, 64, axis=1)
    bound = (sc * 0.5 + np.repeat(clamp, 64, axis=1) + np.abs(x) * 2 ** -7
             + sc * nb * 2 ** -8 + 1e-6)
    assert (np.abs(y - x) <= bound).all()
    err = np.abs(y - x).mean()
    if bits == 8:
        assert err < 0.05  # the reference's own 8-bit error gate (tests/test_cache.py:113)


def test_8bit_error_smaller_than_4bit():
    rng = np.random.default_rng(1)
    x = Q.randn_bf16(rng, (256, 128))
    e = {}
    for bits in (8, 4):
        c, s, b = Q.quantize(x, 64, bits)
        y = Q.dequantize(Q.pack_codes(c, bits), s, b, 64, bits)
        e[bits] = np.abs(y - x).mean()
    assert e[8] < e[4]


def test_larger_edge_reconstructs_exactly():
    # bias is the larger-magnitude edge, so that value maps to code 0 and back exactly
    rng = np.random.default_rng(2)
    x = Q.randn_bf16(rng, (64, 64))
    codes, s, b = Q.quantize(x, 64, 8)
    bias = Q.bf16_bits_to_f32(b)[:, 0]
    edge = np.where(np.abs(x.min(1)) > np.abs(x.max(1)), x.min(1), x.max(1))
    assert (bias == edge).all()  # edges are bf16 values, so bf16(bias) is exact
    idx = np.argmax(x == edge[:, None], axis=1)
    assert (codes[np.arange(64), idx] == 0).all()


# ---------------------------------------------------------------------------------------------
# layout: bytes == MLX uint32 words (low byte / low nibble first)
# ---------------------------------------------------------------------------------------------

def test_8bit_bytes_are_mlx_words_little_endian():
    codes = np.arange(128, dtype=np.uint8)[None]
    words = Q.mlx_words(codes, 8)
    assert words.shape == (1, 32)
    assert int(words[0, 0]) == 0x03020100  # element 0 in the low byte (q8_attn.py:8-10)
    assert Q.pack_codes(codes, 8).view("<u4").tolist() == words.tolist()


def test_4bit_nibbles_even_low():
    codes = (np.arange(128) % 16).astype(np.uint8)[None]
    packed = Q.pack_codes(codes, 4)
    assert packed.shape == (1, 64)
    assert int(packed[0, 0]) == 0x10  # element 0 -> low nibble, element 1 -> high nibble
    assert packed.view("<u4").tolist() == Q.mlx_words(codes, 4).tolist()
    assert (Q.unpack_codes(packed, 4) == codes).all()


def test_bf16_rne_and_nan():
    f = np.array([1.0, 1.00390625, 1.01171875, -2.5, np.inf, np.nan], np.float32)
    # 1 + 2^-8 is a tie -> even (1.0); 1 + 3*2^-8 is a tie -> even (1 + 2^-6)
    bits = Q.f32_to_bf16_bits(f)
    assert bits[0] == 0x3F80 and bits[1] == 0x3F80 and bits[2] == 0x3F82
    assert bits[3] == 0xC020 and bits[4] == 0x7F80 and bits[5] == 0x7FC0


# ---------------------------------------------------------------------------------------------
# planted mistakes must be caught by the checks above
# ---------------------------------------------------------------------------------------------

def test_planted_round_half_even_is_caught(monkeypatch):
    monkeypatch.setattr(Q, "round_half_away", lambda x: np.rint(np.asarray(x, np.float32)))
    with pytest.raises(AssertionError):
        test_rounding_is_half_away_from_zero()


def test_planted_missing_q0_adjustment_is_caught(monkeypatch):
    real = Q.quantize

    def no_adjust(x, group_size=64, bits=8):
        x = np.asarray(x, np.float32)
        g = x.reshape(-1, group_size)
        nb = np.float32((1 << bits) - 1)
        mx_, mn_ = g.max(1), g.min(1)
        d = np.maximum((mx_ - mn_) / nb, Q.EPS).astype(np.float32)
        side = np.abs(mn_) > np.abs(mx_)
        sc = np.where(side, d, -d).astype(np.float32)
        bi = np.where(side, mn_, mx_).astype(np.float32)
        c = np.minimum(Q.round_half_away((g - bi[:, None]) / sc[:, None]), nb).astype(np.uint8)
        return (c.reshape(x.shape), Q.f32_to_bf16_bits(sc)[None], Q.f32_to_bf16_bits(bi)[None])

    monkeypatch.setattr(Q, "quantize", no_adjust)
    with pytest.raises(AssertionError):
        test_q0_adjustment_4bit()
    monkeypatch.setattr(Q, "quantize", real)


def test_planted_nibble_swap_is_caught(monkeypatch):
    monkeypatch.setattr(Q, "pack_codes",
                        lambda c, bits: (np.asarray(c)[..., 1::2] | (np.asarray(c)[..., 0::2] << 4)).astype(np.uint8))
    with pytest.raises(AssertionError):
        test_4bit_nibbles_even_low()


def test_planted_no_bf16_rounding_in_dequant_is_caught(monkeypatch):
    # dequantize must return bf16 values; dropping the rounding leaves fp32 values with low bits
    rng = np.random.default_rng(4)
    x = Q.randn_bf16(rng, (8, 64))
    c, s, b = Q.quantize(x, 64, 8)
    y = Q.dequantize(c, s, b, 64, 8)
    assert (Q.round_bf16(y) == y).all()
    y2 = Q.dequantize_f32(c, s, b, 64, 8)
    assert not (Q.round_bf16(y2) == y2).all()
