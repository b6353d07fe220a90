"""Oracle: MLX affine quantize / dequantize (group-wise, 8- or 4-bit) and bf16 helpers.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

What it restates. The reference appends K/V through mlx-lm 0.31.3's ``QuantizedKVCache``
(``laguna_mlx/cache.py:83,90``), which calls ``mx.quantize(x, group_size, bits)`` of MLX 0.32.0
(``README.md:161``; also ``scripts/micro_kv_decode.py:36``). The unfused path dequantizes with
``mx.dequantize`` (``cache.py:100``). MLX is a third-party dependency that is not present under
the reference tree, so its published algorithm (the Metal ``affine_quantize`` kernel) is restated
here, per 64-element group of fp32 values ``x``::

    n_bins = 2**bits - 1
    delta  = max((max(x) - min(x)) / n_bins, 1e-7)
    side   = |min(x)| > |max(x)|
    scale  = delta if side else -delta
    edge   = min(x) if side else max(x)
    q0     = round(edge / scale)
    scale, bias = (edge / q0, edge) if q0 != 0 else (scale, 0)
    code_i = min(round((x_i - bias) / scale), n_bins)
    stored scale, bias = bf16(scale), bf16(bias)        (round to nearest even)

``round`` is Metal's ``round``: halves away from zero. All arithmetic is IEEE fp32 with correctly
rounded division. The codes are computed from the fp32 scale/bias, the stored values are their
bf16 roundings. Layout (``q8_attn.py:8-10``): 8-bit codes are bytes in element order, which is
byte-identical to MLX's uint32 packing (4 codes per word, low byte first); 4-bit codes are two
per byte, the even element in the low nibble (8 per uint32, low nibble first).

Dequantize: ``bf16(fp32(scale) * code + fp32(bias))``, one fp32 product and sum, rounded to bf16.

Parity status. No MLX build exists anywhere in this pipeline, so these functions cannot be
compared with MLX output. They are pinned by hand-derived known answers, by the invariants the
algorithm fixes (range, exact reconstruction of the larger-magnitude edge, chunking invariance,
error bound) and by the reference's own invariant tests (``tests/test_cache.py:50-71``). Codes and
scales relative to MLX itself stay **parity unpinned** at the MLX boundary; recorded assumptions:
(1) Metal ``round`` is half-away-from-zero, (2) Metal fp32 division is correctly rounded,
(3) the group maximum starts from the first element, not from 0 (differs only for groups whose
64 values are all negative), (4) dequantize rounds once to bf16.
"""
from __future__ import annotations

import numpy as np

F32 = np.float32
EPS = F32(1e-7)


# ----------------------------------------------------------------------------------------------
# bf16 helpers (bit patterns held in uint16)
# ----------------------------------------------------------------------------------------------

def f32_to_bf16_bits(x) -> np.ndarray:
    """fp32 -> bf16 bit pattern, round to nearest even; NaN maps to the quiet NaN 0x7FC0."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(F32)


def round_bf16(x) -> np.ndarray:
    """Values of ``x`` rounded to bf16 (returned as fp32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(x))


def round_half_away(x) -> np.ndarray:
    """Metal/C ``round``: nearest integer, halves away from zero, exact in fp32."""
    x = np.asarray(x, dtype=F32)
    t = np.trunc(x)
    frac = np.abs(x - t)  # exact: x and trunc(x) share the exponent range
    return (t + np.where(frac >= F32(0.5), np.sign(x), F32(0))).astype(F32)


# ----------------------------------------------------------------------------------------------
# quantize / dequantize
# ----------------------------------------------------------------------------------------------

def quantize(x, group_size: int = 64, bits: int = 8):
    """Affine group quantization of fp32 values ``x[..., D]`` (normally bf16-exact).

    Returns ``(codes, scales, biases)``: ``codes`` uint8 ``[..., D]`` (one unpacked code per
    element, use :func:`pack_codes` for the cache layout), ``scales``/``biases`` as bf16 bit
    patterns uint16 ``[..., D // group_size]``.
    """
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    x = np.asarray(x, dtype=F32)
    D = x.shape[-1]
    if D % group_size:
        raise ValueError(f"last dim {D} is not a multiple of group_size {group_size}")
    n_bins = F32((1 << bits) - 1)
    g = x.reshape(-1, group_size)
    w_max = g.max(axis=1)
    w_min = g.min(axis=1)
    delta = np.maximum((w_max - w_min) / n_bins, EPS).astype(F32)
    side = np.abs(w_min) > np.abs(w_max)
    scale = np.where(side, delta, -delta).astype(F32)
    edge = np.where(side, w_min, w_max).astype(F32)
    q0 = round_half_away(edge / scale)
    at_zero = q0 == 0
    with np.errstate(divide="ignore", invalid="ignore"):
        scale = np.where(at_zero, scale, edge / np.where(at_zero, F32(1), q0)).astype(F32)
    bias = np.where(at_zero, F32(0), edge).astype(F32)
    q = round_half_away((g - bias[:, None]) / scale[:, None])
    assert (q >= 0).all(), "affine codes are non-negative by construction"
    codes = np.minimum(q, n_bins).astype(np.uint8)
    lead = x.shape[:-1]
    ng = D // group_size
    return (codes.reshape(*lead, D),
            f32_to_bf16_bits(scale).reshape(*lead, ng),
            f32_to_bf16_bits(bias).reshape(*lead, ng))


def pack_codes(codes, bits: int) -> np.ndarray:
    """Unpacked codes ``[..., D]`` -> cache bytes ``[..., D * bits // 8]``."""
    codes = np.asarray(codes, dtype=np.uint8)
    if bits == 8:
        return codes.copy()
    if bits == 4:
        return (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    raise ValueError("bits must be 4 or 8")


def unpack_codes(packed, bits: int) -> np.ndarray:
    packed = np.asarray(packed, dtype=np.uint8)
    if bits == 8:
        return packed.copy()
    if bits == 4:
        out = np.empty(packed.shape[:-1] + (packed.shape[-1] * 2,), dtype=np.uint8)
        out[..., 0::2] = packed & 0x0F
        out[..., 1::2] = packed >> 4
        return out
    raise ValueError("bits must be 4 or 8")


def mlx_words(codes, bits: int) -> np.ndarray:
    """MLX's uint32 packing of unpacked codes: word j holds 32/bits codes, lowest first."""
    codes = np.asarray(codes, dtype=np.uint32)
    per = 32 // bits
    c = codes.reshape(*codes.shape[:-1], codes.shape[-1] // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(c << shifts, axis=-1).astype(np.uint32)


def quantize_packed(x, group_size: int = 64, bits: int = 8):
    """:func:`quantize` with the codes in the cache layout (:func:`pack_codes`)."""
    c, s, b = quantize(x, group_size, bits)
    return pack_codes(c, bits), s, b


def dequantize(packed, scales, biases, group_size: int = 64, bits: int = 8) -> np.ndarray:
    """Cache bytes + bf16 scale/bias bits -> fp32 values that are exactly bf16."""
    c = unpack_codes(packed, bits).astype(F32)
    D = c.shape[-1]
    s = np.repeat(bf16_bits_to_f32(scales), group_size, axis=-1)[..., :D]
    b = np.repeat(bf16_bits_to_f32(biases), group_size, axis=-1)[..., :D]
    return round_bf16((s * c).astype(F32) + b)


def dequantize_f32(packed, scales, biases, group_size: int = 64, bits: int = 8) -> np.ndarray:
    """Like :func:`dequantize` without the final bf16 rounding (the fused kernel's view,
    ``q8_attn.py:46-55``: ``scale * code + bias`` kept in fp32)."""
    c = unpack_codes(packed, bits).astype(F32)
    D = c.shape[-1]
    s = np.repeat(bf16_bits_to_f32(scales), group_size, axis=-1)[..., :D]
    b = np.repeat(bf16_bits_to_f32(biases), group_size, axis=-1)[..., :D]
    return ((s * c).astype(F32) + b).astype(F32)


def randn_bf16(rng: np.random.Generator, shape) -> np.ndarray:
    """N(0,1) draw rounded to bf16, as fp32 values (the synthetic-input convention)."""
    return round_bf16(rng.standard_normal(shape, dtype=np.float32))
