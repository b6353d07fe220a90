"""Affine group quantization of K/V rows on the GPU (liblaguna_hip.so).

``quantize`` / ``dequantize`` mirror ``mx.quantize`` / ``mx.dequantize`` as the reference's cache
uses them (``laguna_mlx/cache.py:90,100``; ``scripts/micro_kv_decode.py:36``), returning the cache
layout: codes uint8 ``[..., D * bits // 8]`` (8-bit: one byte per element; 4-bit: two per byte,
even element in the low nibble), bf16 scales and biases ``[..., D // group_size]``.
``quantize_into`` is the quantize-on-append primitive: it writes rows ``[offset, offset + L)`` of
existing full-capacity cache buffers in place; ``quantize_kv_into`` does K and V in one launch.
"""
from __future__ import annotations

import torch

from . import _lib


def _check_bits(bits, group_size):
    if bits not in (4, 8):
        raise ValueError(f"bits must be 4 or 8, got {bits}")
    if group_size not in (32, 64, 128):
        raise ValueError(f"group_size must be 32, 64 or 128, got {group_size}")


def _check_append(x, codes, scales, biases, group_size, bits):
    if x.dtype != torch.bfloat16:
        raise ValueError(f"K/V rows must be bfloat16, got {x.dtype}")
    if x.dim() != 4:
        raise ValueError(f"expected [B, H, L, D], got {tuple(x.shape)}")
    B, H, L, D = x.shape
    if D % group_size:
        raise ValueError(f"head_dim {D} is not a multiple of group_size {group_size}")
    cap = codes.shape[2]
    want_c = (B, H, cap, D * bits // 8)
    want_s = (B, H, cap, D // group_size)
    if tuple(codes.shape) != want_c or codes.dtype != torch.uint8 or not codes.is_contiguous():
        raise ValueError(f"codes must be contiguous uint8 {want_c}, got {tuple(codes.shape)} {codes.dtype}")
    for t in (scales, biases):
        if tuple(t.shape) != want_s or t.dtype != torch.bfloat16 or not t.is_contiguous():
            raise ValueError(f"scales/biases must be contiguous bf16 {want_s}")
    return x.contiguous(), cap


def quantize_into(x: torch.Tensor, codes: torch.Tensor, scales: torch.Tensor,
                  biases: torch.Tensor, offset: int, group_size: int = 64, bits: int = 8):
    """Quantize ``x [B, H, L, D]`` (bf16) into rows ``[offset, offset+L)`` of the cache buffers
    ``codes [B, H, cap, D*bits/8]`` (uint8), ``scales``/``biases [B, H, cap, D/group]`` (bf16)."""
    lib = _lib.load()
    _check_bits(bits, group_size)
    dev = _lib.require_device(x, codes, scales, biases)
    x, cap = _check_append(x, codes, scales, biases, group_size, bits)
    B, H, L, D = x.shape
    st = lib.lq_quantize_append(x.data_ptr(), B, H, L, D, codes.data_ptr(), scales.data_ptr(),
                                biases.data_ptr(), cap, int(offset), bits, group_size,
                                _lib.stream_ptr(dev))
    _lib.check(st, "lq_quantize_append")


def quantize_kv_into(k: torch.Tensor, v: torch.Tensor, kbuf, vbuf, offset: int,
                     group_size: int = 64, bits: int = 8):
    """:func:`quantize_into` of the keys into ``kbuf`` and of the values into ``vbuf`` (each a
    ``(codes, scales, biases)`` tuple of one cache) in a single launch."""
    lib = _lib.load()
    _check_bits(bits, group_size)
    dev = _lib.require_device(k, v, *kbuf, *vbuf)
    k, cap = _check_append(k, *kbuf, group_size, bits)
    v, cap_v = _check_append(v, *vbuf, group_size, bits)
    if k.shape != v.shape or cap != cap_v:
        raise ValueError(f"K {tuple(k.shape)} and V {tuple(v.shape)} rows or capacities differ")
    B, H, L, D = k.shape
    st = lib.lq_quantize_append_kv(k.data_ptr(), v.data_ptr(), B, H, L, D, kbuf[0].data_ptr(),
                                   kbuf[1].data_ptr(), kbuf[2].data_ptr(), vbuf[0].data_ptr(),
                                   vbuf[1].data_ptr(), vbuf[2].data_ptr(), cap, int(offset), bits,
                                   group_size, _lib.stream_ptr(dev))
    _lib.check(st, "lq_quantize_append_kv")


def quantize(w: torch.Tensor, group_size: int = 64, bits: int = 8):
    """``mx.quantize`` equivalent for bf16 ``w [..., D]``: returns (codes, scales, biases)."""
    _check_bits(bits, group_size)
    *lead, D = w.shape
    rows = 1
    for s in lead:
        rows *= s
    x = w.reshape(1, 1, rows, D)
    codes = torch.empty((1, 1, rows, D * bits // 8), dtype=torch.uint8, device=w.device)
    scales = torch.empty((1, 1, rows, D // group_size), dtype=torch.bfloat16, device=w.device)
    biases = torch.empty_like(scales)
    quantize_into(x, codes, scales, biases, 0, group_size, bits)
    return (codes.reshape(*lead, D * bits // 8), scales.reshape(*lead, D // group_size),
            biases.reshape(*lead, D // group_size))


def dequantize(codes: torch.Tensor, scales: torch.Tensor, biases: torch.Tensor,
               group_size: int = 64, bits: int = 8, n: int | None = None) -> torch.Tensor:
    """``mx.dequantize`` equivalent: rows ``[0, n)`` of ``[B, H, cap, .]`` cache buffers (or of
    any ``[..., rows, .]`` tensors) to bf16 ``[..., n, D]``."""
    lib = _lib.load()
    _check_bits(bits, group_size)
    dev = _lib.require_device(codes, scales, biases)
    if codes.dtype in (torch.int32, torch.uint32):
        codes = codes.contiguous().view(torch.uint8)
    lead = codes.shape[:-2]
    cap, nb = codes.shape[-2], codes.shape[-1]
    D = nb * 8 // bits
    n = cap if n is None else int(n)
    BH = 1
    for s in lead:
        BH *= s
    c = codes.contiguous()
    s_, b_ = scales.contiguous(), biases.contiguous()
    if s_.dtype != torch.bfloat16 or b_.dtype != torch.bfloat16:
        raise ValueError("scales/biases must be bfloat16")
    out = torch.empty((*lead, n, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_dequantize(c.data_ptr(), s_.data_ptr(), b_.data_ptr(), 1, BH, cap, n, D, bits,
                           group_size, out.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(st, "lq_dequantize")
    return out
