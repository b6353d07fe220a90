"""Fused attention over the quantized KV cache, on liblaguna_hip.so.

Drop-in for ``laguna_mlx/q8_attn.py``: :func:`q8_decode_attention` keeps the reference signature
``q8_decode_attention(q, keys, values, n, scale)`` (``q8_attn.py:102``), its argument meaning
(full-capacity ``(codes, scales, biases)`` tuples of which the first ``n`` rows are valid, output
``[B, Hq, 1, D]`` in q's dtype) and its error behaviour (``AssertionError`` for a non-decode
query, a head_dim other than 128, a cache that is not 8-bit, or too many query heads per KV head,
``q8_attn.py:110-115``). Codes may be given as uint8 ``[..., D]`` or as MLX-style 32-bit words
``[..., D // 4]`` (int32/uint32; byte-identical on little-endian hosts).

Additions behind the same layout: ragged batches with per-sequence
lengths (:func:`decode_attention` with ``lens``), the multi-query causal verify step
(:func:`q8_verify_attention`), and 4-bit / plain-bf16 caches (:func:`decode_attention` with
``kind``).
"""
from __future__ import annotations

import torch

from . import _lib

BLOCK = 512  # key-block size of the reference kernel (q8_attn.py:14); kept for callers that import it

_workspaces: dict = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-(device, stream) attention workspace, grown on demand. Calls on one stream are ordered,
    so reuse is safe; different streams get different buffers. A new buffer starts zeroed: its
    first LQ_WS_ZERO_BYTES bytes are the kernels' arrival and tile counters, which every call
    leaves at zero, so only attention calls may use it."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _workspaces.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.zeros(max(nbytes, 1 << 16), dtype=torch.uint8, device=device)
        _workspaces[key] = ws
    return ws


def _checked(status: int, what: str, ws: torch.Tensor):
    """``_lib.check`` for calls that use an attention workspace. A HIP-side failure (a launch that
    did not start, or a merge launch that failed after the attention kernel ran) can leave the
    workspace's arrival and tile counters non-zero, and every later call on that stream would then
    merge too early or skip tiles without an error: the counter area is cleared (on the call's
    stream, ordered after whatever did run) before the error is raised. Argument errors return
    before any launch and leave it untouched."""
    if status == _lib.LQ_EHIP:
        ws[:_lib.LQ_WS_ZERO_BYTES].zero_()
    _lib.check(status, what)


def reset_workspaces():
    """Clears the counter area of every cached attention workspace (queued on the streams they
    belong to). For callers that abandoned a stream's work part way -- an attention launch that
    was aborted or never completed leaves its counters non-zero."""
    for (device, stream), ws in _workspaces.items():
        with torch.cuda.stream(torch.cuda.ExternalStream(stream, device=device)):
            ws[:_lib.LQ_WS_ZERO_BYTES].zero_()


def _as_bytes(codes: torch.Tensor) -> torch.Tensor:
    """Cache codes as a contiguous uint8 tensor [B, H, cap, row_bytes]."""
    if codes.dtype in (torch.int32, torch.uint32):
        codes = codes.contiguous().view(torch.uint8)
    if codes.dtype != torch.uint8:
        raise ValueError(f"cache codes must be uint8 or 32-bit words, got {codes.dtype}")
    return codes.contiguous()


def _bf16(t: torch.Tensor, what: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{what} must be bfloat16, got {t.dtype}")
    return t.contiguous()


def _kind_of(keys, D: int) -> int:
    codes = keys[0]
    row = codes.shape[-1] * (4 if codes.dtype in (torch.int32, torch.uint32) else 1)
    if codes.dtype == torch.bfloat16:
        return _lib.LQ_KV_BF16
    if row == D:
        return _lib.LQ_KV_Q8
    if row == D // 2:
        return _lib.LQ_KV_Q4
    raise ValueError(f"cache rows of {row} bytes do not match head_dim {D} at 8 or 4 bits")


def _decode_operands(q, keys, values):
    """Validated operands of a decode call: (kind, q, (kc, ks, kb), (vc, vs, vb), Hkv, cap)."""
    if not isinstance(keys, (tuple, list)):
        keys, values = (keys, None, None), (values, None, None)
    B, Hq, L, D = q.shape
    if L != 1:
        raise ValueError("decode_attention takes one query row per sequence")
    kind = _kind_of(keys, D)
    kc, ks, kb = keys
    vc, vs, vb = values
    _lib.require_device(q, kc, ks, kb, vc, vs, vb)
    q = _bf16(q, "q")
    if kind == _lib.LQ_KV_BF16:
        kc, vc = _bf16(kc, "keys"), _bf16(vc, "values")
        ks = kb = vs = vb = None
    else:
        kc, vc = _as_bytes(kc), _as_bytes(vc)
        ks, kb, vs, vb = (_bf16(t, "scales/biases") for t in (ks, kb, vs, vb))
    if kc.dim() != 4:
        raise ValueError(f"cache codes must be [B, Hkv, cap, .], got {tuple(kc.shape)}")
    Hkv, cap = kc.shape[1], kc.shape[2]
    row = {_lib.LQ_KV_Q8: D, _lib.LQ_KV_Q4: D // 2, _lib.LQ_KV_BF16: D}[kind]
    for t in (kc, vc):
        if tuple(t.shape) != (B, Hkv, cap, row):
            raise ValueError(f"cache buffer {tuple(t.shape)} does not match {(B, Hkv, cap, row)}")
    if kind != _lib.LQ_KV_BF16:
        for t in (ks, kb, vs, vb):
            if tuple(t.shape) != (B, Hkv, cap, D // 64):
                raise ValueError(f"scales/biases {tuple(t.shape)} do not match {(B, Hkv, cap, D // 64)}")
    if Hkv < 1 or Hq % Hkv:
        raise ValueError(f"{Hq} query heads are not a multiple of {Hkv} KV heads")
    return kind, q, (kc, ks, kb), (vc, vs, vb), Hkv, cap


def _lens(lens, B):
    lens_list = [int(x) for x in (lens.tolist() if torch.is_tensor(lens) else lens)]
    if len(lens_list) != B:
        raise ValueError(f"lens has {len(lens_list)} entries for a batch of {B}")
    return lens_list


def decode_attention(q: torch.Tensor, keys, values, n: int | None = None, scale: float = None,
                     lens=None) -> torch.Tensor:
    """Single-token attention over a quantized (or plain bf16) KV cache.

    q [B, Hq, 1, 128] bf16. ``keys``/``values``: ``(codes, scales, biases)`` of shape
    ``[B, Hkv, cap, .]`` (8- or 4-bit, group 64), or a plain bf16 tensor ``[B, Hkv, cap, 128]``.
    Either ``n`` (every sequence has ``n`` valid rows) or ``lens`` (B lengths; ragged batch).
    Returns ``[B, Hq, 1, 128]`` bf16.
    """
    lib = _lib.load()
    kind, q, (kc, ks, kb), (vc, vs, vb), Hkv, cap = _decode_operands(q, keys, values)
    B, Hq, _, D = q.shape
    dev = q.device
    lens_arr = None
    if lens is not None:
        lens_list = _lens(lens, B)
        lens_arr = _lib.C.cast((_lib.C.c_int32 * B)(*lens_list), _lib.C.c_void_p)
        n = 0
    elif n is None:
        raise ValueError("give n or lens")
    if scale is None:
        scale = D ** -0.5
    ws_bytes = lib.lq_decode_workspace_bytes(kind, B, Hq, Hkv, D, int(n), lens_arr)
    if ws_bytes < 0:
        raise ValueError(lib.lq_last_error().decode())
    ws = _workspace(dev, ws_bytes)
    out = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_decode_attn(kind, q.data_ptr(), kc.data_ptr(), _lib.ptr(ks), _lib.ptr(kb),
                            vc.data_ptr(), _lib.ptr(vs), _lib.ptr(vb), B, Hq, Hkv, D, cap, int(n),
                            lens_arr, float(scale), out.data_ptr(), ws.data_ptr(), ws.numel(),
                            _lib.stream_ptr(dev))
    _checked(st, "lq_decode_attn", ws)
    return out


def decode_append_attention(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, keys,
                            values, n: int | None = None, scale: float = None,
                            lens=None) -> torch.Tensor:
    """One fused decode step on the 8-bit cache: quantize-append the new rows ``k_new``/``v_new``
    (bf16 ``[B, Hkv, 1, 128]``) at row ``n`` (``lens[b]``) of the full-capacity ``keys``/``values``
    tuples, then attend over ``n + 1`` (``lens[b] + 1``) rows -- ``update_and_fetch`` followed by
    ``attend`` (``laguna_mlx/cache.py:89-106``), the append inside the attention kernel (one launch
    when Hq / Hkv <= 4, plus the split-merge launch above that).
    ``n`` and ``lens`` count the rows before the append. Returns ``[B, Hq, 1, 128]`` bf16."""
    lib = _lib.load()
    kind, q, (kc, ks, kb), (vc, vs, vb), Hkv, cap = _decode_operands(q, keys, values)
    if kind != _lib.LQ_KV_Q8:
        raise ValueError("the fused decode step runs on the 8-bit cache only")
    B, Hq, _, D = q.shape
    dev = q.device
    _lib.require_device(k_new, v_new)
    k_new, v_new = _bf16(k_new, "new keys"), _bf16(v_new, "new values")
    for t in (k_new, v_new):
        if tuple(t.shape) != (B, Hkv, 1, D):
            raise ValueError(f"new rows {tuple(t.shape)} do not match {(B, Hkv, 1, D)}")
    for t in (*keys, *values):
        if not t.is_contiguous():
            raise ValueError("the fused decode step writes the cache in place: its buffers must "
                             "be contiguous")
    lens_arr = after = None
    if lens is not None:
        lens_list = _lens(lens, B)
        lens_arr = _lib.C.cast((_lib.C.c_int32 * B)(*lens_list), _lib.C.c_void_p)
        after = _lib.C.cast((_lib.C.c_int32 * B)(*[x + 1 for x in lens_list]), _lib.C.c_void_p)
        n = 0
    elif n is None:
        raise ValueError("give n or lens")
    if scale is None:
        scale = D ** -0.5
    ws_bytes = lib.lq_decode_workspace_bytes(kind, B, Hq, Hkv, D, int(n) + 1, after)
    if ws_bytes < 0:
        raise ValueError(lib.lq_last_error().decode())
    ws = _workspace(dev, ws_bytes)
    out = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_q8_decode_append_attn(q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
                                      kc.data_ptr(), ks.data_ptr(), kb.data_ptr(), vc.data_ptr(),
                                      vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, D, cap, int(n),
                                      lens_arr, float(scale), out.data_ptr(), ws.data_ptr(),
                                      ws.numel(), _lib.stream_ptr(dev))
    _checked(st, "lq_q8_decode_append_attn", ws)
    return out


def q8_decode_attention(q, keys, values, n, scale):
    """q [B, Hq, 1, D]; keys/values: the cache's full-capacity (codes, scales, biases) tuples,
    of which the first ``n`` rows are valid. Returns [B, Hq, 1, D] in q's dtype
    (``laguna_mlx/q8_attn.py:102-130``)."""
    B, Hq, L, D = q.shape
    if not (L == 1 and D == 128):
        raise AssertionError("decode only, head_dim 128")
    codes = keys[0]
    words = codes.shape[-1] * (1 if codes.dtype == torch.uint8 else 4) // 4
    if words != D // 4:
        raise AssertionError("8-bit, group_size 64 only")
    hkv = codes.shape[1]
    G = Hq // hkv
    if G > 16 or Hq % hkv:
        raise AssertionError(f"{G} q heads per kv head is too many for one workgroup")
    out = decode_attention(q.to(torch.bfloat16), keys, values, n=int(n), scale=scale)
    return out.to(q.dtype)


def _full_capacity(t: torch.Tensor):
    """``(buffer, n)`` for a row-prefix view ``t = buf[:, :, :n]`` of a contiguous full-capacity
    cache buffer ``buf [B, H, cap, w]`` (what ``update_and_fetch`` returns): the buffer is rebuilt
    as a strided view of the same storage, so the kernels read it in place. Any other layout is
    copied to a contiguous tensor (then cap = n)."""
    B, H, n, w = t.shape
    s0, s1, s2, s3 = t.stride()
    if s3 == 1 and s2 == w and w > 0 and s1 % w == 0 and s1 // w >= n and s0 == H * s1:
        cap = s1 // w
        need = (t.storage_offset() + B * H * cap * w) * t.element_size()
        if need <= t.untyped_storage().nbytes():
            return t.as_strided((B, H, cap, w), (s0, s1, s2, 1)), n
    return t.contiguous(), n


def quantized_scaled_dot_product_attention(queries, q_keys, q_values, scale, mask=None,
                                           group_size=64, bits=8):
    """Attention over the packed ``(codes, scales, biases)`` views that a ``quantized_decode``
    step hands the caller -- the routing mlx-lm's SDPA takes when ``hasattr(cache, "bits")``
    (``laguna_mlx/cache.py:73-77,95-98``; ``docs/interfaces.md:29``). ``q_keys``/``q_values`` are
    the first ``offset`` rows of the cache buffers; the kernel reads them in place (8- or 4-bit,
    group 64). Single query rows (the steps on which the cache exposes ``bits``) take the decode
    kernels; an 8-bit block of up to 16 rows with the bottom-right causal mask takes the verify
    kernel. Returns ``[B, Hq, L, 128]`` in the queries' dtype."""
    if group_size != 64:
        raise ValueError(f"quantized attention takes group_size 64, got {group_size}")
    B, Hq, L, D = queries.shape
    kc, n = _full_capacity(q_keys[0])
    vc, _ = _full_capacity(q_values[0])
    keys = (kc,) + tuple(_full_capacity(t)[0] for t in q_keys[1:])
    values = (vc,) + tuple(_full_capacity(t)[0] for t in q_values[1:])
    row = kc.shape[-1] * (4 if kc.dtype in (torch.int32, torch.uint32) else 1)
    if row * 8 != D * bits:
        raise ValueError(f"cache rows of {row} bytes are not {bits}-bit codes of {D} dims")
    if L == 1:
        if mask is not None and not isinstance(mask, str):
            if not bool(torch.as_tensor(mask).all()):
                raise ValueError("a single query row over the cache takes no mask")
        out = decode_attention(queries.to(torch.bfloat16), keys, values, n=n, scale=scale)
        return out.to(queries.dtype)
    if bits != 8 or L > 16 or mask not in ("causal",):
        raise ValueError("multi-row quantized attention takes the 8-bit cache, at most 16 rows "
                         "and the causal mask")
    return q8_verify_attention(queries, keys, values, n, scale)


def q8_verify_attention(q, keys, values, n, scale):
    """Multi-query causal attention for a verify block over the 8-bit cache.

    q [B, Hq, L, 128] with 1 <= L <= 16; the block's own L keys are the last L of the first
    ``n`` cache rows; query row i sees keys 0 .. n-L+i (bottom-right causal, as the reference's
    verify forward masks it, ``laguna_mlx/laguna.py:183-186``). Returns [B, Hq, L, 128] in q's
    dtype."""
    lib = _lib.load()
    B, Hq, L, D = q.shape
    if D != 128 or not 1 <= L <= 16:
        raise ValueError("verify needs head_dim 128 and 1 <= L <= 16")
    kc, ks, kb = keys
    vc, vs, vb = values
    dev = _lib.require_device(q, kc, ks, kb, vc, vs, vb)
    qb = _bf16(q.to(torch.bfloat16), "q")
    kc, vc = _as_bytes(kc), _as_bytes(vc)
    if kc.shape[-1] != D:
        raise ValueError("verify runs on the 8-bit cache only")
    ks, kb, vs, vb = (_bf16(t, "scales/biases") for t in (ks, kb, vs, vb))
    Hkv, cap = kc.shape[1], kc.shape[2]
    for t in (kc, vc):
        if tuple(t.shape) != (B, Hkv, cap, D):
            raise ValueError(f"cache buffer {tuple(t.shape)} does not match {(B, Hkv, cap, D)}")
    for t in (ks, kb, vs, vb):
        if tuple(t.shape) != (B, Hkv, cap, D // 64):
            raise ValueError(f"scales/biases {tuple(t.shape)} do not match {(B, Hkv, cap, D // 64)}")
    if not L <= int(n) <= cap:
        raise ValueError(f"n={n} must cover the {L} block rows and fit the capacity {cap}")
    ws_bytes = lib.lq_verify_workspace_bytes(B, Hq, Hkv, L, D, int(n))
    if ws_bytes < 0:
        raise ValueError(lib.lq_last_error().decode())
    ws = _workspace(dev, ws_bytes)
    out = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_q8_verify_attn(qb.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                               vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, L, D, cap,
                               int(n), float(scale), out.data_ptr(), ws.data_ptr(), ws.numel(),
                               _lib.stream_ptr(dev))
    _checked(st, "lq_q8_verify_attn", ws)
    return out.to(q.dtype)


def q8_verify_append_attention(q, k_new, v_new, keys, values, n, scale):
    """One fused verify step on the 8-bit cache: quantize-append the block's ``L`` new rows
    ``k_new``/``v_new`` (bf16 ``[B, Hkv, L, 128]``) at rows ``n .. n+L-1`` of the full-capacity
    ``keys``/``values`` tuples, then the causal verify attention of :func:`q8_verify_attention`
    over the ``n + L`` rows -- ``update_and_fetch`` then the verify forward's attention
    (``laguna_mlx/cache.py:89-100``, ``laguna.py:107``), the append inside the attention kernel
    when G * L > 4. ``n`` counts the rows before the append. Returns [B, Hq, L, 128] in q's
    dtype."""
    lib = _lib.load()
    B, Hq, L, D = q.shape
    if D != 128 or not 1 <= L <= 16:
        raise ValueError("verify needs head_dim 128 and 1 <= L <= 16")
    kc, ks, kb = keys
    vc, vs, vb = values
    dev = _lib.require_device(q, k_new, v_new, kc, ks, kb, vc, vs, vb)
    qb = _bf16(q.to(torch.bfloat16), "q")
    kc, vc = _as_bytes(kc), _as_bytes(vc)
    if kc.shape[-1] != D:
        raise ValueError("verify runs on the 8-bit cache only")
    ks, kb, vs, vb = (_bf16(t, "scales/biases") for t in (ks, kb, vs, vb))
    Hkv, cap = kc.shape[1], kc.shape[2]
    for t in (kc, vc):
        if tuple(t.shape) != (B, Hkv, cap, D):
            raise ValueError(f"cache buffer {tuple(t.shape)} does not match {(B, Hkv, cap, D)}")
    for t in (ks, kb, vs, vb):
        if tuple(t.shape) != (B, Hkv, cap, D // 64):
            raise ValueError(f"scales/biases {tuple(t.shape)} do not match {(B, Hkv, cap, D // 64)}")
    for t in (*keys, *values):
        if not t.is_contiguous():
            raise ValueError("the fused verify step writes the cache in place: its buffers must "
                             "be contiguous")
    k_new, v_new = _bf16(k_new, "new keys"), _bf16(v_new, "new values")
    for t in (k_new, v_new):
        if tuple(t.shape) != (B, Hkv, L, D):
            raise ValueError(f"new rows {tuple(t.shape)} do not match {(B, Hkv, L, D)}")
    if not (0 <= int(n) and int(n) + L <= cap):
        raise ValueError(f"n={n} + {L} new rows must fit the capacity {cap}")
    ws_bytes = lib.lq_verify_workspace_bytes(B, Hq, Hkv, L, D, int(n) + L)
    if ws_bytes < 0:
        raise ValueError(lib.lq_last_error().decode())
    ws = _workspace(dev, ws_bytes)
    out = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_q8_verify_append_attn(qb.data_ptr(), k_new.data_ptr(), v_new.data_ptr(),
                                      kc.data_ptr(), ks.data_ptr(), kb.data_ptr(), vc.data_ptr(),
                                      vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, L, D, cap, int(n),
                                      float(scale), out.data_ptr(), ws.data_ptr(), ws.numel(),
                                      _lib.stream_ptr(dev))
    _checked(st, "lq_q8_verify_append_attn", ws)
    return out.to(q.dtype)


def q8_prefill_attention(q, keys, values, n, scale):
    """Causal attention of a prefill chunk over the 8-bit cache, without materializing the score
    matrix or a dequantized copy of the cache (the step before decode: ``L`` > 1 chunks on the
    quantized cache, ``laguna_mlx/cache.py:99-100``, whose reference path dequantizes the whole
    cache and runs SDPA; ``tests/test_cache.py:79-93`` guards its peak memory).

    q [B, Hq, L, 128] for the chunk's positions n-L .. n-1, whose K/V are already the last L of
    the first ``n`` cache rows; row i sees keys 0 .. n-L+i. Any L >= 1. Chunks of more than 16
    rows with 1, 2, 4 or 8 query heads per KV head run ``lq_q8_prefill_attn`` (one launch: 256
    query rows per workgroup over shared, once-dequantized K/V tiles); other shapes go through
    the verify kernel block by block. Returns [B, Hq, L, 128] in q's dtype."""
    B, Hq, L, D = q.shape
    kc, ks, kb = keys
    Hkv = kc.shape[1]
    if D != 128 or Hkv < 1 or Hq % Hkv:
        raise ValueError("prefill needs head_dim 128 and Hq a multiple of Hkv")
    if L <= 16:
        return q8_verify_attention(q, keys, values, n, scale)
    if Hq // Hkv not in (1, 2, 4, 8):
        return _prefill_blocked(q, keys, values, n, scale)
    lib = _lib.load()
    vc, vs, vb = values
    dev = _lib.require_device(q, kc, ks, kb, vc, vs, vb)
    qb = _bf16(q.to(torch.bfloat16), "q")
    kc, vc = _as_bytes(kc), _as_bytes(vc)
    if kc.shape[-1] != D:
        raise ValueError("prefill runs on the 8-bit cache only")
    ks, kb, vs, vb = (_bf16(t, "scales/biases") for t in (ks, kb, vs, vb))
    cap = kc.shape[2]
    for t in (kc, vc):
        if tuple(t.shape) != (B, Hkv, cap, D):
            raise ValueError(f"cache buffer {tuple(t.shape)} does not match {(B, Hkv, cap, D)}")
    for t in (ks, kb, vs, vb):
        if tuple(t.shape) != (B, Hkv, cap, D // 64):
            raise ValueError(f"scales/biases {tuple(t.shape)} do not match {(B, Hkv, cap, D // 64)}")
    if not L <= int(n) <= cap:
        raise ValueError(f"n={n} must cover the {L} chunk rows and fit the capacity {cap}")
    out = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=dev)
    st = lib.lq_q8_prefill_attn(qb.data_ptr(), kc.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                vc.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, L, D, cap,
                                int(n), float(scale), out.data_ptr(), _lib.stream_ptr(dev))
    _lib.check(st, "lq_q8_prefill_attn")
    return out.to(q.dtype)


def _prefill_blocked(q, keys, values, n, scale):
    """q8_prefill_attention for any head grouping: blocks of P = min(16, 64 / G) positions through
    the verify kernel (one launch and one merge per block; a ragged first block of L mod P rows),
    each block over the keys its last row sees."""
    lib = _lib.load()
    B, Hq, L, D = q.shape
    kc, ks, kb = keys
    Hkv = kc.shape[1]
    G = Hq // Hkv
    if G > 64:
        raise ValueError(f"{G} query heads per KV head exceed 64")
    P = max(1, min(16, 64 // G))
    if L <= P:
        return q8_verify_attention(q, keys, values, n, scale)
    n = int(n)
    if not L <= n:
        raise ValueError(f"n={n} must cover the {L} chunk rows")
    r = L % P
    out = torch.empty((B, Hq, L, D), dtype=torch.bfloat16, device=q.device)
    if r:
        out[:, :, :r] = q8_verify_attention(q[:, :, :r].contiguous(), keys, values, n - L + r,
                                            scale).to(torch.bfloat16)
    nb = (L - r) // P
    qb = q[:, :, r:].to(torch.bfloat16).reshape(B, Hq, nb, P, D).permute(2, 0, 1, 3, 4).contiguous()
    # one validation pass through the checked wrapper (block 0), then the same call per block
    ob = torch.empty_like(qb)
    ob[0] = q8_verify_attention(qb[0], keys, values, n - L + r + P, scale).to(torch.bfloat16)
    vc, vs, vb = values
    kc8, vc8 = _as_bytes(kc), _as_bytes(vc)
    ks, kb, vs, vb = (_bf16(t, "scales/biases") for t in (ks, kb, vs, vb))
    cap = kc8.shape[2]
    dev = q.device
    ws_bytes = lib.lq_verify_workspace_bytes(B, Hq, Hkv, P, D, n)
    if ws_bytes < 0:
        raise ValueError(lib.lq_last_error().decode())
    ws = _workspace(dev, ws_bytes)
    sp = _lib.stream_ptr(dev)
    blk = B * Hq * P * D * 2  # bytes per block of qb / ob
    q0, o0 = qb.data_ptr(), ob.data_ptr()
    for j in range(1, nb):
        st = lib.lq_q8_verify_attn(q0 + j * blk, kc8.data_ptr(), ks.data_ptr(), kb.data_ptr(),
                                   vc8.data_ptr(), vs.data_ptr(), vb.data_ptr(), B, Hq, Hkv, P, D,
                                   cap, n - L + r + P * (j + 1), float(scale), o0 + j * blk,
                                   ws.data_ptr(), ws.numel(), sp)
        _checked(st, "lq_q8_verify_attn", ws)
    out[:, :, r:] = ob.permute(1, 2, 0, 3, 4).reshape(B, Hq, L - r, D)
    return out.to(q.dtype)
