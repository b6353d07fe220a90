"""KV caches for the quantized decode path (PyTorch-ROCm host side, HIP kernels underneath).

Drop-in for ``laguna_mlx/cache.py``:

* :class:`QuantizedKVCache` -- the mlx-lm 0.31.3 class ``DequantKVCache`` wraps
  (``cache.py:83``): full-capacity buffers grown in steps of 256 rows, quantize-on-append of the
  new rows at ``offset`` (now the HIP kernel ``lq_quantize_append``), views of the first
  ``offset`` rows returned, ``trim`` only moves ``offset``.
* :class:`DequantKVCache` -- same constructor, properties and switches as the reference
  (``cache.py:66-144``): by default multi-token and single-token steps get dequantized bf16 K/V;
  ``quantized_decode`` hands single-token steps the packed tuples and exposes ``bits`` for that
  step only; ``fused_decode`` sets ``fused_step`` and ``attend`` runs the fused HIP kernel.
  Extension (``fused_verify``, default: follows ``fused_decode``): multi-token steps of up to 16
  rows -- the speculative verify block -- also take a fused kernel (causal, bottom-right).
  Extension (``fused_prefill``, default off): longer steps -- prefill chunks -- are quantized
  into the cache and attended straight off it (blocked causal kernel, no dequantized copy, no
  score matrix).
* :func:`make_quantized_cache` -- per-layer factory (``cache.py:147-157``);
  :func:`make_trimmable_cache` / :class:`TrimmableWindowCache` -- the plain bf16 caches of the
  speculative loop (``cache.py:7-63``).
* :class:`RotatingKVCache` -- plain bf16 sliding-window cache for sliding layers (mlx-lm's
  ``RotatingKVCache(max_size=window)``, kept minimal: the last ``max_size`` rows).
"""
from __future__ import annotations

import torch

from .quant import dequantize, quantize_kv_into


def create_attention_mask(N: int, offset: int = 0, return_array: bool = False,
                          window_size: int | None = None):
    """mlx-lm's convention: None for one row, "causal" for several, or a boolean [N, offset+N]
    mask (True = attend) aligned to the bottom-right."""
    if window_size is None and N == 1:
        return None
    if window_size is None and not return_array:
        return "causal"
    q = torch.arange(offset, offset + N)[:, None]
    k = torch.arange(offset + N)[None, :]
    m = k <= q
    if window_size is not None:
        m &= k > q - window_size
    return m


class QuantizedKVCache:
    step = 256

    def __init__(self, group_size: int = 64, bits: int = 8):
        self.group_size, self.bits = group_size, bits
        self.keys = self.values = None  # (codes, scales, biases), full capacity
        self.offset = 0

    def _alloc(self, B, H, rows, D, device):
        return (torch.zeros((B, H, rows, D * self.bits // 8), dtype=torch.uint8, device=device),
                torch.zeros((B, H, rows, D // self.group_size), dtype=torch.bfloat16, device=device),
                torch.zeros((B, H, rows, D // self.group_size), dtype=torch.bfloat16, device=device))

    def update_and_fetch(self, keys: torch.Tensor, values: torch.Tensor):
        prev = self.reserve(keys, values)
        quantize_kv_into(keys, values, self.keys, self.values, prev, self.group_size, self.bits)
        return self.views()

    def views(self):
        """The first ``offset`` rows of the full-capacity buffers, as returned by update_and_fetch."""
        return (tuple(t[:, :, :self.offset] for t in self.keys),
                tuple(t[:, :, :self.offset] for t in self.values))

    def reserve(self, keys: torch.Tensor, values: torch.Tensor) -> int:
        """Grows the buffers (256-row steps) for ``keys``/``values`` and advances ``offset`` over
        them without writing them; returns the first row they go to."""
        B, H, L, Dk = keys.shape
        Dv = values.shape[-1]
        prev = self.offset
        if self.keys is None or prev + L > self.keys[0].shape[2]:
            new_steps = (self.step + L - 1) // self.step * self.step
            if self.keys is None:
                self.keys = self._alloc(B, H, new_steps, Dk, keys.device)
                self.values = self._alloc(B, H, new_steps, Dv, values.device)
            else:
                if prev % self.step != 0:
                    self.keys = tuple(t[:, :, :prev] for t in self.keys)
                    self.values = tuple(t[:, :, :prev] for t in self.values)
                self.keys = tuple(torch.cat([t, z], dim=2) for t, z in
                                  zip(self.keys, self._alloc(B, H, new_steps, Dk, keys.device)))
                self.values = tuple(torch.cat([t, z], dim=2) for t, z in
                                    zip(self.values, self._alloc(B, H, new_steps, Dv, values.device)))
        self.offset += L
        return prev

    @property
    def state(self):
        if self.keys is None:
            return None, None
        if self.offset == self.keys[0].shape[2]:
            return self.keys, self.values
        return (tuple(t[:, :, :self.offset] for t in self.keys),
                tuple(t[:, :, :self.offset] for t in self.values))

    @state.setter
    def state(self, v):
        """mlx-lm's setter: the ``(codes, scales, biases)`` tuples of the valid rows become the
        buffers (contiguous copies) and ``offset`` their row count; the next append grows them."""
        keys, values = v
        if keys is None:
            self.keys = self.values = None
            self.offset = 0
            return
        self.keys = tuple(t.contiguous() for t in keys)
        self.values = tuple(t.contiguous() for t in values)
        self.offset = self.keys[0].shape[2]

    @property
    def meta_state(self):
        return tuple(map(str, (self.step, self.offset, self.group_size, self.bits)))

    @meta_state.setter
    def meta_state(self, v):
        step, self.offset, self.group_size, self.bits = map(int, v)
        if step != self.step:
            raise ValueError(f"saved step {step} differs from {self.step}")

    def make_mask(self, N, return_array=False, window_size=None):
        return create_attention_mask(N, offset=self.offset, return_array=return_array,
                                     window_size=window_size)

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        if self.keys is None:
            return 0
        return sum(t.numel() * t.element_size() for t in (*self.keys, *self.values))


class _PendingRows(tuple):
    """The ``(codes, scales, biases)`` views returned on a fused single-token step. The new row
    is quantized and written by the following ``attend`` (one fused kernel with the attention);
    indexing or unpacking this tuple first completes the append, so its contents are always the
    reference's."""

    def __new__(cls, items, cache):
        obj = super().__new__(cls, items)
        obj._cache = cache
        return obj

    def __getitem__(self, i):
        self._cache._flush()
        return super().__getitem__(i)

    def __iter__(self):
        self._cache._flush()
        return super().__iter__()


class DequantKVCache:
    """Stores K/V quantized and, by default, hands attention dequantized bf16 K/V
    (``laguna_mlx/cache.py:66-144``). No ``bits`` attribute except on single-token
    ``quantized_decode`` steps.

    Fused steps (``fused_decode``; verify blocks of up to 16 rows with ``fused_verify``):
    ``update_and_fetch`` reserves the new rows and ``attend`` quantizes, stores and attends over
    them in the attention launch (``lq_q8_decode_append_attn``, ``lq_q8_verify_append_attn``). Any
    other use of the cache before ``attend`` (``state``, ``trim``, the next ``update_and_fetch``,
    indexing the returned tuples) writes the rows first."""

    def __init__(self, group_size=64, bits=8, quantized_decode=False, fused_decode=False,
                 fused_verify=None, fused_prefill=False):
        if (fused_decode or fused_prefill) and (bits, group_size) != (8, 64):
            raise ValueError("fused_decode needs 8-bit, group_size 64")
        self.q = QuantizedKVCache(group_size=group_size, bits=bits)
        self.quantized_decode = quantized_decode
        self.fused_decode = fused_decode
        self.fused_verify = fused_decode if fused_verify is None else fused_verify
        self.fused_prefill = fused_prefill
        self._quantized_step = False
        self.fused_step = False
        self._pending = None  # (keys, values, row) of a fused step until attend() writes it

    def _flush(self):
        if self._pending is not None:
            k, v, row = self._pending
            self._pending = None
            quantize_kv_into(k, v, self.q.keys, self.q.values, row, self.q.group_size, self.q.bits)

    def update_and_fetch(self, keys, values):
        self._flush()
        L = keys.shape[2]
        # Attention checks `fused_step` and then calls attend(); the K/V returned are unused
        self.fused_step = self.fused_decode and (L == 1 or (self.fused_verify and L <= 16))
        if self.fused_step:
            row = self.q.reserve(keys, values)
            self._pending = (keys, values, row)
            self._quantized_step = False
            qk, qv = self.q.views()
            return _PendingRows(qk, self), _PendingRows(qv, self)
        qk, qv = self.q.update_and_fetch(keys, values)
        if self.fused_prefill and L > 16:  # a prefill chunk: attend() reads the packed cache
            self.fused_step = True
            self._quantized_step = False
            return qk, qv
        self._quantized_step = self.quantized_decode and L == 1
        if self._quantized_step:
            return qk, qv
        g, b = self.q.group_size, self.q.bits
        n = self.q.offset
        return dequantize(*self.q.keys, g, b, n=n), dequantize(*self.q.values, g, b, n=n)

    def attend(self, queries, scale):
        """Attention straight off the packed cache: the fused decode kernel for one query row,
        the fused causal verify kernel for a block of up to 16 rows, the blocked causal kernel
        for longer chunks; the step's pending new rows are appended by the same call."""
        from .q8_attn import (decode_append_attention, q8_decode_attention,
                              q8_prefill_attention, q8_verify_append_attention,
                              q8_verify_attention)

        L = queries.shape[2]
        if self._pending is not None and self._pending[0].shape[2] == L:
            k, v, row = self._pending
            if queries.shape[3] != 128:
                raise AssertionError("head_dim 128")
            self._pending = None
            if L == 1:
                out = decode_append_attention(queries.to(torch.bfloat16), k, v, self.q.keys,
                                              self.q.values, n=row, scale=scale)
                return out.to(queries.dtype)
            return q8_verify_append_attention(queries, k, v, self.q.keys, self.q.values, row,
                                              scale)
        self._flush()
        if L == 1:
            return q8_decode_attention(queries, self.q.keys, self.q.values, self.q.offset, scale)
        if L > 16:
            return q8_prefill_attention(queries, self.q.keys, self.q.values, self.q.offset, scale)
        return q8_verify_attention(queries, self.q.keys, self.q.values, self.q.offset, scale)

    @property
    def bits(self):
        if not self._quantized_step:
            raise AttributeError("bits")  # hasattr(cache, "bits") is False off quantized steps
        return self.q.bits

    @property
    def offset(self):
        return self.q.offset

    @property
    def kv_bits(self):
        return self.q.bits

    @property
    def group_size(self):
        return self.q.group_size

    def make_mask(self, *args, **kwargs):
        return self.q.make_mask(*args, **kwargs)

    @property
    def state(self):
        self._flush()
        return self.q.state

    @state.setter
    def state(self, v):
        """Extension: the reference class has no setter (``docs/architecture.md:347-349``), so its
        prompt caches cannot be loaded; here the packed tuples load into the wrapped cache."""
        self._pending = None
        self._quantized_step = self.fused_step = False
        self.q.state = v

    @property
    def meta_state(self):
        return self.q.meta_state + tuple(
            str(int(x)) for x in (self.quantized_decode, self.fused_decode, self.fused_verify,
                                  self.fused_prefill))

    @meta_state.setter
    def meta_state(self, v):
        self.q.meta_state = v[:4]
        self.quantized_decode, self.fused_decode, self.fused_verify = (bool(int(x)) for x in v[4:7])
        self.fused_prefill = len(v) > 7 and bool(int(v[7]))
        if (self.fused_decode or self.fused_prefill) and (self.q.bits, self.q.group_size) != (8, 64):
            raise ValueError("fused_decode needs 8-bit, group_size 64")

    def is_trimmable(self):
        return True

    def trim(self, n):
        self._flush()
        return self.q.trim(n)

    def empty(self):
        return self.q.empty()

    @property
    def nbytes(self):
        return self.q.nbytes


class KVCache:
    """Plain bf16 cache (mlx-lm ``KVCache``): grows in 256-row steps, returns ``[:offset]``."""

    step = 256

    def __init__(self):
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        B, H, L, D = keys.shape
        prev = self.offset
        if self.keys is None or prev + L > self.keys.shape[2]:
            new = (self.step + L - 1) // self.step * self.step
            zk = torch.zeros((B, H, new, D), dtype=keys.dtype, device=keys.device)
            zv = torch.zeros((B, H, new, values.shape[-1]), dtype=values.dtype, device=values.device)
            if self.keys is None:
                self.keys, self.values = zk, zv
            else:
                self.keys = torch.cat([self.keys[:, :, :prev], zk], dim=2)
                self.values = torch.cat([self.values[:, :, :prev], zv], dim=2)
        self.offset += L
        self.keys[:, :, prev:self.offset] = keys
        self.values[:, :, prev:self.offset] = values
        return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]

    def make_mask(self, N, return_array=False, window_size=None):
        return create_attention_mask(N, offset=self.offset, return_array=return_array,
                                     window_size=window_size)

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(self.offset, n)
        self.offset -= n
        return n

    def empty(self):
        return self.keys is None

    @property
    def state(self):
        if self.keys is None:
            return None, None
        return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]

    @state.setter
    def state(self, v):
        self.keys, self.values = (None, None) if v[0] is None else (v[0].contiguous(), v[1].contiguous())
        self.offset = 0 if self.keys is None else self.keys.shape[2]

    @property
    def meta_state(self):
        return ()

    @meta_state.setter
    def meta_state(self, v):
        if v:
            raise ValueError("KVCache has no meta state")

    @property
    def nbytes(self):
        return 0 if self.keys is None else self.keys.nbytes + self.values.nbytes


class RotatingKVCache:
    """Sliding-window bf16 cache: keeps the last ``max_size`` rows; ``offset`` is absolute."""

    def __init__(self, max_size):
        self.max_size = max_size
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, keys, values):
        if self.keys is None:
            self.keys, self.values = keys, values
        else:
            self.keys = torch.cat([self.keys[:, :, -(self.max_size - 1):], keys], dim=2)
            self.values = torch.cat([self.values[:, :, -(self.max_size - 1):], values], dim=2)
        self.offset += keys.shape[2]
        return self.keys, self.values

    def make_mask(self, N, return_array=False, window_size=None):
        # update_and_fetch keeps the last max_size - 1 rows before appending
        stored = 0 if self.keys is None else min(self.keys.shape[2], self.max_size - 1)
        return create_attention_mask(N, offset=stored, return_array=True,
                                     window_size=window_size or self.max_size)

    def is_trimmable(self):
        return False

    def empty(self):
        return self.keys is None

    @property
    def state(self):
        return self.keys, self.values

    @state.setter
    def state(self, v):
        self.keys, self.values = v

    @property
    def meta_state(self):
        return tuple(map(str, (self.max_size, self.offset)))

    @meta_state.setter
    def meta_state(self, v):
        self.max_size, self.offset = map(int, v)

    @property
    def nbytes(self):
        return 0 if self.keys is None else self.keys.nbytes + self.values.nbytes


class TrimmableWindowCache:
    """Sliding-window bf16 cache for speculative decoding (``laguna_mlx/cache.py:7-55``): keeps
    the last ``window + slack`` rows so that up to ``slack`` rows past the latest update can be
    trimmed; ``offset`` stays the absolute position."""

    def __init__(self, window, slack=64):
        self.window, self.slack = window, slack
        self.keys = self.values = None
        self.offset = 0

    def _stored(self):
        return 0 if self.keys is None else min(self.keys.shape[2], self.window + self.slack)

    def update_and_fetch(self, keys, values):
        if self.keys is None:
            self.keys, self.values = keys, values
        else:
            keep = self.window + self.slack
            self.keys = torch.cat([self.keys[:, :, -keep:], keys], dim=2)
            self.values = torch.cat([self.values[:, :, -keep:], values], dim=2)
        self.offset += keys.shape[2]
        return self.keys, self.values

    def make_mask(self, N, return_array=False, window_size=None):
        return create_attention_mask(N, offset=self._stored(), return_array=True,
                                     window_size=window_size or self.window)

    @property
    def state(self):
        return self.keys, self.values

    @state.setter
    def state(self, v):
        self.keys, self.values = v

    @property
    def meta_state(self):
        return tuple(map(str, (self.window, self.slack, self.offset)))

    @meta_state.setter
    def meta_state(self, v):
        self.window, self.slack, self.offset = map(int, v)

    def is_trimmable(self):
        return True

    def trim(self, n):
        n = min(n, 0 if self.keys is None else self.keys.shape[2])
        if n:
            self.keys, self.values = self.keys[:, :, :-n], self.values[:, :, :-n]
            self.offset -= n
        return n

    def empty(self):
        return self.keys is None

    @property
    def nbytes(self):
        return 0 if self.keys is None else self.keys.nbytes + self.values.nbytes


def make_trimmable_cache(model, slack=64):
    """Plain bf16 caches that speculative decoding can trim (``laguna_mlx/cache.py:58-63``)."""
    return [TrimmableWindowCache(model.args.sliding_window, slack)
            if lt == "sliding_attention" else KVCache()
            for lt in model.args.layer_types]


def make_quantized_cache(model, bits=8, group_size=64, quantized_decode=False, fused_decode=False,
                         trim_slack=None, fused_prefill=False):
    """One cache per layer: a :class:`DequantKVCache` (8- or 4-bit codes) for each full-attention
    layer and a rotating window for each sliding-window layer, as the reference's factory lays
    them out (``laguna_mlx/cache.py:147-157``). Extensions: with ``trim_slack`` the sliding layers get
    :class:`TrimmableWindowCache` with that slack, so that every layer can be trimmed and the
    speculative loop can run over the quantized cache; ``fused_prefill`` is passed to every
    :class:`DequantKVCache`."""
    a = model.args
    if a.head_dim % group_size:
        raise ValueError(f"head_dim {a.head_dim} is not a multiple of group_size {group_size}")

    def window():
        if trim_slack is None:
            return RotatingKVCache(max_size=a.sliding_window)
        return TrimmableWindowCache(a.sliding_window, trim_slack)

    return [
        window() if lt == "sliding_attention" else DequantKVCache(group_size=group_size, bits=bits,
                                                                  quantized_decode=quantized_decode,
                                                                  fused_decode=fused_decode,
                                                                  fused_prefill=fused_prefill)
        for lt in a.layer_types
    ]
