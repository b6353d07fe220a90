"""CPU oracle for the q8 KV-cache decode path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy on the CPU, what the reference computes on the hot path:

* ``quantize``  -- MLX 0.32.0 affine ``mx.quantize`` / ``mx.dequantize`` as called by
  ``laguna_mlx/cache.py:90,100`` (through mlx-lm's ``QuantizedKVCache``), 8- and 4-bit, and the
  uint32 packing the reference kernel reads (``laguna_mlx/q8_attn.py:8-10``).
* ``attention`` -- the unfused path that is the reference's correctness oracle
  (``cache.py:99-100`` dequantize to bf16, then SDPA at ``laguna_mlx/laguna.py:107``), the
  bottom-right causal mask for multi-token steps, and a restatement of the fused kernel's
  per-block partials and block merge (``q8_attn.py:44-91,126-130``).
* ``lookup``    -- prompt-lookup drafting (``laguna_mlx/dflash.py:145-167``, brute force of
  ``tests/test_dflash.py:90-98``) and greedy acceptance (``dflash.py:195-198``).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg may import
this package, and only as the checker or the timed CPU baseline. The product package
``lagunalab_amd`` never imports it and has no CPU fallback.

Parity status of each function is stated in its module docstring.
"""
