"""lagunalab_amd: MI355X (gfx950) implementation of lagunaLab's quantized KV-cache decode path.

Python surface (drop-in names of ``laguna_mlx``):
  cache.DequantKVCache, cache.make_quantized_cache, cache.QuantizedKVCache
  q8_attn.q8_decode_attention (+ decode_attention for ragged / 4-bit / bf16, q8_verify_attention)
  lookup.NgramIndex, lookup.ngram_propose, lookup.greedy_accept, lookup.DeviceNgramIndex
  quant.quantize / quant.dequantize / quant.quantize_into
All compute runs in liblaguna_hip.so (hand-written HIP for gfx950); there is no CPU fallback.
"""
__version__ = "0.1.0"
