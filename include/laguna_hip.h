/*
 * laguna_hip.h -- C ABI of liblaguna_hip.so: MI355X (gfx950) kernels for lagunaLab's quantized
 * KV-cache decode path.
 *
 * Conventions
 *  - Every entry point returns an int status (LQ_OK == 0) and never throws. On failure
 *    lq_last_error() returns a thread-local message. Arguments are validated before any launch.
 *  - Pointers are device pointers unless the comment says "host". The library allocates no
 *    memory; scratch space is passed in as `workspace` (size from the matching *_bytes query).
 *  - Work is enqueued on `stream` (a hipStream_t, passed as void*) and is asynchronous.
 *  - bf16 values are passed as uint16_t bit patterns.
 *
 * Cache layout (the reference's, laguna_mlx/q8_attn.py:8-10; mlx-lm QuantizedKVCache): per layer
 *   codes  uint8  [B, Hkv, cap, D*bits/8]  8-bit: one byte per element in order (byte-identical to
 *                                          MLX's uint32 words, low byte first); 4-bit: two per
 *                                          byte, even element in the low nibble
 *   scales bf16   [B, Hkv, cap, D/group]
 *   biases bf16   [B, Hkv, cap, D/group]
 * Rows [0, n) of the full-capacity buffers are valid.
 */
#ifndef LAGUNA_HIP_H
#define LAGUNA_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LQ_OK 0
#define LQ_EINVAL 1     /* bad argument (shape, size, dtype contract) */
#define LQ_EHIP 2       /* HIP runtime error (launch, attribute query) */
#define LQ_EWORKSPACE 3 /* workspace missing or too small */

#define LQ_MAX_SEQS 64  /* sequences per ragged decode call */

/*
 * Attention workspaces (lq_decode_attn, lq_q8_verify_attn) start with LQ_WS_ZERO_BYTES bytes of
 * counters (per sequence and KV head: an arrival count and a work-distribution count) that must
 * be zero before the first call that uses the workspace (clear them once after allocating it);
 * every call leaves them zero again. Calls that share a workspace must be ordered (one stream).
 * At most 2048 (sequence, KV head) pairs per call.
 */
#define LQ_WS_ZERO_BYTES 131072

/* Library version (major*10000 + minor*100 + patch). */
int lq_version(void);

/* Message for the last failing call on this thread ("" if none). */
const char* lq_last_error(void);

/*
 * Quantize-on-append. Replaces mx.quantize inside mlx-lm QuantizedKVCache.update_and_fetch as
 * called from DequantKVCache.update_and_fetch (laguna_mlx/cache.py:89-90): quantizes
 * src[B, H, L, D] (bf16, contiguous) group-wise and writes rows [offset, offset+L) of the cache
 * buffers (capacity `cap` rows). bits in {4, 8}; group_size in {32, 64, 128}; D % group_size == 0.
 */
int lq_quantize_append(const uint16_t* src, int64_t B, int64_t H, int64_t L, int64_t D,
                       uint8_t* codes, uint16_t* scales, uint16_t* biases, int64_t cap,
                       int64_t offset, int bits, int group_size, void* stream);

/*
 * Quantize-on-append of the keys and the values of one update in a single launch: the same as
 * lq_quantize_append on (k_src -> k_*) and on (v_src -> v_*). Replaces the paired mx.quantize of K
 * and V in QuantizedKVCache.update_and_fetch (laguna_mlx/cache.py:90).
 */
int lq_quantize_append_kv(const uint16_t* k_src, const uint16_t* v_src, int64_t B, int64_t H,
                          int64_t L, int64_t D, uint8_t* k_codes, uint16_t* k_scales,
                          uint16_t* k_biases, uint8_t* v_codes, uint16_t* v_scales,
                          uint16_t* v_biases, int64_t cap, int64_t offset, int bits,
                          int group_size, void* stream);

/*
 * Dequantize rows [0, n) of a cache to bf16 out[B, H, n, D]. Replaces mx.dequantize on the
 * unfused path (laguna_mlx/cache.py:99-100).
 */
int lq_dequantize(const uint8_t* codes, const uint16_t* scales, const uint16_t* biases,
                  int64_t B, int64_t H, int64_t cap, int64_t n, int64_t D, int bits,
                  int group_size, uint16_t* out, void* stream);

/*
 * Scratch bytes for lq_decode_attn with the same B / Hq / Hkv / lengths. `lens_host` (host, B
 * entries) may be NULL, then every sequence has length n. Returns a negative value on bad args.
 * The size never falls as a length grows (same kind, B, Hq, Hkv): a workspace sized for a
 * session's longest lengths serves every shorter call of the same shape.
 */
int64_t lq_decode_workspace_bytes(int kind, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                  int64_t n, const int32_t* lens_host);

/* kind for lq_decode_attn / lq_decode_workspace_bytes */
#define LQ_KV_Q8 8    /* 8-bit affine group-64 codes */
#define LQ_KV_Q4 4    /* 4-bit affine group-64 codes */
#define LQ_KV_BF16 16 /* plain bf16 K/V [B, Hkv, cap, D]; scale/bias pointers unused */

/*
 * Fused single-token decode attention. Replaces q8_decode_attention(q, keys, values, n, scale)
 * (laguna_mlx/q8_attn.py:102-130: the Metal kernel N1 at :17-99 and the block merge at
 * :126-130) and generalises it to 4-bit and plain-bf16 caches and to ragged batches.
 *   q    bf16 [B, Hq, 1, D] contiguous, D == 128, Hq % Hkv == 0, Hq / Hkv <= 16 (<= 4 for
 *        LQ_KV_Q4 and LQ_KV_BF16)
 *   kc..vb the cache buffers of one layer (layout above; for LQ_KV_BF16, kc and vc are bf16
 *          [B, Hkv, cap, D])
 *   n    valid rows when lens_host == NULL; otherwise lens_host[b] (host array, B <= 64,
 *        1 <= lens <= cap) gives each sequence's length (variable-length split-K with a
 *        per-sequence log-sum-exp merge)
 *   out  bf16 [B, Hq, 1, D]
 * softmax scale `scale` (the reference passes head_dim**-0.5, laguna_mlx/laguna.py:76).
 */
int lq_decode_attn(int kind, const uint16_t* q, const void* kc, const uint16_t* ks,
                   const uint16_t* kb, const void* vc, const uint16_t* vs, const uint16_t* vb,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t cap, int64_t n,
                   const int32_t* lens_host, float scale, uint16_t* out, void* workspace,
                   int64_t workspace_bytes, void* stream);

/*
 * One fused single-token decode step on the 8-bit cache: appends the new key and value row of
 * every sequence (bf16 k_new, v_new [B, Hkv, 1, D], quantized exactly as lq_quantize_append_kv)
 * at row n (or lens_host[b]) and attends over the n + 1 (lens_host[b] + 1) rows, as
 * DequantKVCache.update_and_fetch followed by attend on a fused step (laguna_mlx/cache.py:89-92,
 * 102-106; laguna_mlx/laguna.py:103-105) -- in one kernel launch when Hq / Hkv <= 4. n and
 * lens_host count the rows BEFORE the append and must leave one free row (< cap). Workspace:
 * lq_decode_workspace_bytes(LQ_KV_Q8, ...) for the lengths after the append.
 */
int lq_q8_decode_append_attn(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint8_t* kc, uint16_t* ks, uint16_t* kb, uint8_t* vc, uint16_t* vs,
                             uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                             int64_t cap, int64_t n, const int32_t* lens_host, float scale,
                             uint16_t* out, void* workspace, int64_t workspace_bytes,
                             void* stream);

/*
 * Scratch bytes for lq_q8_verify_attn; like lq_decode_workspace_bytes, never falling as n grows.
 */
int64_t lq_verify_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                                  int64_t n);

/*
 * Fused multi-query causal verify attention over the 8-bit cache. Replaces the unfused verify
 * forward of the speculative loop (laguna_mlx/dflash.py:195 -> laguna.py:107 with the causal
 * mask of laguna.py:183-186, over DequantKVCache's dequantized K/V, cache.py:99-100):
 *   q   bf16 [B, Hq, L, D] contiguous, 1 <= L <= 16, D == 128; the last L of the n valid rows are
 *       the block's own keys; query row i sees keys 0 .. n-L+i (bottom-right causal).
 *   out bf16 [B, Hq, L, D]
 */
int lq_q8_verify_attn(const uint16_t* q, const uint8_t* kc, const uint16_t* ks,
                      const uint16_t* kb, const uint8_t* vc, const uint16_t* vs,
                      const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                      int64_t D, int64_t cap, int64_t n, float scale, uint16_t* out,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * One fused verify step on the 8-bit cache: appends the block's L new key and value rows of
 * every sequence (bf16 k_new, v_new [B, Hkv, L, D], quantized exactly as lq_quantize_append_kv)
 * at rows n .. n+L-1 and runs lq_q8_verify_attn over the n + L rows, as
 * DequantKVCache.update_and_fetch followed by the verify forward's attention
 * (laguna_mlx/cache.py:89-100; laguna_mlx/dflash.py:195 -> laguna.py:107) -- the append inside
 * the attention kernel when G * L > 4. n counts the rows BEFORE the append; n + L <= cap.
 * Workspace: lq_verify_workspace_bytes for n + L rows.
 */
int lq_q8_verify_append_attn(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                             uint8_t* kc, uint16_t* ks, uint16_t* kb, uint8_t* vc, uint16_t* vs,
                             uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                             int64_t D, int64_t cap, int64_t n, float scale, uint16_t* out,
                             void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Prompt-lookup draft search. Replaces NgramIndex.propose (laguna_mlx/dflash.py:164-167) for a
 * history held on the device: finds the most recent start s <= T-g-1 with
 * hist[s:s+g] == hist[T-g:T] and returns up to n following ids (never past T).
 *   hist int32 [T] (device)
 *   out  int32 [2 + n] (device): out[0] = count, out[1] = s (-1 if none), out[2..2+count) ids
 * 1 <= g <= 16, 1 <= n <= 64.
 */
int64_t lq_ngram_workspace_bytes(int64_t T);
int lq_ngram_propose(const int32_t* hist, int64_t T, int g, int n, int32_t* out,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Greedy acceptance of a verified draft block. Replaces the argmax + longest-prefix loop of
 * generate_lookup (laguna_mlx/dflash.py:195-198):
 *   logits fp32 [L, V] (row stride V), drafts int32 [m] (device), m <= L - 1
 *   out int32 [2 + L] (device): out[0] = k (accepted drafts), out[1] = next token pred[k],
 *       out[2 + i] = argmax of row i (first index on ties)
 */
int64_t lq_accept_workspace_bytes(int64_t L, int64_t V);
int lq_greedy_accept(const float* logits, int64_t L, int64_t V, const int32_t* drafts,
                     int64_t m, int32_t* out, void* workspace, int64_t workspace_bytes,
                     void* stream);

/*
 * The fused decode step of a full-attention layer from raw projections: q (bf16 [B, Hq, 1, D]) and
 * k_new are the rows before the layer's q_norm / k_norm and RoPE (laguna_mlx/laguna.py:97-101),
 * which the attention kernel applies itself (norm weights bf16 [128], norm_eps; RoPE at the append
 * row, inv_freq fp32 [rot_dims / 2], rot_dims a multiple of 4 up to 128, rotated dims scaled by
 * mscale; the same arithmetic as lq_qk_norm_rope) before the fused append and attention of
 * lq_q8_decode_append_attn. pos: as lq_q8_decode_append_attn_pos (device append rows), or null:
 * every sequence appends at row n_plan. Workspace sized for n_plan + 1 rows. With more than 4 query
 * heads per KV head the norm and RoPE run as a launch of their own before the attention kernel
 * (their output rows live in the workspace).
 */
int lq_q8_decode_norm_append_attn(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                  uint8_t* kc, uint16_t* ks, uint16_t* kb, uint8_t* vc,
                                  uint16_t* vs, uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv,
                                  int64_t D, int64_t cap, int64_t n_plan, const int32_t* pos,
                                  const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                                  float norm_eps, const float* inv_freq, int64_t rot_dims,
                                  float mscale, float scale, uint16_t* out, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * lq_q8_decode_append_attn with the append rows read on the device: pos int32 [B] (device) is the
 * row each sequence appends at (its rows before the append), so that one recorded launch -- a HIP
 * graph of a decode step -- serves every step; the split plan and the workspace are those of
 * n_plan rows per sequence (size the workspace with lq_decode_workspace_bytes for n_plan + 1).
 * Each sequence attends over min(pos[b] + 1, cap) rows; keep pos[b] < cap.
 */
int lq_q8_decode_append_attn_pos(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new,
                                 uint8_t* kc, uint16_t* ks, uint16_t* kb, uint8_t* vc,
                                 uint16_t* vs, uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv,
                                 int64_t D, int64_t cap, int64_t n_plan, const int32_t* pos,
                                 float scale, uint16_t* out, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/*
 * q/k RMSNorm + RoPE of the attention block (laguna_mlx/laguna.py:97-101: q_norm / k_norm over
 * head_dim, then rope at the cache offset; mlx-lm initialize_rope frequencies, passed in):
 *   q bf16 [B, Hq, L, 128], k bf16 [B, Hkv, L, 128] -> q_out, k_out (same shapes; may alias)
 *   q_norm_w, k_norm_w bf16 [128]; inv_freq fp32 [rot_dims / 2] (device): dim i < rot_dims / 2
 *   pairs with i + rot_dims / 2 at angle (offset + l) * inv_freq[i] (offsets int32 [B], device,
 *   per sequence when not null); mscale scales the rotated dims (YaRN); dims >= rot_dims pass.
 * rot_dims a multiple of 4 in [0, 128].
 */
int lq_qk_norm_rope(const uint16_t* q, const uint16_t* k, uint16_t* q_out, uint16_t* k_out,
                    const uint16_t* q_norm_w, const uint16_t* k_norm_w, int64_t B, int64_t Hq,
                    int64_t Hkv, int64_t L, int64_t D, float eps, const float* inv_freq,
                    int64_t rot_dims, float mscale, int64_t offset, const int32_t* offsets,
                    void* stream);

/*
 * Output gate of the attention block (laguna_mlx/laguna.py:108-110):
 *   out[b, l, h, :] = attn[b, h, l, :] * softplus(gate)   (bf16, o_proj's [B, L, Hq, 128] layout)
 *   gate bf16 [B, L, Hq] (per-head gating) or [B, L, Hq, 128] (per_dim != 0)
 */
int lq_gate_heads(const uint16_t* attn, const uint16_t* gate, uint16_t* out, int64_t B,
                  int64_t Hq, int64_t L, int64_t D, int per_dim, void* stream);

/*
 * Residual add + RMSNorm of a decoder layer's input (laguna.py's input_layernorm after the
 * previous block's residual add): h_out = h + d (bf16; d may be null: no add, h_out unused),
 * y = RMSNorm(h_out) * w (bf16), rows of C values, C a multiple of 8 up to 8192. h_out may alias h.
 */
int lq_add_rms_norm(const uint16_t* h, const uint16_t* d, const uint16_t* w, uint16_t* h_out,
                    uint16_t* y, int64_t rows, int64_t C, float eps, void* stream);

/*
 * y = W x for one input row (the projections of a decode step, laguna.py:97-99,110 at L = 1):
 * W bf16 [N, K] row-major, x bf16 [K], y bf16 [N]; fp32 accumulation; K a multiple of 8.
 */
int lq_gemv_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, int64_t N, int64_t K,
                 void* stream);

/*
 * The projections of a decode step with their neighbours fused in (one input row, W bf16 [N, K],
 * K a multiple of 8 up to 4096):
 *   mode 1 (input projection): y = W (RMSNorm(x) * aux), x the residual stream [K], aux the
 *          layer's input-norm weights [K] (the norm's output rounded to bf16 as in the reference);
 *   mode 2 (output projection): y = W (x * softplus(aux)), x the attention output [K = H * 128],
 *          aux the gate logits [H] (per head) or [K] (per_dim != 0), gate and product in bf16;
 *   res (may be null or equal y): y[n] = res[n] + (W . x)[n] in bf16, the residual add.
 */
int lq_gemv_fused(const uint16_t* W, const uint16_t* x, const uint16_t* aux, const uint16_t* res,
                  uint16_t* y, int64_t N, int64_t K, int mode, float eps, int per_dim,
                  void* stream);

/*
 * Causal attention of a prefill chunk over the 8-bit cache, without the score matrix or a
 * dequantized copy of the cache (replaces, for prefill chunks, DequantKVCache's dequantize,
 * laguna_mlx/cache.py:99-100, and the SDPA of laguna.py:107 with the causal mask; the reference
 * guards the peak memory of that path in tests/test_cache.py:79-93):
 *   q   bf16 [B, Hq, L, D] contiguous, D == 128, Hq / Hkv in {1, 2, 4, 8}; the chunk's positions
 *       are n-L .. n-1, their K/V already the last L of the first n cache rows; row i sees keys
 *       0 .. n-L+i.
 *   out bf16 [B, Hq, L, D]
 * No workspace.
 */
int lq_q8_prefill_attn(const uint16_t* q, const uint8_t* kc, const uint16_t* ks, const uint16_t* kb,
                       const uint8_t* vc, const uint16_t* vs, const uint16_t* vb, int64_t B,
                       int64_t Hq, int64_t Hkv, int64_t L, int64_t D, int64_t cap, int64_t n,
                       float scale, uint16_t* out, void* stream);

/*
 * The input half of a decode step's attention block in one launch (one input row; laguna.py's
 * input_layernorm, then laguna.py:97-101 at L = 1): y = W (RMSNorm(x) * norm_w) as lq_gemv_fused
 * mode 1, then the first (Hq + Hkv) x 128 outputs, the q heads followed by the k heads, each get
 * their RMSNorm (q_norm_w / k_norm_w, head_eps) and RoPE at position `offset` (or *offsets when
 * offsets is non-null, a device int32) as lq_qk_norm_rope computes them, in place. N >= 128 (Hq +
 * Hkv); the remaining outputs (v, gate logits) are plain projections. counters: Hq + Hkv uint32 in
 * device memory, zero before the first call; every call leaves them zero. Calls that share
 * counters must not overlap.
 */
int lq_gemv_norm_rope(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w, uint16_t* y,
                      int64_t N, int64_t K, float eps, const uint16_t* q_norm_w,
                      const uint16_t* k_norm_w, int64_t Hq, int64_t Hkv, float head_eps,
                      const float* inv_freq, int64_t rot_dims, float mscale, int64_t offset,
                      const int32_t* offsets, uint32_t* counters, void* stream);

/*
 * No counterpart in the reference: lq_q8_decode_append_attn without a caller workspace, for
 * callers that cannot allocate device memory (code under HIP graph capture, serving loops that
 * forbid allocation). Same arguments, results and errors otherwise. The workspace is a static
 * 4 MiB device array, one per GPU the library runs on, held until the process ends; a call that
 * would need more (lq_decode_workspace_bytes of its shape) returns LQ_EWORKSPACE before any launch
 * (32q/8kv at any length needs about 0.66 MiB). The first call on a device queues a clear of the
 * array's counters on its stream (it may be made during a graph capture); every call leaves them
 * clear. All calls on one GPU share the array and the first call binds it to its stream: a later
 * call on another stream returns LQ_EINVAL before any launch. Replays of a captured graph that
 * overlap each other or an eager call on another stream still race (the library cannot see them).
 */
int lq_q8_decode_append_attn_noalloc(const uint16_t* q, const uint16_t* k_new,
                                     const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
                                     uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t cap,
                                     int64_t n, const int32_t* lens_host, float scale,
                                     uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LAGUNA_HIP_H */
