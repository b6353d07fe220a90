// Shared declarations of the split-K attention kernels: the per-call split plan and the entry
// points of the MFMA kernels (qattn.hip) used by the decode and verify C ABI (decode.hip,
// verify.hip).
#pragma once

#include "common.h"

namespace lq {

constexpr int D = 128;  // head_dim of the fused kernels

// Variable-length split plan, passed by value as a kernel argument. Sequence b owns the global
// splits [split_begin[b], split_begin[b+1]); split s of it covers keys
// [s * chunk, min((s + 1) * chunk, len[b])).
struct DecodePlan {
  int32_t nseq;
  int32_t chunk;
  int32_t split_begin[LQ_MAX_SEQS + 1];
  int32_t len[LQ_MAX_SEQS];
};

__device__ __forceinline__ void find_seq(const DecodePlan& plan, int x, int& b) {
  b = 0;
  for (int i = 1; i < plan.nseq; ++i)
    if (x >= plan.split_begin[i]) b = i;
}

// The sequence of global split x: its index, first split, split count and length (rows). A
// single sequence (decode or verify of one stream) takes them from fixed argument offsets, in
// one batch of argument loads with nseq; a batch searches the plan, whose index-dependent
// argument loads are a second round trip before the kernel's first copy.
struct SeqSplits {
  int b, s0, ns, len;
};
// Kernel arguments the prologue needs before its first copy, listed as SGPR inputs of one empty
// asm statement right after they are read: the compiler then issues all their loads in one batch
// (left alone, it issued some only behind the first branch on the others -- a second argument
// round trip of ~0.3 us before any copy could start).
#define LQ_ARG_BATCH(...) asm volatile("" ::__VA_ARGS__)
__device__ __forceinline__ SeqSplits seq_splits(const DecodePlan& plan, int x) {
  SeqSplits s{0, 0, plan.split_begin[1], plan.len[0]};  // split_begin[0] is 0
  if (plan.nseq > 1) {
    find_seq(plan, x, s.b);
    s.s0 = plan.split_begin[s.b];
    s.ns = plan.split_begin[s.b + 1] - s.s0;
    s.len = plan.len[s.b];
  }
  return s;
}

// Arguments of the attention kernels (kernel argument block, passed by value).
struct AttnArgs {
  const uint16_t* q;  // bf16 [B, Hkv * G, L, D]
  uint8_t* kc;        // cache buffers of one layer (written only for the fused append)
  uint16_t* ks;
  uint16_t* kb;
  uint8_t* vc;
  uint16_t* vs;
  uint16_t* vb;
  // Fused append (packed kernel only; null otherwise): bf16 rows [B, Hkv, 1, D] that become row
  // len - 1 of each sequence; the kernel quantizes them, attends over them and stores them.
  const uint16_t* knew;
  const uint16_t* vnew;
  // Device positions (packed kernel with the fused append only; null otherwise): int32 [B], the
  // row sequence b appends at; its length is then pos[b] + 1 (clamped to [1, cap]) instead of
  // the plan's len[b], so that a launch recorded in a HIP graph serves every decode step.
  const int32_t* pos;
  float* part_acc;    // workspace: split partials
  float2* part_ml;
  uint32_t* counters; // workspace: arrival and tile counters (zero between calls)
  uint16_t* out;      // bf16 [B, Hkv * G, L, D]
  int64_t cap;
  int Hkv, G, L;
  float qk_scale_log2;  // softmax scale * log2(e)
};

typedef void (*QAttnFn)(AttnArgs, DecodePlan);

// Workspace of the attention calls: per sequence and KV head i one 64-byte line of counters
// (atomics on one line serialize at ~10 ns each, so every pair gets its own): the workgroups'
// arrival count (uint32 at CTR_STRIDE i) and the packed kernels' tile count (at CTR_STRIDE i +
// 4), both zero between calls (each call's last arrival resets them), then the split partials.
// The counter area has a fixed size so that calls of any shape can share a workspace.
constexpr int64_t WS_COUNTER_BYTES = LQ_WS_ZERO_BYTES;
constexpr int64_t MAX_COUNTERS = 2048;
constexpr int CTR_STRIDE = 64;
static_assert(CTR_STRIDE * MAX_COUNTERS <= WS_COUNTER_BYTES, "counter area too small");
__host__ __device__ inline uint32_t* arrival_counter(uint32_t* counters, int i) {
  return reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(counters) + CTR_STRIDE * i);
}

// Packed 8-bit kernel (qattn.hip) for G * L <= 4 query rows per KV head, causal for multi-row
// verify blocks; it also merges the splits (no decode_merge_kernel launch).
QAttnFn q8_attn_fn(bool causal);
// q/k RMSNorm + RoPE inside the packed kernel (fused append with L = 1): the staged q rows and
// new K row are raw projections, normalized (weights qn_w / kn_w, bf16 [128], epsilon norm_eps)
// and rotated at position len - 1 (inv_freq fp32 [rot_dims / 2], rotated dims scaled by mscale)
// before use. A separate argument of that variant only, so that the other kernels' argument
// blocks stay as they are.
struct NormArgs {
  const uint16_t* qn_w;
  const uint16_t* kn_w;
  const float* inv_freq;
  int rot_dims;
  float mscale, norm_eps;
};
// Launches the decode variant (no causal mask) with the in-kernel q/k norm on an S x Hkv grid.
void launch_q8_attn_norm(unsigned S, unsigned Hkv, hipStream_t st, const AttnArgs& a,
                         const DecodePlan& plan, const NormArgs& nargs);
// Dense-layout kernel (attn_dense.hip) for 4 < G * L <= 16 nt rows per KV head, and for up to 4
// over one sequence of at most 65,536 rows; partials merged by decode_merge_kernel, or (merge:
// decode with at most 8 rows per KV head, nt = 1) by the kernel's last workgroup per KV head.
QAttnFn q8_dense_attn_fn(int nt, bool causal, bool merge);
// Its workgroup size for nt column tiles.
int q8_dense_threads(int nt);

// The attention kernel for one call: its function and workgroup size.
struct AttnKernel {
  QAttnFn fn;
  int threads;
  bool merges;  // the kernel merges the split partials itself (else decode_merge_kernel does)
  bool packed;  // a packed kernel (8-bit, 4-bit, bf16): at most 4 rows per KV head, one or more
                // workgroups per CU; else the dense kernel (one workgroup per CU)
};

// Plain-bf16 cache kernel (attn_bf16.hip), G * L <= 4.
QAttnFn bf16_attn_fn(bool causal);
// 4-bit cache kernel (attn_q4.hip), G * L <= 4.
QAttnFn q4_attn_fn(bool causal);

// Plan + workspace bytes for an attention call of `kind` (LQ_KV_*) with L query rows per head;
// returns the number of splits (or -1: bad lengths or an unsupported configuration) and selects
// the kernel.
int64_t attn_plan(int kind, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t n,
                  const int32_t* lens, int64_t cap, DecodePlan& plan, AttnKernel& k,
                  int64_t& ws_bytes);

// Workspace bytes reported to callers for such a call (-1 as attn_plan): the call's own need,
// except that for one sequence of more than 65,536 rows with G * L <= 4 (packed kernel) it also
// covers the dense kernel's need at 65,536 rows, the longest length that kernel serves. The
// reported size then never falls as the length grows, so one workspace sized for a session's
// longest length serves every shorter call of the same shape.
int64_t attn_workspace_bytes(int kind, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t n,
                             const int32_t* lens);


// Per-sequence log-sum-exp merge of split partials: rows_per_seq = Hq * L partial rows per split.
void launch_merge(const float* part_acc, const float2* part_ml, int rows_per_seq,
                  const DecodePlan& plan, int64_t B, uint16_t* out, hipStream_t st);

}  // namespace lq
