// Single-token decode attention over the quantized KV cache: split plan, launch and the
// log-sum-exp merge of the split partials.
//
// Replaces q8_decode_attention (laguna_mlx/q8_attn.py:102-130): the Metal kernel that reads the
// packed cache once, dequantizes in registers and keeps an online softmax per block of keys
// (:17-99), and the log-sum-exp merge of the block partials (:126-130). The attention kernels
// themselves (MFMA, global-to-LDS pipeline) are in qattn.hip; this file owns
//  * the split plan: grid (split, kv head); the workgroups of one sequence and KV head share its
//    keys (8-bit kernels: super-tiles in turn; 4-bit and bf16: contiguous chunks) and serve all G
//    query heads of that KV head, so every K/V byte is read from HBM exactly once; the grid is
//    one wave of resident workgroups over all CUs, for uniform and ragged batches alike (make_plan);
//  * the merge: partials (m, l, acc[128]) per (split, query row) are combined per sequence.
#include <mutex>

#include "common.h"
#include "qattn.h"

namespace lq {
namespace {

constexpr int MIN_CHUNK = 256;  // keys per split at least (4,096 keys: 16 splits per head)
constexpr int64_t MAX_SPLITS = 32;    // kernels that merge their own splits (merge_rows4)
constexpr int64_t MERGE_SPLITS = 64;  // kernels whose splits decode_merge_kernel merges

// ----------------------------------------------------------------------------------------------
// merge kernel: 64 dims of one partial row per workgroup (one wave); each group of four dims is
// merged by four lanes 16 apart, each over a quarter of the splits
// ----------------------------------------------------------------------------------------------

// rows = partial rows per sequence (Hq * L). A sequence has at most MS <= MERGE_SPLITS splits
// (make_plan). Lane l takes dims d0 = 64 (workgroup % 2) + 4 (l % 16) .. d0 + 3 of the splits
// l / 16 + 4 k, k < MS / 4: it loads their (m, l) and the 16 bytes of acc in one round trip, the
// four lanes of a dim group find the largest m with two lane swaps, weigh their splits against it
// (log-sum-exp) and add up their sums with two more swaps. Four lanes per dim group put the same
// partials in flight with a quarter of the loads per lane and four times the waves.
template <int MS>
__global__ __launch_bounds__(64) void decode_merge_kernel(const float* __restrict__ part_acc,
                                                           const float2* __restrict__ part_ml,
                                                           int rows, int total_rows,
                                                           DecodePlan plan,
                                                           uint16_t* __restrict__ out) {
  constexpr int PER = MS / 4;
  // one batch of argument loads: a single sequence's split range sits at fixed offsets (an
  // index-dependent load would be a second argument round trip before the first partial load)
  LQ_ARG_BATCH("s"(part_acc), "s"(part_ml), "s"(rows), "s"(total_rows), "s"(plan.nseq),
               "s"(plan.split_begin[1]));
  const int grow = blockIdx.x >> 1;  // (sequence, row) index
  if (grow >= total_rows) return;    // workgroup-uniform
  const int lane = threadIdx.x;
  const int qt = lane >> 4;
  const int d0 = 64 * (blockIdx.x & 1) + 4 * (lane & 15);
  const int b = grow / rows;
  const int hq = grow - b * rows;
  int s0 = 0, ns = min(plan.split_begin[1], MS);
  if (plan.nseq > 1) {
    s0 = plan.split_begin[b];
    ns = min(plan.split_begin[b + 1] - s0, MS);
  }
  float m[PER], l[PER];
  float4 a[PER];
  // The (m, l) index is the same in 16 lanes; hidden from the compiler so that the loads stay
  // vector loads issued together (as scalar loads it waited for each one in turn).
  int base = s0;
  asm volatile("" : "+v"(base));
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const int64_t r = (int64_t)(base + min(qt + 4 * k, ns - 1)) * rows + hq;
    const float2 ml = part_ml[r];  // past ns: split ns - 1 again, weighted 0 below
    m[k] = ml.x;
    l[k] = ml.y;
    a[k] = *reinterpret_cast<const float4*>(part_acc + r * D + d0);
  }
  float M = -INFINITY;
#pragma unroll
  for (int k = 0; k < PER; ++k) M = max_ieee(M, qt + 4 * k < ns ? m[k] : -INFINITY);
  M = max_xor32(max_xor16(M));
  float n0 = 0.0f, n1 = 0.0f, n2 = 0.0f, n3 = 0.0f, den = 0.0f;
#pragma unroll
  for (int k = 0; k < PER; ++k) {
    const bool use = qt + 4 * k < ns && m[k] != -INFINITY;
    const float w = use ? __builtin_amdgcn_exp2f(m[k] - M) : 0.0f;  // argument <= 0
    n0 = fmaf(w, a[k].x, n0);
    n1 = fmaf(w, a[k].y, n1);
    n2 = fmaf(w, a[k].z, n2);
    n3 = fmaf(w, a[k].w, n3);
    den = fmaf(w, l[k], den);
  }
  n0 = sum_xor32(sum_xor16(n0));
  n1 = sum_xor32(sum_xor16(n1));
  n2 = sum_xor32(sum_xor16(n2));
  n3 = sum_xor32(sum_xor16(n3));
  den = sum_xor32(sum_xor16(den));
  if (qt == 0) {
    const float inv = 1.0f / den;
    const uint32_t lo = (uint32_t)f32_to_bf16(n0 * inv) | ((uint32_t)f32_to_bf16(n1 * inv) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(n2 * inv) | ((uint32_t)f32_to_bf16(n3 * inv) << 16);
    *reinterpret_cast<uint2*>(out + (int64_t)grow * D + d0) = make_uint2(lo, hi);
  }
}

// ----------------------------------------------------------------------------------------------
// host side
// ----------------------------------------------------------------------------------------------

// Builds the split plan. Returns total splits, or -1 on bad lengths.
//  * Chunked kernels (4-bit, bf16): split s of sequence b covers keys [s chunk, (s + 1) chunk),
//    one `chunk` for all sequences, sized so that the splits of all sequences fill about one wave
//    of resident workgroups.
//  * Interleaved kernels (8-bit): the waves of all of a sequence's splits take its super-tiles in
//    turn, so only the split count per sequence matters. Each KV head gets at most
//    wgs_target / Hkv splits (one wave of resident workgroups: nothing waits for a second wave),
//    apportioned min-max: every sequence starts with one split and each further split goes to
//    the sequence with the most keys per split, so that the slowest sequence (the one that ends
//    the launch) has as few keys per split as the budget allows.
int64_t make_plan(int64_t B, int64_t Hkv, int64_t n, const int32_t* lens, int64_t cap,
                  int wgs_target, bool interleaved, int64_t max_splits, DecodePlan& plan) {
  if (B < 1 || B > LQ_MAX_SEQS) return -1;
  int64_t total = 0, longest = 0;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t l = lens ? lens[b] : n;
    if (l < 1 || (cap > 0 && l > cap)) return -1;
    plan.len[b] = (int32_t)l;
    total += l;
    longest = std::max<int64_t>(longest, l);
  }
  const int64_t per_head = std::max<int64_t>(1, wgs_target / Hkv);
  plan.nseq = (int32_t)B;
  if (interleaved) {
    int64_t ns[LQ_MAX_SEQS];
    for (int64_t b = 0; b < B; ++b) ns[b] = 1;
    for (int64_t budget = per_head - B; budget > 0; --budget) {
      int64_t best = -1;  // most keys per split among sequences that may take another split
      for (int64_t b = 0; b < B; ++b) {
        const int64_t lim =
            std::min<int64_t>(max_splits, (plan.len[b] + MIN_CHUNK - 1) / MIN_CHUNK);
        if (ns[b] >= lim) continue;
        if (best < 0 || (int64_t)plan.len[b] * ns[best] > (int64_t)plan.len[best] * ns[b])
          best = b;
      }
      if (best < 0) break;
      ++ns[best];
    }
    int64_t s = 0, chunk = 0;
    for (int64_t b = 0; b < B; ++b) {
      plan.split_begin[b] = (int32_t)s;
      s += ns[b];
      chunk = std::max<int64_t>(chunk, (plan.len[b] + ns[b] - 1) / ns[b]);
    }
    plan.split_begin[B] = (int32_t)s;
    plan.chunk = (int32_t)chunk;  // largest keys per split (informational)
    return s;
  }
  int64_t chunk = (total + per_head - 1) / per_head;
  chunk = std::max<int64_t>(chunk, MIN_CHUNK);
  // at most max_splits splits per sequence: the in-kernel merge reads them in one round trip
  chunk = std::max<int64_t>(chunk, (longest + max_splits - 1) / max_splits);
  chunk = (chunk + 15) / 16 * 16;
  plan.chunk = (int32_t)chunk;
  int64_t s = 0;
  for (int64_t b = 0; b < B; ++b) {
    plan.split_begin[b] = (int32_t)s;
    s += (plan.len[b] + chunk - 1) / chunk;
  }
  plan.split_begin[B] = (int32_t)s;
  return s;
}

// Resident workgroups per CU for an attention kernel (cached per kernel; host threads may plan
// calls concurrently, so the cache is read and filled under a lock).
int attn_occupancy(QAttnFn fn, int threads) {
  static std::mutex mu;
  static QAttnFn fns[32];
  static int occ[32];
  static int nf = 0;
  std::lock_guard<std::mutex> lock(mu);
  for (int i = 0; i < nf; ++i)
    if (fns[i] == fn) return occ[i];
  int k = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, reinterpret_cast<const void*>(fn), threads,
                                                   0) != hipSuccess ||
      k < 1)
    k = 1;
  if (nf < 32) {
    fns[nf] = fn;
    occ[nf] = k;
    ++nf;
  }
  return k;
}

}  // namespace

void launch_merge(const float* part_acc, const float2* part_ml, int rows_per_seq,
                  const DecodePlan& plan, int64_t B, uint16_t* out, hipStream_t st) {
  int most = 1;
  for (int64_t b = 0; b < B; ++b)
    most = std::max(most, plan.split_begin[b + 1] - plan.split_begin[b]);
  const int total = (int)(B * rows_per_seq);
  // one wave per half row (64 dims)
  const dim3 grid((unsigned)(2 * total)), block(64);
  if (most <= 32)
    decode_merge_kernel<32><<<grid, block, 0, st>>>(part_acc, part_ml, rows_per_seq, total, plan, out);
  else
    decode_merge_kernel<MERGE_SPLITS><<<grid, block, 0, st>>>(part_acc, part_ml, rows_per_seq, total,
                                                              plan, out);
}

// 8-bit cache, at most 4 query rows per KV head: the packed kernel (in-kernel split merge) unless
// there is one sequence of at most DENSE_BELOW rows, where the dense kernel on 32-key
// super-tiles with 8 waves per workgroup and a merge launch is faster (µs per decode step,
// 32q/8kv: 1,024 keys 12.1 -> 11.6, 4,096 13.4 -> 12.2, 16,384 18.5 -> 16.3, 32,768 22.8 -> 20.9;
// at 82,671 both 37.5; a ragged batch of 8 long sequences 182.8 -> 193.5, so not there).
constexpr int64_t DENSE_BELOW = 65536;
bool q8_packed(int64_t R, int64_t B, int64_t longest) {
  return R <= 4 && !(B == 1 && longest <= DENSE_BELOW);
}

// Decode on the dense kernel with at most 8 rows per KV head merges its splits in the kernel (at
// most 32 splits x 8 rows of partials per KV head for the last workgroup to read) instead of a
// decode_merge_kernel launch.
bool dense_merges(int64_t R, int64_t L) { return L == 1 && R <= 8; }

// Decode with the dense kernel: where the q and new K rows after q/k norm + RoPE go in the
// workspace (behind the partials, 256-byte aligned).
int64_t norm_rows_offset(int64_t partials_end) { return (partials_end + 255) / 256 * 256; }

// Shared by decode (L = 1) and verify (L <= 16): kernel choice, plan and workspace size.
int64_t attn_plan(int kind, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t n,
                  const int32_t* lens, int64_t cap, DecodePlan& plan, AttnKernel& k,
                  int64_t& ws_bytes) {
  const int64_t R = (Hq / Hkv) * L;
  if (B < 1 || B > LQ_MAX_SEQS) return -1;
  int64_t longest = n;
  if (lens) {
    longest = 0;
    for (int64_t b = 0; b < B; ++b) longest = std::max<int64_t>(longest, lens[b]);
  }
  if (kind == LQ_KV_Q8) {
    const int nt = (int)((R + 15) / 16);
    if (q8_packed(R, B, longest)) {
      k = {q8_attn_fn(L > 1), 256, true, true};
    } else {
      const bool merge = dense_merges(R, L);
      k = {q8_dense_attn_fn(nt, L > 1, merge), q8_dense_threads(nt), merge, false};
    }
  } else if (kind == LQ_KV_BF16 && R <= 4) {
    k = {bf16_attn_fn(L > 1), 128, true, true};
  } else if (kind == LQ_KV_Q4 && R <= 4) {
    k = {q4_attn_fn(L > 1), 256, true, true};
  } else {
    return -1;
  }
  if (!k.fn) return -1;
  if (B * Hkv > MAX_COUNTERS) return -1;
  // One workgroup per CU for the dense kernel (its 8 or 4 waves hold about 150 KB of LDS).
  const int per_cu = k.packed ? attn_occupancy(k.fn, k.threads) : 1;
  const int64_t S = make_plan(B, Hkv, n, lens, cap, per_cu * device_cu_count(),
                              kind == LQ_KV_Q8, k.merges ? MAX_SPLITS : MERGE_SPLITS, plan);
  if (S < 0) return -1;
  ws_bytes = WS_COUNTER_BYTES + S * Hkv * R * (int64_t)(D * sizeof(float) + sizeof(float2));
  if (kind == LQ_KV_Q8 && L == 1 && !k.packed)  // normalized q / k rows (norm entry)
    ws_bytes = norm_rows_offset(ws_bytes) + B * (Hq + Hkv) * D * (int64_t)sizeof(uint16_t);
  return S;
}

int64_t attn_workspace_bytes(int kind, int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t n,
                             const int32_t* lens) {
  DecodePlan plan;
  AttnKernel k;
  int64_t ws = 0;
  if (attn_plan(kind, B, Hq, Hkv, L, n, lens, 0, plan, k, ws) < 0) return -1;
  const int64_t longest = lens ? lens[0] : n;
  const int64_t R = (Hq / Hkv) * L;
  if (kind != LQ_KV_Q8) {
    // Chunked plans (4-bit, bf16): the chunk is rounded up, so the split count can fall by one
    // as a length grows; report the plan's bound instead (its chunk covers the keys of all
    // sequences in at most per_head splits, plus one partial split per sequence, and at most
    // MAX_SPLITS per sequence).
    const int64_t per_head =
        std::max<int64_t>(1, attn_occupancy(k.fn, k.threads) * device_cu_count() / Hkv);
    const int64_t smax = std::min<int64_t>(per_head + B, MAX_SPLITS * B);
    ws = std::max(ws, WS_COUNTER_BYTES + smax * Hkv * R * (int64_t)(D * sizeof(float) + sizeof(float2)));
  } else if (B == 1 && longest > DENSE_BELOW && R <= 4) {
    int64_t dense = 0;
    if (attn_plan(kind, 1, Hq, Hkv, L, DENSE_BELOW, nullptr, 0, plan, k, dense) < 0) return -1;
    ws = std::max(ws, dense);
  }
  return ws;
}

}  // namespace lq

extern "C" int64_t lq_decode_workspace_bytes(int kind, int64_t B, int64_t Hq, int64_t Hkv,
                                             int64_t D, int64_t n, const int32_t* lens_host) {
  using namespace lq;
  clear_error();
  if (D != 128 || Hkv < 1 || Hq % Hkv || Hq / Hkv > 16) {
    set_error("unsupported decode configuration");
    return -1;
  }
  if (kind != LQ_KV_Q8 && !((kind == LQ_KV_BF16 || kind == LQ_KV_Q4) && Hq / Hkv <= 4)) {
    set_error("kv kind %d not supported for these shapes (4-bit and bf16: Hq / Hkv <= 4)", kind);
    return -1;
  }
  const int64_t ws = attn_workspace_bytes(kind, B, Hq, Hkv, 1, n, lens_host);
  if (ws < 0) set_error("bad sequence lengths");
  return ws;
}

namespace lq {
namespace {

// Decode attention over n (or lens[b]) rows; with k_new/v_new the last row of every sequence is
// first appended from them (n and lens count the rows after the append).
int decode_attn(int kind, const uint16_t* q, void* kc, uint16_t* ks, uint16_t* kb, void* vc,
                uint16_t* vs, uint16_t* vb, const uint16_t* k_new, const uint16_t* v_new,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t cap, int64_t n,
                const int32_t* lens, float scale, uint16_t* out, void* workspace,
                int64_t workspace_bytes, hipStream_t st, const int32_t* pos_dev = nullptr,
                const NormArgs* norm = nullptr) {
  LQ_CHECK_ARG(kind == LQ_KV_Q8 ||
                   ((kind == LQ_KV_BF16 || kind == LQ_KV_Q4) && Hkv >= 1 && Hq / Hkv <= 4 && !k_new),
               "kv kind %d not supported for these shapes (4-bit and bf16: Hq / Hkv <= 4)", kind);
  LQ_CHECK_ARG(D == 128, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "Hq=%lld must be a multiple of Hkv=%lld",
               (long long)Hq, (long long)Hkv);
  LQ_CHECK_ARG(Hq / Hkv <= 16, "at most 16 query heads per KV head (got %lld)",
               (long long)(Hq / Hkv));
  LQ_CHECK_ARG(B >= 1 && B <= LQ_MAX_SEQS, "batch %lld outside [1, %d]", (long long)B, LQ_MAX_SEQS);
  LQ_CHECK_ARG(cap >= 1 && cap <= (1 << 24), "capacity %lld outside [1, 2^24]", (long long)cap);
  LQ_CHECK_ARG(B * Hkv <= MAX_COUNTERS, "B * Hkv = %lld exceeds %lld", (long long)(B * Hkv),
               (long long)MAX_COUNTERS);
  LQ_CHECK_ARG(q && kc && vc && out && (kind == LQ_KV_BF16 || (ks && kb && vs && vb)),
               "null pointer");
  DecodePlan plan;
  AttnKernel kern;
  int64_t need = 0;
  const int64_t S = attn_plan(kind, B, Hq, Hkv, 1, n, lens, cap, plan, kern, need);
  LQ_CHECK_ARG(S > 0, "sequence lengths must be in [1, cap=%lld]", (long long)cap);
  if (!workspace || workspace_bytes < need) {
    set_error("workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
              (long long)need);
    return LQ_EWORKSPACE;
  }
  const bool fused_merge = kern.merges;
  const bool packed = kern.packed;
  LQ_CHECK_ARG(!pos_dev || (kind == LQ_KV_Q8 && k_new),
               "device positions need the fused 8-bit append");
  LQ_CHECK_ARG(!norm || (kind == LQ_KV_Q8 && k_new), "the q/k norm needs the fused 8-bit append");
  if (norm && !packed) {
    // Dense kernel (more than 4 query heads per KV head): q/k RMSNorm + RoPE as a launch of its
    // own (the same arithmetic as the packed kernel's prologue) into the workspace, at the append
    // row (device positions, or n - 1), then the fused step from those rows.
    const int64_t parts = WS_COUNTER_BYTES + S * Hq * (int64_t)(D * sizeof(float) + sizeof(float2));
    uint16_t* qn = reinterpret_cast<uint16_t*>(static_cast<char*>(workspace) +
                                               norm_rows_offset(parts));
    uint16_t* kn = qn + B * Hq * D;
    const int rs = lq_qk_norm_rope(q, k_new, qn, kn, norm->qn_w, norm->kn_w, B, Hq, Hkv, 1, D,
                                   norm->norm_eps, norm->inv_freq, norm->rot_dims, norm->mscale,
                                   n - 1, pos_dev, st);
    if (rs != LQ_OK) return rs;
    q = qn;
    k_new = kn;
    norm = nullptr;
  }
  AttnArgs a{};
  a.pos = pos_dev;
  a.q = q;
  a.kc = static_cast<uint8_t*>(kc);
  a.ks = ks;
  a.kb = kb;
  a.vc = static_cast<uint8_t*>(vc);
  a.vs = vs;
  a.vb = vb;
  if (k_new) {  // the packed and the dense kernels append the new row of every sequence themselves
    a.knew = k_new;
    a.vnew = v_new;
  }

  a.counters = reinterpret_cast<uint32_t*>(workspace);
  a.part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + WS_COUNTER_BYTES);
  a.part_ml = reinterpret_cast<float2*>(a.part_acc + S * Hq * D);
  a.out = out;
  a.cap = cap;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.L = 1;
  a.qk_scale_log2 = scale * 1.4426950408889634f;
  if (norm)
    launch_q8_attn_norm((unsigned)S, (unsigned)Hkv, st, a, plan, *norm);
  else
    hipLaunchKernelGGL(kern.fn, dim3((unsigned)S, (unsigned)Hkv), dim3((unsigned)kern.threads), 0,
                     st, a, plan);
  LQ_CHECK_LAUNCH("attention kernel");
  if (!fused_merge) {
    launch_merge(a.part_acc, a.part_ml, (int)Hq, plan, B, out, st);
    LQ_CHECK_LAUNCH("decode_merge_kernel");
  }
  return LQ_OK;
}

}  // namespace
}  // namespace lq

extern "C" int lq_decode_attn(int kind, const uint16_t* q, const void* kc, const uint16_t* ks,
                              const uint16_t* kb, const void* vc, const uint16_t* vs,
                              const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                              int64_t cap, int64_t n, const int32_t* lens_host, float scale,
                              uint16_t* out, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  using namespace lq;
  clear_error();
  return decode_attn(kind, q, const_cast<void*>(kc), const_cast<uint16_t*>(ks),
                     const_cast<uint16_t*>(kb), const_cast<void*>(vc), const_cast<uint16_t*>(vs),
                     const_cast<uint16_t*>(vb), nullptr, nullptr, B, Hq, Hkv, D, cap, n,
                     lens_host, scale, out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int lq_q8_decode_append_attn(const uint16_t* q, const uint16_t* k_new,
                                        const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
                                        uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb,
                                        int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                        int64_t cap, int64_t n, const int32_t* lens_host,
                                        float scale, uint16_t* out, void* workspace,
                                        int64_t workspace_bytes, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(k_new && v_new, "null pointer");
  LQ_CHECK_ARG(B >= 1 && B <= LQ_MAX_SEQS, "batch %lld outside [1, %d]", (long long)B, LQ_MAX_SEQS);
  // lengths after the append: one more row per sequence
  int32_t after[LQ_MAX_SEQS];
  if (lens_host) {
    for (int64_t b = 0; b < B; ++b) {
      LQ_CHECK_ARG(lens_host[b] >= 0 && lens_host[b] < cap,
                   "sequence %lld: %d rows leave no room to append in capacity %lld",
                   (long long)b, lens_host[b], (long long)cap);
      after[b] = lens_host[b] + 1;
    }
  } else {
    LQ_CHECK_ARG(n >= 0 && n < cap, "n=%lld leaves no room to append in capacity %lld",
                 (long long)n, (long long)cap);
  }
  return decode_attn(LQ_KV_Q8, q, kc, ks, kb, vc, vs, vb, k_new, v_new, B, Hq, Hkv, D, cap,
                     n + 1, lens_host ? after : nullptr, scale, out, workspace, workspace_bytes,
                     (hipStream_t)stream);
}

extern "C" int lq_q8_decode_norm_append_attn(
    const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
    uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv,
    int64_t D, int64_t cap, int64_t n_plan, const int32_t* pos, const uint16_t* q_norm_w,
    const uint16_t* k_norm_w, float norm_eps, const float* inv_freq, int64_t rot_dims,
    float mscale, float scale, uint16_t* out, void* workspace, int64_t workspace_bytes,
    void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(k_new && v_new && q_norm_w && k_norm_w && (inv_freq || rot_dims == 0),
               "null pointer");
  LQ_CHECK_ARG(rot_dims >= 0 && rot_dims <= 128 && rot_dims % 4 == 0,
               "rot_dims must be a multiple of 4 in [0, 128] (got %lld)", (long long)rot_dims);
  LQ_CHECK_ARG(n_plan >= 0 && n_plan < cap, "n_plan=%lld leaves no room to append in capacity %lld",
               (long long)n_plan, (long long)cap);
  NormArgs norm{};
  norm.qn_w = q_norm_w;
  norm.kn_w = k_norm_w;
  norm.inv_freq = inv_freq;
  norm.rot_dims = (int)rot_dims;
  norm.mscale = mscale;
  norm.norm_eps = norm_eps;
  return decode_attn(LQ_KV_Q8, q, kc, ks, kb, vc, vs, vb, k_new, v_new, B, Hq, Hkv, D, cap,
                     n_plan + 1, nullptr, scale, out, workspace, workspace_bytes,
                     (hipStream_t)stream, pos, &norm);
}

extern "C" int lq_q8_decode_append_attn_pos(const uint16_t* q, const uint16_t* k_new,
                                            const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
                                            uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb,
                                            int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                            int64_t cap, int64_t n_plan, const int32_t* pos,
                                            float scale, uint16_t* out, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(k_new && v_new && pos, "null pointer");
  LQ_CHECK_ARG(n_plan >= 0 && n_plan < cap, "n_plan=%lld leaves no room to append in capacity %lld",
               (long long)n_plan, (long long)cap);
  return decode_attn(LQ_KV_Q8, q, kc, ks, kb, vc, vs, vb, k_new, v_new, B, Hq, Hkv, D, cap,
                     n_plan + 1, nullptr, scale, out, workspace, workspace_bytes,
                     (hipStream_t)stream, pos);
}

// ----------------------------------------------------------------------------------------------
// The fused decode step without a caller workspace, for callers that cannot allocate (code under
// HIP graph capture, serving loops that forbid allocation). Its workspace -- the arrival and tile
// counters, then the split partials -- is a static device array, one per GPU the library runs on,
// held until the process ends.
// ----------------------------------------------------------------------------------------------

namespace lq {
namespace {

constexpr int64_t SCRATCH_BYTES = 4 << 20;  // 4 MiB: ~7,800 partial rows after the counters
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex scratch_mu;
void* scratch_ptr[MAX_DEVICES];  // this device's copy of `scratch`, from hipGetSymbolAddress
bool scratch_cleared[MAX_DEVICES];
// The stream of the first call on each device: every later call must be on it, so that calls
// sharing the device's scratch are ordered (calls on two streams could overlap and race on it).
hipStream_t scratch_stream[MAX_DEVICES];
bool scratch_bound[MAX_DEVICES];

__global__ void clear_words_kernel(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

// Zeroes the counter area of the scratch on `st` (a fill kernel, so that a caller's graph capture
// records no memset node).
int clear_scratch_counters(void* p, hipStream_t st) {
  hipLaunchKernelGGL(clear_words_kernel, dim3(32), dim3(256), 0, st, static_cast<uint32_t*>(p),
                     (int)(WS_COUNTER_BYTES / 4));
  LQ_CHECK_LAUNCH("clear_words_kernel");
  return LQ_OK;
}

// The current device's scratch address (looked up once per device with that device current,
// kept for later calls); on its first use the counter area is cleared on `st`. A call on another
// stream than the device's first call is refused before anything is launched.
int current_scratch(hipStream_t st, void** out) {
  int dev = 0;
  LQ_CHECK_HIP(hipGetDevice(&dev));
  LQ_CHECK_ARG(dev >= 0 && dev < MAX_DEVICES, "device %d outside [0, %d)", dev, MAX_DEVICES);
  std::lock_guard<std::mutex> lock(scratch_mu);
  LQ_CHECK_ARG(!scratch_bound[dev] || scratch_stream[dev] == st,
               "the static scratch of device %d is bound to stream %p, the stream of the first "
               "lq_q8_decode_append_attn_noalloc call on it; this call is on stream %p (calls on "
               "two streams could overlap and race on the scratch)",
               dev, (void*)scratch_stream[dev], (void*)st);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    LQ_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    LQ_CHECK_ARG(p != nullptr, "no device address for the static scratch");
    scratch_ptr[dev] = p;
  }
  if (!scratch_cleared[dev]) {
    const int st_clear = clear_scratch_counters(scratch_ptr[dev], st);
    if (st_clear != LQ_OK) return st_clear;
    scratch_cleared[dev] = true;
  }
  scratch_stream[dev] = st;
  scratch_bound[dev] = true;
  *out = scratch_ptr[dev];
  return LQ_OK;
}

}  // namespace
}  // namespace lq

extern "C" int lq_q8_decode_append_attn_noalloc(const uint16_t* q, const uint16_t* k_new,
                                                const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
                                                uint16_t* kb, uint8_t* vc, uint16_t* vs,
                                                uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv,
                                                int64_t D, int64_t cap, int64_t n,
                                                const int32_t* lens_host, float scale,
                                                uint16_t* out, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(B >= 1 && B <= LQ_MAX_SEQS, "batch %lld outside [1, %d]", (long long)B, LQ_MAX_SEQS);
  // the workspace this call needs (lengths after the append), against the scratch's size
  int32_t after[LQ_MAX_SEQS];
  if (lens_host)
    for (int64_t b = 0; b < B; ++b) after[b] = lens_host[b] + 1;
  const int64_t need = lq_decode_workspace_bytes(LQ_KV_Q8, B, Hq, Hkv, D, n + 1,
                                                 lens_host ? after : nullptr);
  if (need < 0) return LQ_EINVAL;  // error set
  if (need > SCRATCH_BYTES) {
    set_error("this call needs a %lld-byte workspace; the static scratch of "
              "lq_q8_decode_append_attn_noalloc holds %lld bytes (call lq_q8_decode_append_attn "
              "with a workspace instead)",
              (long long)need, (long long)SCRATCH_BYTES);
    return LQ_EWORKSPACE;
  }
  void* ws = nullptr;
  const hipStream_t st = (hipStream_t)stream;
  int rc = current_scratch(st, &ws);
  if (rc != LQ_OK) return rc;
  rc = lq_q8_decode_append_attn(q, k_new, v_new, kc, ks, kb, vc, vs, vb, B, Hq, Hkv, D, cap, n,
                                lens_host, scale, out, ws, SCRATCH_BYTES, stream);
  if (rc == LQ_EHIP) {  // a launch may have left counters set: clear them for the next call
    std::string msg = lq_last_error();
    clear_scratch_counters(ws, st);
    set_error("%s", msg.c_str());
  }
  return rc;
}
