// Multi-query causal verify attention over the 8-bit cache (speculative-decoding verify step).
//
// Replaces the verify forward's attention of the reference's speculative loop
// (laguna_mlx/dflash.py:195) over DequantKVCache's dequantized K/V (cache.py:99-100) with the
// bottom-right causal mask (laguna.py:107, 183-186): the L query rows of each head are the
// block's own last L keys, and row i sees keys 0 .. n-L+i. G*L <= 4 rows per KV head take the
// packed decode kernel (qattn.hip) -- except a single sequence of at most 65,536 rows --, the
// rest the dense kernel (attn_dense.hip), with the causal bound applied per query row.
#include "common.h"
#include "qattn.h"

extern "C" int64_t lq_verify_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                             int64_t D, int64_t n) {
  using namespace lq;
  clear_error();
  if (D != 128 || Hkv < 1 || Hq % Hkv || L < 1 || L > 16 || (Hq / Hkv) * L > 64) {
    set_error("unsupported verify configuration");
    return -1;
  }
  const int64_t ws = attn_workspace_bytes(LQ_KV_Q8, B, Hq, Hkv, L, n, nullptr);
  if (ws < 0) set_error("bad sequence length");
  return ws;
}

namespace lq {
namespace {

// Causal verify attention over n rows (the block's L rows are the last L). With k_new/v_new the
// block's rows [n - L, n) are first appended from them: inside the dense kernel when
// G * L > 4, else by one quantize_append launch before the packed kernel.
int verify_attn(const uint16_t* q, const uint16_t* k_new, const uint16_t* v_new, uint8_t* kc,
                uint16_t* ks, uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb, int64_t B,
                int64_t Hq, int64_t Hkv, int64_t L, int64_t D, int64_t cap, int64_t n, float scale,
                uint16_t* out, void* workspace, int64_t workspace_bytes, hipStream_t st) {
  LQ_CHECK_ARG(D == 128, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(L >= 1 && L <= 16, "verify block of %lld rows outside [1, 16]", (long long)L);
  LQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "Hq=%lld must be a multiple of Hkv=%lld",
               (long long)Hq, (long long)Hkv);
  LQ_CHECK_ARG((Hq / Hkv) * L <= 64, "G * L = %lld query rows per KV head exceed 64",
               (long long)((Hq / Hkv) * L));
  LQ_CHECK_ARG(B >= 1 && B <= LQ_MAX_SEQS, "batch %lld outside [1, %d]", (long long)B, LQ_MAX_SEQS);
  LQ_CHECK_ARG(n >= L && n <= cap && cap <= (1 << 24),
               "n=%lld must be in [L, cap=%lld], cap <= 2^24", (long long)n, (long long)cap);
  LQ_CHECK_ARG(B * Hkv <= MAX_COUNTERS, "B * Hkv = %lld exceeds %lld", (long long)(B * Hkv),
               (long long)MAX_COUNTERS);
  LQ_CHECK_ARG(q && kc && ks && kb && vc && vs && vb && out, "null pointer");
  DecodePlan plan;
  AttnKernel kern;
  int64_t need = 0;
  const int64_t S = attn_plan(LQ_KV_Q8, B, Hq, Hkv, L, n, nullptr, cap, plan, kern, need);
  LQ_CHECK_ARG(S > 0, "bad sequence length");
  if (!workspace || workspace_bytes < need) {
    set_error("workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
              (long long)need);
    return LQ_EWORKSPACE;
  }
  const bool packed = kern.packed;
  AttnArgs a{};
  a.q = q;
  a.kc = kc;
  a.ks = ks;
  a.kb = kb;
  a.vc = vc;
  a.vs = vs;
  a.vb = vb;
  if (k_new && !packed) {  // the dense kernel appends the block's rows itself
    a.knew = k_new;
    a.vnew = v_new;
  } else if (k_new) {  // one launch for K and V of every sequence: rows [n - L, n)
    const int rc = quantize_append(AppendTarget{k_new, kc, ks, kb}, AppendTarget{v_new, vc, vs, vb},
                                   1, B, Hkv, L, D, cap, n - L, 8, 64, st);
    if (rc != LQ_OK) return rc;
  }
  a.counters = reinterpret_cast<uint32_t*>(workspace);
  a.part_acc = reinterpret_cast<float*>(static_cast<char*>(workspace) + WS_COUNTER_BYTES);
  a.part_ml = reinterpret_cast<float2*>(a.part_acc + S * Hq * L * D);
  a.out = out;
  a.cap = cap;
  a.Hkv = (int)Hkv;
  a.G = (int)(Hq / Hkv);
  a.L = (int)L;
  a.qk_scale_log2 = scale * 1.4426950408889634f;
  hipLaunchKernelGGL(kern.fn, dim3((unsigned)S, (unsigned)Hkv), dim3((unsigned)kern.threads), 0,
                     st, a, plan);
  LQ_CHECK_LAUNCH("q8 attention kernel");
  if (!kern.merges) {
    launch_merge(a.part_acc, a.part_ml, (int)(Hq * L), plan, B, out, st);
    LQ_CHECK_LAUNCH("decode_merge_kernel");
  }
  return LQ_OK;
}

}  // namespace
}  // namespace lq

extern "C" int lq_q8_verify_attn(const uint16_t* q, const uint8_t* kc, const uint16_t* ks,
                                 const uint16_t* kb, const uint8_t* vc, const uint16_t* vs,
                                 const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                 int64_t D, int64_t cap, int64_t n, float scale, uint16_t* out,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  lq::clear_error();
  return lq::verify_attn(q, nullptr, nullptr, const_cast<uint8_t*>(kc), const_cast<uint16_t*>(ks),
                         const_cast<uint16_t*>(kb), const_cast<uint8_t*>(vc),
                         const_cast<uint16_t*>(vs), const_cast<uint16_t*>(vb), B, Hq, Hkv, L, D,
                         cap, n, scale, out, workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int lq_q8_verify_append_attn(const uint16_t* q, const uint16_t* k_new,
                                        const uint16_t* v_new, uint8_t* kc, uint16_t* ks,
                                        uint16_t* kb, uint8_t* vc, uint16_t* vs, uint16_t* vb,
                                        int64_t B, int64_t Hq, int64_t Hkv, int64_t L, int64_t D,
                                        int64_t cap, int64_t n, float scale, uint16_t* out,
                                        void* workspace, int64_t workspace_bytes, void* stream) {
  lq::clear_error();
  LQ_CHECK_ARG(k_new && v_new, "null pointer");
  LQ_CHECK_ARG(n >= 0 && L >= 1 && n + L <= cap, "n=%lld + L=%lld rows exceed capacity %lld",
               (long long)n, (long long)L, (long long)cap);
  return lq::verify_attn(q, k_new, v_new, kc, ks, kb, vc, vs, vb, B, Hq, Hkv, L, D, cap, n + L,
                         scale, out, workspace, workspace_bytes, (hipStream_t)stream);
}
