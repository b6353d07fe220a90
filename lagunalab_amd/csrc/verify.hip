// Multi-query causal verify attention over the 8-bit cache (speculative-decoding verify step).
#include "common.h"

extern "C" int64_t lq_verify_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                             int64_t D, int64_t n) {
  (void)B; (void)Hq; (void)Hkv; (void)L; (void)D; (void)n;
  lq::set_error("lq_q8_verify_attn is not built yet");
  return -1;
}

extern "C" int lq_q8_verify_attn(const uint16_t* q, const uint8_t* kc, const uint16_t* ks,
                                 const uint16_t* kb, const uint8_t* vc, const uint16_t* vs,
                                 const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t L,
                                 int64_t D, int64_t cap, int64_t n, float scale, uint16_t* out,
                                 void* workspace, int64_t workspace_bytes, void* stream) {
  (void)q; (void)kc; (void)ks; (void)kb; (void)vc; (void)vs; (void)vb; (void)B; (void)Hq;
  (void)Hkv; (void)L; (void)D; (void)cap; (void)n; (void)scale; (void)out; (void)workspace;
  (void)workspace_bytes; (void)stream;
  lq::set_error("lq_q8_verify_attn is not built yet");
  return LQ_EINVAL;
}
