// Single-token decode attention over the 4-bit cache (group 64, two codes per byte, the even
// element in the low nibble). The reference refuses a fused 4-bit decode
// (laguna_mlx/cache.py:81-82) and runs dequantize + SDPA for it (cache.py:99-100,
// laguna.py:107); this is that computation in one pass over the packed cache.
//
// Same plan and structure as the packed 8-bit kernel (qattn.hip), with what 4 bits change:
//  * A 64-key super-tile is 4 KB of K, 4 KB of V and the four scale/bias word arrays (12 copies);
//    with the shared q rows the workgroup takes 83.6 KB of LDS, one workgroup per CU (at long
//    contexts the 32-split cap of the in-kernel merge gives one per CU anyway; 64 splits on two
//    per CU, when two still fitted, were slower).
//  * Rows are 64 bytes; chunk c of row r sits at chunk position c ^ ((r >> 2) & 3), which puts
//    the 16 rows read together in 16 different bank quarters.
//  * Codes become fp16 subnormals by masking: a 16-bit half keeps one nibble, at c * 2^-24 (low
//    nibble) or 16 c * 2^-24 (high nibble), so 8 codes take 5 operations (two masks of the word,
//    one shift, two masks of the shifted word) and come out in the k-slot order {0, 4, 1, 5, 2, 6,
//    3, 7}. One 32-bit word of K (8 dims) is one MFMA step; the q operands follow that order with
//    1/16 on the high-nibble slots. One ds_read_b64_tr_b8 of V gives every lane 8 keys of two
//    adjacent dims, i.e. two A operands (even dims at 2^-24, odd dims at 16 * 2^-24: their
//    accumulators are scaled by 1/16 at the end), with the P operand in the same key order.
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

constexpr int QW = 4;
constexpr int QTHR = 64 * QW;
constexpr int QPST = 64;
constexpr int QROW = D / 2;  // bytes per 4-bit row

struct Q4Buf {
  uint8_t k[QPST * QROW];
  uint8_t v[QPST * QROW];
  uint32_t ks[QPST];
  uint32_t kb[QPST];
  uint32_t vs[QPST];
  uint32_t vb[QPST];
};

struct Q4Terms {  // per key of the current super-tile
  float ks0[QPST], ks1[QPST], ku0[QPST], ku1[QPST];
  float vs0[QPST], vs1[QPST], vb0[QPST], vb1[QPST];
};

struct Q4Smem {
  struct {
    Q4Buf buf[QW][2];  // a wave's two also hold its partial rows after its loop
    Q4Terms terms[QW];
  } loop;
  struct {
    alignas(16) float st[QW][4][6];
    int last;
  } fin;
};
static_assert(sizeof(Q4Buf) * 2 >= sizeof(float) * (6 * 128 + 256), "wave buffers hold the finish rows");

// The q rows as fp16 B operands in k-slot order, written once per workgroup (wave r converts row
// r), with each row's half sums times the score scale; row QW is the zero row of the lanes that
// hold no operand.
struct Q4QRows {
  alignas(16) _Float16 h[QW + 1][128];
  float s[QW][2];
};
static_assert(QW >= 4, "one wave per q row");

// 8 nibble codes of one word (element 2j in the low nibble of byte j) as fp16 subnormals, in the
// k-slot order {0, 4, 1, 5, 2, 6, 3, 7}: masks keep two nibbles per word, one in each half, so
// that each 16-bit half holds one code. Low nibbles land at c * 2^-24, high nibbles (bits 4-7 of a
// half) at 16 c * 2^-24; the other operand carries 1/16 for those slots. Five operations per eight
// codes.
constexpr uint32_t NIB_LO = 0x000f000fu, NIB_HI = 0x00f000f0u;
__device__ __forceinline__ half8_t nib8_sub(uint32_t w) {
  const uint32_t w8 = w >> 8;
  typedef uint32_t u4v_t __attribute__((ext_vector_type(4)));
  const u4v_t u = {w & NIB_LO, w & NIB_HI, w8 & NIB_LO, w8 & NIB_HI};
  return __builtin_bit_cast(half8_t, u);
}

template <bool CAUSAL>
__global__ __launch_bounds__(QTHR) void q4_attn_packed_kernel(AttnArgs args, DecodePlan plan) {
  __shared__ Q4Smem sm;
  __shared__ Q4QRows qsh;

  const uint16_t* __restrict__ q = args.q;
  const uint8_t* __restrict__ kc = args.kc;
  const uint16_t* __restrict__ ks = args.ks;
  const uint16_t* __restrict__ kb = args.kb;
  const uint8_t* __restrict__ vc = args.vc;
  const uint16_t* __restrict__ vs = args.vs;
  const uint16_t* __restrict__ vb = args.vb;
  const int Hkv = args.Hkv, G = args.G, L = args.L;
  const int64_t cap = args.cap;
  const float qk_scale_log2 = args.qk_scale_log2;
  LQ_ARG_BATCH("s"(q), "s"(kc), "s"(ks), "s"(kb), "s"(vc), "s"(vs), "s"(vb), "s"(cap), "s"(Hkv),
               "s"(G), "s"(L), "s"(plan.nseq), "s"(plan.chunk), "s"(plan.split_begin[1]),
               "s"(plan.len[0]));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  const SeqSplits sq = seq_splits(plan, x);
  const int b = sq.b;
  const int n = sq.len;
  const int c_begin = (x - sq.s0) * plan.chunk;
  const int c_end = min(c_begin + plan.chunk, n);
  const int sub = (c_end - c_begin + QW - 1) / QW;
  const int w_begin = min(c_begin + wv * sub, c_end);
  const int w_end = min(w_begin + sub, c_end);
  const int nst = (w_end - w_begin + QPST - 1) / QPST;
  const int R = G * L;  // <= 4
  const int Hq = Hkv * G;
  const int64_t row0 = ((int64_t)b * Hkv + hk) * cap;

  const int lc = lane & 15;
  const int lq4 = lane >> 4;
  const int mt = lc >> 2;
  const int rho = lc & 3;
  const bool qvalid = rho < R;
  const int gh = qvalid ? rho / L : 0;
  const int qi = qvalid ? rho - gh * L : 0;
  const int causal_bound = n - L + qi;

  half8_t qb[16];
  float qsum[2];
  f4_t oacc[8];  // tile 2t + p: dims 32 t + 2 row + p
  float m_run = -INFINITY, lsum = 0.f, bsum0 = 0.f, bsum1 = 0.f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};

  const uint8_t* kbase = kc + row0 * QROW;
  const uint8_t* vbase = vc + row0 * QROW;
  const uint32_t* ksw = reinterpret_cast<const uint32_t*>(ks + row0 * 2);
  const uint32_t* kbw = reinterpret_cast<const uint32_t*>(kb + row0 * 2);
  const uint32_t* vsw = reinterpret_cast<const uint32_t*>(vs + row0 * 2);
  const uint32_t* vbw = reinterpret_cast<const uint32_t*>(vb + row0 * 2);
  Q4Terms& tm = sm.loop.terms[wv];

  // 12 copies per super-tile: copy u of lane l moves 16 bytes of row 16 u + l / 4, chunk
  // (l % 4) ^ (l / 16) (= chunk position l % 4 with the row's swizzle), plus the 4 word arrays.
  // A full super-tile takes three copy groups (K, V, words) under one M0 each, at a 32-bit
  // per-lane offset from fixed bases (the word bases shifted back by the arrays' LDS spacing);
  // the wave's last, partial super-tile clamps each lane's rows and goes copy by copy.
  const uint32_t lds_bufs = lds_addr(&sm.loop.buf[wv][0]);
  const uint32_t col_off = (uint32_t)(16 * ((lane & 3) ^ (lane >> 4)));
  const uint32_t ro0 = (uint32_t)((lane >> 2) * QROW) + col_off;
  constexpr int WSP = QPST * 4;  // bytes between the word arrays in LDS
  static_assert(offsetof(Q4Buf, kb) == offsetof(Q4Buf, ks) + WSP &&
                offsetof(Q4Buf, vs) == offsetof(Q4Buf, ks) + 2 * WSP &&
                offsetof(Q4Buf, vb) == offsetof(Q4Buf, ks) + 3 * WSP, "word arrays WSP apart");
  const uint8_t* kbw_s = reinterpret_cast<const uint8_t*>(kbw) - WSP;
  const uint8_t* vsw_s = reinterpret_cast<const uint8_t*>(vsw) - 2 * WSP;
  const uint8_t* vbw_s = reinterpret_cast<const uint8_t*>(vbw) - 3 * WSP;
  auto issue = [&](int si, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr int OK = offsetof(Q4Buf, k), OV = offsetof(Q4Buf, v);
    constexpr int OKS = offsetof(Q4Buf, ks), OKB = offsetof(Q4Buf, kb);
    constexpr int OVS = offsetof(Q4Buf, vs), OVB = offsetof(Q4Buf, vb);
    const int t0 = w_begin + si * QPST;
    const uint32_t lb = lds_bufs + (uint32_t)(BUF * sizeof(Q4Buf));
    if (t0 + QPST <= w_end) {
      const uint32_t vo = ro0 + (uint32_t)t0 * QROW;
      dma4_b128<OK, 16 * QROW>(kbase, vo, lb);
      dma4_b128<OV, 16 * QROW>(vbase, vo, lb);
      dma4_b32<OKS, WSP>(ksw, kbw_s, vsw_s, vbw_s, 4u * (uint32_t)(t0 + lane), lb);
      return;
    }
    const int last = max(w_end - 1, 0);
    uint32_t ro[4];
#pragma unroll
    for (int u = 0; u < 4; ++u)
      ro[u] = (uint32_t)min(t0 + 16 * u + (lane >> 2), last) * QROW + col_off;
    const uint32_t wo = 4u * (uint32_t)min(t0 + lane, last);
    dma_b128<OK + 0>(kbase, ro[0], lb);
    dma_b128<OK + 1024>(kbase, ro[1], lb);
    dma_b128<OK + 2048>(kbase, ro[2], lb);
    dma_b128<OK + 3072>(kbase, ro[3], lb);
    dma_b128<OV + 0>(vbase, ro[0], lb);
    dma_b128<OV + 1024>(vbase, ro[1], lb);
    dma_b128<OV + 2048>(vbase, ro[2], lb);
    dma_b128<OV + 3072>(vbase, ro[3], lb);
    dma_b32<OKS>(ksw, wo, lb);
    dma_b32<OKB>(kbw, wo, lb);
    dma_b32<OVS>(vsw, wo, lb);
    dma_b32<OVB>(vbw, wo, lb);
  };

  const uint32_t sel_lo0 = mt == 0 ? ~0u : 0u, sel_hi0 = mt == 1 ? ~0u : 0u;
  const uint32_t sel_lo1 = mt == 2 ? ~0u : 0u, sel_hi1 = mt == 3 ? ~0u : 0u;
  // Per-key K factor: scale * log2(e) * 2^24 (codes enter the MFMA as c * 2^-24) / 2^kq (the q
  // operands' power-of-two factor, set with them below).
  float kscale = qk_scale_log2 * 16777216.0f;
  VScale vsc;  // P.V factors 2^kv of the two quant groups (set by the first tile)

  auto process = [&](int si, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = w_begin + si * QPST;
    const Q4Buf& pb = sm.loop.buf[wv][BUF];
    float sv0, sv1, va0, va1;  // V scales of this lane's key; |scale_v| if valid
    {
      const uint32_t a = pb.ks[lane], c = pb.kb[lane], e = pb.vs[lane], f = pb.vb[lane];
      sv0 = bf16_lo(e);
      sv1 = bf16_hi(e);
      const bool kv = t0 + lane < w_end;  // rows past the wave's range are clamped copies
      va0 = kv ? fabsf(sv0) : 0.0f;
      va1 = kv ? fabsf(sv1) : 0.0f;
      tm.ks0[lane] = bf16_lo(a) * kscale;
      tm.ks1[lane] = bf16_hi(a) * kscale;
      tm.ku0[lane] = bf16_lo(c);
      tm.ku1[lane] = bf16_hi(c);
      tm.vs0[lane] = sv0 * vsc.f0;
      tm.vs1[lane] = sv1 * vsc.f1;
      tm.vb0[lane] = bf16_lo(f);
      tm.vb1[lane] = bf16_hi(f);
    }
    // Q.K^T: A = key row lc of tile lq4; chunk c of the row is steps 4c .. 4c + 3 (one word per
    // 8-dim step); chunks 0-1 are quant group 0, chunks 2-3 group 1 (independent chains).
    f4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    {
      const int r = 16 * lq4 + lc;
      const int sw = (r >> 2) & 3;
      const uint8_t* kr = pb.k + r * QROW;
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        const uint4 a = *reinterpret_cast<const uint4*>(kr + 16 * (c2 ^ sw));
        const uint4 g = *reinterpret_cast<const uint4*>(kr + 16 * ((c2 + 2) ^ sw));
        const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, gw[4] = {g.x, g.y, g.z, g.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(nib8_sub(aw[j]), qb[4 * c2 + j], c0, 0, 0, 0);
          c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(nib8_sub(gw[j]), qb[8 + 4 * c2 + j], c1, 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const int k0 = 16 * mt + 4 * lq4;
    const float4 ks0 = *reinterpret_cast<const float4*>(tm.ks0 + k0);
    const float4 ks1 = *reinterpret_cast<const float4*>(tm.ks1 + k0);
    const float4 ku0 = *reinterpret_cast<const float4*>(tm.ku0 + k0);
    const float4 ku1 = *reinterpret_cast<const float4*>(tm.ku1 + k0);
    const float ks0v[4] = {ks0.x, ks0.y, ks0.z, ks0.w}, ks1v[4] = {ks1.x, ks1.y, ks1.z, ks1.w};
    const float ku0v[4] = {ku0.x, ku0.y, ku0.z, ku0.w}, ku1v[4] = {ku1.x, ku1.y, ku1.z, ku1.w};
    float sc[4];
    const bool full = t0 + QPST <= w_end && (!CAUSAL || t0 + QPST - 1 <= n - L);
#pragma unroll
    for (int r = 0; r < 4; ++r)
      sc[r] = fmaf(ks0v[r], c0[r], fmaf(ks1v[r], c1[r], fmaf(ku1v[r], qsum[1], ku0v[r] * qsum[0])));
    if (!full) {  // keys past the wave's range or the row's causal bound (last super-tile only)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + k0 + r;
        bool ok = t < w_end;
        if (CAUSAL) ok = ok && t <= causal_bound;
        sc[r] = ok ? sc[r] : -INFINITY;
      }
    }
    float tmax = fmaxf(fmaxf(sc[0], sc[1]), fmaxf(sc[2], sc[3]));
    tmax = max_ieee(tmax, dpp<DPP_ROW_ROR4>(tmax));
    tmax = max_ieee(tmax, dpp<DPP_ROW_ROR8>(tmax));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    const bool bump = tmax > m_run + RESCALE_LOG2;
    const uint64_t bumps = __builtin_amdgcn_ballot_w64(bump);
    const bool vnew = vscale_check(va0, va1, vsc);
    if (bumps || vnew) {  // rare: a new running max, or new P.V factors
      if (bumps) {
        const float mn = bump ? tmax : m_run;
        const float alpha = m_run == -INFINITY ? 0.0f : exp2_nonpos(m_run - mn);
        // while no lane has seen a key (the wave's first super-tile) the sums are all zero
        if (__builtin_amdgcn_ballot_w64(m_run != -INFINITY)) {
          lsum *= alpha;
          bsum0 *= alpha;
          bsum1 *= alpha;
#pragma unroll
          for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
        }
        m_run = mn;
      }
      if (vnew) {  // the terms read below are rewritten with the new factors
        vscale_apply(va0, va1, vsc, oacc);
        tm.vs0[lane] = sv0 * vsc.f0;
        tm.vs1[lane] = sv1 * vsc.f1;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      }
    }
    const float mref = m_run == -INFINITY ? 0.0f : m_run;
    const float4 vs0 = *reinterpret_cast<const float4*>(tm.vs0 + k0);
    const float4 vs1 = *reinterpret_cast<const float4*>(tm.vs1 + k0);
    const float4 vb0 = *reinterpret_cast<const float4*>(tm.vb0 + k0);
    const float4 vb1 = *reinterpret_cast<const float4*>(tm.vb1 + k0);
    const float vs0v[4] = {vs0.x, vs0.y, vs0.z, vs0.w}, vs1v[4] = {vs1.x, vs1.y, vs1.z, vs1.w};
    const float vb0v[4] = {vb0.x, vb0.y, vb0.z, vb0.w}, vb1v[4] = {vb1.x, vb1.y, vb1.z, vb1.w};
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      p[r] = __builtin_amdgcn_exp2f(sc[r] - mref);
      lsum += p[r];
      bsum0 = fmaf(p[r], vb0v[r], bsum0);
      bsum1 = fmaf(p[r], vb1v[r], bsum1);
    }
    // keys in the V operands' k-slot order: r = 0, 2, 1, 3
    const uint32_t w00 = pack_h2(p[0] * vs0v[0], p[2] * vs0v[2]);
    const uint32_t w01 = pack_h2(p[1] * vs0v[1], p[3] * vs0v[3]);
    const uint32_t w10 = pack_h2(p[0] * vs1v[0], p[2] * vs1v[2]);
    const uint32_t w11 = pack_h2(p[1] * vs1v[1], p[3] * vs1v[3]);
    // P.V: K-step e covers key tiles 2e (slots 0-3) and 2e+1 (slots 4-7); one transposed read of
    // 32-dim slab t gives lane lc the bytes of dims 32 t + 2 lc, + 1 for its 8 keys.
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t slo = e == 0 ? sel_lo0 : sel_lo1, shi = e == 0 ? sel_hi0 : sel_hi1;
      const half8_t b0 = words_as_h8(w00 & slo, w01 & slo, w00 & shi, w01 & shi);
      const half8_t b1 = words_as_h8(w10 & slo, w11 & slo, w10 & shi, w11 & shi);
      const int j = lc >> 1;
      const int key = 16 * (2 * e + (j >> 2)) + 4 * lq4 + (j & 3);
      const uint8_t* vrow = pb.v + key * QROW + 8 * (lc & 1);
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const v2i_t raw =
            __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)(vrow + 16 * (t ^ lq4)));
        // bytes j = keys j of dims (2 lc', 2 lc' + 1); per 4 bytes: keys 0, 2 then 1, 3
        const uint32_t x0 = (uint32_t)raw.x, x1 = (uint32_t)raw.y;
        const uint32_t y0 = x0 >> 8, y1 = x1 >> 8;
        const half8_t ae = words_as_h8(x0 & NIB_LO, y0 & NIB_LO, x1 & NIB_LO, y1 & NIB_LO);
        const half8_t ao = words_as_h8(x0 & NIB_HI, y0 & NIB_HI, x1 & NIB_HI, y1 & NIB_HI);
        const half8_t& bg = t < 2 ? b0 : b1;
        oacc[2 * t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ae, bg, oacc[2 * t], 0, 0, 0);
        oacc[2 * t + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ao, bg, oacc[2 * t + 1], 0, 0, 0);
      }
    }
  };

  const std::integral_constant<int, 0> B0;
  const std::integral_constant<int, 1> B1;
  // Prologue: the R q rows (contiguous, <= 1 KB) go to this wave's terms area by DMA (free until
  // the first super-tile is processed), then super-tile 0; only the q copy is waited for before
  // the q operands are built, and super-tile 1 is issued after them, behind every wave's
  // super-tile 0 (26.5 -> 26.1 us). Nothing is issued for super-tiles past the wave's range.
  {
    const uint16_t* qblk = q + ((int64_t)b * Hq + hk * G) * L * D;
    dma_b128<0>(qblk, (uint32_t)min(16 * lane, R * 2 * D - 16), lds_addr(&tm));
  }
  if (nst > 0) issue(0, B0);
  if (nst > 0)
    asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // q operands times the workgroup's power-of-two q factor 2^kq (from the largest |q| element of
  // its R rows): wave w converts row w (w < R) once for the workgroup into the shared fp16 rows,
  // with the row's two half sums; after a barrier over LDS (the copies of super-tile 0 stay in
  // flight) every lane reads its row whole, the lanes without an operand the zero row. Dim 8 s + e
  // goes to k-slot {0, 2, 4, 6, 1, 3, 5, 7}[e] of qb[s] (the order nib8_sub gives the codes), odd
  // dims times 1/16 (their codes enter at 16 c * 2^-24).
  {
    const uint32_t* own = reinterpret_cast<const uint32_t*>(&tm);  // q rows 64 words apart
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < QW; ++j)
      if (j < R) {
        const uint32_t w = own[64 * j + lane];
        amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(w)), fabsf(bf16_hi(w))));
      }
    const int kq = q_pow2_exp(amax);
    const float qf = pow2f(kq);
    kscale = qk_scale_log2 * pow2f(24 - kq);
    if (wv < R) {  // lane l: dims 2 l, 2 l + 1 = dims e, e + 1 of slab s = l / 4, e = 2 (l % 4)
      const uint32_t xq = own[64 * wv + lane];
      const float lo = bf16_lo(xq), hi = bf16_hi(xq);
      const int e = 2 * (lane & 3);
      const int slot = 2 * (e & 2) + (e >> 2);  // k-slot of dim e; dim e + 1 sits two slots on
      _Float16* hrow = &qsh.h[wv][8 * (lane >> 2)];
      hrow[slot] = (_Float16)(lo * qf);
      hrow[slot + 2] = (_Float16)(hi * (qf * 0.0625f));
      float sg = lo + hi;  // over dims 0-63 (lanes 0-31) and 64-127 (lanes 32-63)
      sg += dpp<DPP_QUAD_XOR1>(sg);
      sg += dpp<DPP_QUAD_XOR2>(sg);
      sg += dpp<DPP_ROW_ROR4>(sg);
      sg += dpp<DPP_ROW_ROR8>(sg);
      sg = sum_xor16(sg);
      if ((lane & 31) == 0) qsh.s[wv][lane >> 5] = sg * qk_scale_log2;
    }
    if (wv == 0) reinterpret_cast<uint32_t*>(&qsh.h[QW][0])[lane] = 0u;
    lds_barrier();
    const bool on = qvalid && mt == lq4;
    const half8_t* qr = reinterpret_cast<const half8_t*>(&qsh.h[on ? rho : QW][0]);
#pragma unroll
    for (int st = 0; st < 16; ++st) qb[st] = qr[st];
    qsum[0] = qvalid ? qsh.s[rho][0] : 0.0f;
    qsum[1] = qvalid ? qsh.s[rho][1] : 0.0f;
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // q reads done before terms overwrite
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (nst > 1) issue(1, B1);

  // Step si waits for super-tile si (all but the copies of si + 1, when those were issued),
  // processes it, then refills its buffer with super-tile si + 2 if that is in range.
  for (int si = 0; si < nst; si += 2) {
    if (si + 1 < nst)
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    process(si, B0);
    if (si + 1 >= nst) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer refilled next are done
    if (si + 2 < nst) issue(si + 2, B0);
    if (si + 2 < nst)
      asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    process(si + 1, B1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (si + 3 < nst) issue(si + 3, B1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  float osc[4];  // output factors: 2^24 over the P.V factors, and 1/16 for the odd dims (their
  vscale_out(vsc, 16777216.0f, 0.0625f, osc);  // codes entered as 16 c)
  packed_finish<QW, true>(oacc, m_run, lsum, bsum0, bsum1, osc,
                          reinterpret_cast<float*>(&sm.loop.buf[0][0]),
                          (int)(2 * sizeof(Q4Buf) / sizeof(float)), &sm.fin.st[0][0][0],
                          &sm.fin.last, args, plan, x, b, hk, R);
}

}  // namespace

QAttnFn q4_attn_fn(bool causal) {
  return causal ? q4_attn_packed_kernel<true> : q4_attn_packed_kernel<false>;
}

}  // namespace lq
