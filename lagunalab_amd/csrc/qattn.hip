// Fused attention over the 8-bit KV cache on MFMA for at most 4 query rows per KV head:
// single-token decode with G <= 4 and small causal verify blocks (G * L <= 4), over batches or
// over a single sequence of more than 65,536 rows. Larger blocks, and shorter single sequences,
// take the dense-layout kernel (attn_dense.hip).
//
// Replaces q8_decode_attention (laguna_mlx/q8_attn.py:102-130: the Metal kernel at :17-99 and the
// block merge at :126-130) and, for verify blocks, the reference's unfused path (dequantize,
// cache.py:99-100, then SDPA with the bottom-right causal mask, laguna.py:107, 183-186).
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;

// ----------------------------------------------------------------------------------------------
// Packed kernel for at most 4 query rows per KV head (decode with G <= 4, small verify blocks).
//
// With G*L <= 4 a 16-column MFMA would leave 12 columns idle, and every softmax instruction would
// do a quarter of useful work. Here the 16 columns are (key tile m, query row rho) = 4 m + rho and
// a super-tile is 4 key tiles x 16 keys = 64 keys:
//  * Q.K^T, 16 steps of 8 dims: k-slot (lane group t, j) = (key tile t, dim 8 s + j). A row i =
//    key row i; lane group t supplies the 8 codes of key (t, i). B[(t, j)][4 m + rho] =
//    q[rho][8 s + j] if t == m else 0 -- a constant per lane, so the product is block-diagonal and
//    column 4 m + rho accumulates exactly key tile m's scores for query rho.
//  * After it every lane holds 4 useful scores (keys 16 m + 4 lane-group + r).
//  * P.V, 2 steps of 32 keys (tiles 2e and 2e+1): k-slot j of lane group q = key
//    16 (2e + j/4) + 4 q + j % 4, i.e. exactly the keys the lane already holds for column tile
//    2e or 2e+1; the B operand is the lane's own 4 weights in the matching half, zeros elsewhere.
//    Columns of different tiles hold partial outputs that are summed once at the end.
//  * Per-key terms (scaled K scale, folded K bias, V scale and bias) are computed once per
//    super-tile by one lane per key and shared through LDS.
// ----------------------------------------------------------------------------------------------

constexpr int PST = 64;  // keys per packed super-tile

struct PackBuf {
  uint8_t k[PST * D];
  uint8_t v[PST * D];
  uint32_t ks[PST];
  uint32_t kb[PST];
  uint32_t vs[PST];
  uint32_t vb[PST];
};

struct PackTerms {  // per key of the current super-tile
  float ks0[PST], ks1[PST], ku0[PST], ku1[PST];  // s_g * scale*log2e, b_g - 1024 s_g
  float vs0[PST], vs1[PST], vb0[PST], vb1[PST];
};

struct PackSmem {
  struct {
    PackBuf buf[NWAVE][2];  // a wave's two also hold its partial rows after its loop
    PackTerms terms[NWAVE];
  } loop;
  alignas(16) float st[NWAVE][4][6];
};
static_assert(sizeof(PackBuf) * 2 >= sizeof(float) * (6 * 128 + 256), "wave buffers hold the finish rows");

// The q rows as fp16 B operands, written once per workgroup (wave r converts row r), with each
// row's half sums (times the score scale) and, in the NORM variant, its largest |element|; row
// NWAVE is the zero row of the lanes that hold no operand.
struct PackQ {
  alignas(16) uint32_t h[NWAVE + 1][64];
  float s[NWAVE][2];
  float amax[NWAVE];
};
static_assert(NWAVE >= 4, "one wave per q row");

// The NORM variant's extra staging (RoPE frequencies of each wave's copy).
template <bool NORM>
struct PackNormSmem {
  alignas(16) float inv_freq[NWAVE][64];
};
template <>
struct PackNormSmem<false> {};

template <bool CAUSAL, bool NORM>
__device__ __forceinline__ void q8_attn_packed_body(const AttnArgs& args, const DecodePlan& plan,
                                                    const NormArgs& nargs) {
  __shared__ PackSmem sm;
  __shared__ PackNormSmem<NORM> nsm;
  __shared__ PackQ qsh;
  __shared__ int sh_last;
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
  LQ_ARG_BATCH("s"(q), "s"(kc), "s"(ks), "s"(kb), "s"(vc), "s"(vs), "s"(vb), "s"(args.knew),
               "s"(args.vnew), "s"(args.pos), "s"(args.counters), "s"(cap), "s"(Hkv), "s"(G),
               "s"(L), "s"(nargs.qn_w), "s"(nargs.kn_w), "s"(nargs.inv_freq), "s"(plan.nseq),
               "s"(plan.split_begin[1]), "s"(plan.len[0]));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  const SeqSplits sq = seq_splits(plan, x);
  const int b = sq.b;
  const int n = args.pos ? (int)min(max((int64_t)args.pos[b] + 1, (int64_t)1), args.cap) : sq.len;
  // Work in super-tiles of PST keys. The NWS waves of the sequence's workgroups take about 90%
  // of them statically (wave gw: super-tiles gw + k NWS for k < NS), the rest one at a time from
  // the (sequence, KV head) tile counter, two super-tiles ahead. Waves that started late or sit
  // on busier parts of the chip (XCDs start up to ~3 us apart and differ by ~10% in the
  // bandwidth they get) then take fewer of the dynamic super-tiles.
  const int T = (n + PST - 1) / PST;
  const int NWS = sq.ns * NWAVE;
  const int gw = (x - sq.s0) * NWAVE + wv;
  const int NS = max(2, (9 * T) / (10 * NWS));  // static super-tiles per wave
  const int R = G * L;  // <= 4
  // Fused append: the wave that gets super-tile app_t (holding row n - 1, the sequence's new last
  // row) patches the new K and V rows, quantized by every wave up front, into its LDS copy of that
  // super-tile (whatever the copy read from the cache row is replaced) and stores them to the
  // cache at the end.
  const int nrow = n - 1;
  const bool app = args.knew != nullptr;
  const int app_t = app ? nrow / PST : -1;
  const int app_r = nrow - (nrow / PST) * PST;
  const int Hq = Hkv * G;
  const int64_t row0 = ((int64_t)b * Hkv + hk) * cap;

  const int lc = lane & 15;
  const int lq4 = lane >> 4;
  const int mt = lc >> 2;   // key tile of this lane's column
  const int rho = lc & 3;   // query row of this lane's column
  const bool qvalid = rho < R;
  const int gh = qvalid ? rho / L : 0;
  const int qi = qvalid ? rho - gh * L : 0;

  half8_t qb[16];  // Q.K^T B operands (filled once the first super-tile is in flight)
  float qsum[2];
  f4_t oacc[8];
  float m_run = -INFINITY, lsum = 0.f, bsum0 = 0.f, bsum1 = 0.f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};

  const uint8_t* kbase = kc + row0 * D;
  const uint8_t* vbase = vc + row0 * D;
  const uint32_t* ksw = reinterpret_cast<const uint32_t*>(ks + row0 * 2);
  const uint32_t* kbw = reinterpret_cast<const uint32_t*>(kb + row0 * 2);
  const uint32_t* vsw = reinterpret_cast<const uint32_t*>(vs + row0 * 2);
  const uint32_t* vbw = reinterpret_cast<const uint32_t*>(vb + row0 * 2);
  const int causal_bound = n - L + qi;  // query qi sees keys t <= causal_bound
  const int last_row = n - 1;
  const uint32_t ctr_off = (uint32_t)(CTR_STRIDE * (b * Hkv + hk) + 4);  // tile counter
  PackTerms& tm = sm.loop.terms[wv];

  // 20 copies per super-tile: 8 K + 8 V (1 KB each) + 4 word arrays. Copy u of lane l moves 16
  // bytes of row 8 u + l / 8, chunk l % 8 to chunk position (l % 8) ^ (l / 8) of the LDS row (the
  // swizzle read back in process). A full super-tile takes five copy groups under one M0 each
  // (K rows 0-31 and 32-63, the same for V, the word arrays), the rows 8 apart as immediate
  // offsets (which move the LDS destination with them), at a 32-bit per-lane offset from fixed
  // bases (the word bases shifted back by the arrays' LDS spacing). The last super-tile clamps
  // each lane's rows to the sequence's last row and goes copy by copy, and so do super-tiles past
  // the end (their copies land in a buffer that is never read).
  const uint32_t lds_bufs = lds_addr(&sm.loop.buf[wv][0]);
  const uint32_t col_off = (uint32_t)(16 * ((lane & 7) ^ (lane >> 3)));
  const uint32_t ro0 = (uint32_t)((lane >> 3) * D) + col_off;
  constexpr int WSP = PST * 4;  // bytes between the word arrays in LDS
  static_assert(offsetof(PackBuf, kb) == offsetof(PackBuf, ks) + WSP &&
                offsetof(PackBuf, vs) == offsetof(PackBuf, ks) + 2 * WSP &&
                offsetof(PackBuf, vb) == offsetof(PackBuf, ks) + 3 * WSP, "word arrays WSP apart");
  const uint8_t* kbase4 = kbase + 32 * D;  // rows 32-63 of a super-tile
  const uint8_t* vbase4 = vbase + 32 * D;
  const uint8_t* kbw_s = reinterpret_cast<const uint8_t*>(kbw) - WSP;
  const uint8_t* vsw_s = reinterpret_cast<const uint8_t*>(vsw) - 2 * WSP;
  const uint8_t* vbw_s = reinterpret_cast<const uint8_t*>(vbw) - 3 * WSP;
  // `between(j)` runs after copy group j (0-2) of a full super-tile, after all copies otherwise:
  // work placed there issues while the memory pipeline takes the copies issued before it.
  auto issue_with = [&](int tile, auto bufc, auto&& between) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * PST;
    const uint32_t lb = lds_bufs + (uint32_t)(BUF * sizeof(PackBuf));
    constexpr int OK = offsetof(PackBuf, k), OV = offsetof(PackBuf, v);
    constexpr int OKS = offsetof(PackBuf, ks), OKB = offsetof(PackBuf, kb);
    constexpr int OVS = offsetof(PackBuf, vs), OVB = offsetof(PackBuf, vb);
    if (t0 + PST <= n) {
      const uint32_t vo = ro0 + (uint32_t)t0 * D;
      dma4_b128<OK, 8 * D>(kbase, vo, lb);
      between(0);
      dma4_b128<OV, 8 * D>(vbase, vo, lb);
      between(1);
      dma4_b128<OK + 32 * D, 8 * D>(kbase4, vo, lb);
      between(2);
      dma4_b128<OV + 32 * D, 8 * D>(vbase4, vo, lb);
      dma4_b32<OKS, WSP>(ksw, kbw_s, vsw_s, vbw_s, 4u * (uint32_t)(t0 + lane), lb);
      return;
    }
    uint32_t ro[8];
#pragma unroll
    for (int u = 0; u < 8; ++u)
      ro[u] = (uint32_t)min(t0 + (lane >> 3) + 8 * u, last_row) * D + col_off;
    const uint32_t wo = 4u * (uint32_t)min(t0 + lane, last_row);
    dma_b128<OK + 0>(kbase, ro[0], lb);
    dma_b128<OK + 1024>(kbase, ro[1], lb);
    dma_b128<OK + 2048>(kbase, ro[2], lb);
    dma_b128<OK + 3072>(kbase, ro[3], lb);
    dma_b128<OV + 0>(vbase, ro[0], lb);
    dma_b128<OV + 1024>(vbase, ro[1], lb);
    dma_b128<OV + 2048>(vbase, ro[2], lb);
    dma_b128<OV + 3072>(vbase, ro[3], lb);
    dma_b128<OK + 4096>(kbase, ro[4], lb);
    dma_b128<OK + 5120>(kbase, ro[5], lb);
    dma_b128<OK + 6144>(kbase, ro[6], lb);
    dma_b128<OK + 7168>(kbase, ro[7], lb);
    dma_b128<OV + 4096>(vbase, ro[4], lb);
    dma_b128<OV + 5120>(vbase, ro[5], lb);
    dma_b128<OV + 6144>(vbase, ro[6], lb);
    dma_b128<OV + 7168>(vbase, ro[7], lb);
    dma_b32<OKS>(ksw, wo, lb);
    dma_b32<OKB>(kbw, wo, lb);
    dma_b32<OVS>(vsw, wo, lb);
    dma_b32<OVB>(vbw, wo, lb);
    between(0);
    between(1);
    between(2);
  };
  auto issue = [&](int tile, auto bufc) { issue_with(tile, bufc, [](int) {}); };

  // Lane masks selecting the P.V B-operand half of K-step e (key tile 2e in slots 0-3, 2e+1 in
  // slots 4-7): this lane's own key tile is mt.
  const uint32_t sel_lo0 = mt == 0 ? ~0u : 0u, sel_hi0 = mt == 1 ? ~0u : 0u;
  const uint32_t sel_lo1 = mt == 2 ? ~0u : 0u, sel_hi1 = mt == 3 ? ~0u : 0u;
  // Per-key K factor: scale * log2(e) * 2^24 (codes enter the MFMA as c * 2^-24) / 2^kq (the q
  // operands' power-of-two factor, set with them below).
  float kscale = qk_scale_log2 * 16777216.0f;
  VScale vsc;  // P.V factors 2^kv of the two quant groups (set by the first tile)

  auto process = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * PST;
    const PackBuf& pb = sm.loop.buf[wv][BUF];
    // per-key terms, one lane per key: K scale * scale * log2(e) * 2^24, K bias, V scale, V bias
    // (V scales scaled by the wave's P.V factors; |scale_v| of valid keys kept for their check)
    float sv0, sv1, va0, va1;
    {
      const uint32_t a = pb.ks[lane], c = pb.kb[lane], e = pb.vs[lane], f = pb.vb[lane];
      sv0 = bf16_lo(e);
      sv1 = bf16_hi(e);
      const bool kv = t0 + lane < n;  // rows past n are clamped copies, never attended
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
    // Q.K^T: A = key row lc of tile lq4 (codes as fp16 subnormals c * 2^-24), 16 steps of 8 dims
    // (two steps per 16-byte LDS read); the two quant groups accumulate in independent chains.
    f4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    {
      const int r = 16 * lq4 + lc;
      const uint8_t* kr = pb.k + r * D;
#pragma unroll
      for (int s2 = 0; s2 < 4; ++s2) {
        const uint4 a = *reinterpret_cast<const uint4*>(kr + 16 * (s2 ^ (r & 7)));
        const uint4 b = *reinterpret_cast<const uint4*>(kr + 16 * ((s2 + 4) ^ (r & 7)));
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes8_sub(a.x, a.y), qb[2 * s2], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes8_sub(b.x, b.y), qb[2 * s2 + 8], c1, 0, 0, 0);
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes8_sub(a.z, a.w), qb[2 * s2 + 1], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(codes8_sub(b.z, b.w), qb[2 * s2 + 9], c1, 0, 0, 0);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // this lane's keys: k0 + r, r = 0..3
    const int k0 = 16 * mt + 4 * lq4;
    const float4 ks0 = *reinterpret_cast<const float4*>(tm.ks0 + k0);
    const float4 ks1 = *reinterpret_cast<const float4*>(tm.ks1 + k0);
    const float4 ku0 = *reinterpret_cast<const float4*>(tm.ku0 + k0);
    const float4 ku1 = *reinterpret_cast<const float4*>(tm.ku1 + k0);
    const float ks0v[4] = {ks0.x, ks0.y, ks0.z, ks0.w}, ks1v[4] = {ks1.x, ks1.y, ks1.z, ks1.w};
    const float ku0v[4] = {ku0.x, ku0.y, ku0.z, ku0.w}, ku1v[4] = {ku1.x, ku1.y, ku1.z, ku1.w};
    float sc[4];
    float tmax = -INFINITY;
    const bool full = t0 + PST <= n && (!CAUSAL || t0 + PST - 1 <= n - L);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = fmaf(ks0v[r], c0[r], fmaf(ks1v[r], c1[r], fmaf(ku1v[r], qsum[1], ku0v[r] * qsum[0])));
      if (!full) {
        const int t = t0 + k0 + r;
        bool ok = t < n;
        if (CAUSAL) ok = ok && t <= causal_bound;
        v = ok ? v : -INFINITY;
      }
      sc[r] = v;
      tmax = fmaxf(tmax, v);
    }
    // max over the 4 key tiles (lanes 4 apart in a row) and the 4 lane groups
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
    // P * scale_v * 2^kv in fp16, two keys per dword, per quant group
    const uint32_t w00 = pack_h2(p[0] * vs0v[0], p[1] * vs0v[1]);
    const uint32_t w01 = pack_h2(p[2] * vs0v[2], p[3] * vs0v[3]);
    const uint32_t w10 = pack_h2(p[0] * vs1v[0], p[1] * vs1v[1]);
    const uint32_t w11 = pack_h2(p[2] * vs1v[2], p[3] * vs1v[3]);
    // P.V, K-step e covers key tiles 2e (slots 0-3) and 2e+1 (slots 4-7)
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t slo = e == 0 ? sel_lo0 : sel_lo1, shi = e == 0 ? sel_hi0 : sel_hi1;
      const half8_t b0 = words_as_h8(w00 & slo, w01 & slo, w00 & shi, w01 & shi);
      const half8_t b1 = words_as_h8(w10 & slo, w11 & slo, w10 & shi, w11 & shi);
      const int j = lc >> 1;
      const int key = 16 * (2 * e + (j >> 2)) + 4 * lq4 + (j & 3);
      const uint8_t* vrow = pb.v + key * D + 8 * (lc & 1);
      const int sw = key & 7;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const v2i_t raw = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)(vrow + 16 * (dt ^ sw)));
        const half8_t a = codes8_sub((uint32_t)raw.x, (uint32_t)raw.y);
        oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, dt < 4 ? b0 : b1, oacc[dt], 0, 0, 0);
      }
    }
  };

  const std::integral_constant<int, 0> B0;
  const std::integral_constant<int, 1> B1;
  // One tile-counter increment by lane 0 when `dyn` (exec narrowed to lane 0 inside the asm, or
  // to no lane for a static step: the same instruction sequence every step, so that the waits
  // below keep fixed counts), the old value landing later in lane 0 of g. Inline asm like the
  // copies, so that the compiler inserts no wait for it: `landed` reads it in the same statement
  // as the explicit s_waitcnt that covers it, and g is an in-out operand of both statements so
  // that it stays in its register in between (vector memory operations complete in issue order;
  // every step ends with a grab and the 20 copies of a super-tile, and waits at its start until
  // only those are outstanding).
  auto grab = [&](uint32_t& g, bool dyn) {
    uint64_t sv;
    const uint32_t mask = __builtin_amdgcn_readfirstlane(dyn ? 1u : 0u);
    asm volatile("s_mov_b64 %1, exec\n\ts_mov_b32 exec_lo, %4\n\ts_mov_b32 exec_hi, 0\n\t"
                 "global_atomic_add %0, %2, %5, %3 sc0\n\ts_mov_b64 exec, %1"
                 : "+v"(g), "=&s"(sv)
                 : "v"(ctr_off), "s"(args.counters), "s"(mask), "v"(1u)
                 : "memory");
  };
  // Waits for super-tile k (the copies issued before the last grab) and that grab; returns the
  // index of the wave's super-tile number k + 2: static below NS, else the grabbed value past the
  // static ones, clamped to (nxt, T] so that the loop always advances and every copy address
  // stays inside the sequence. No copies are issued for super-tiles past the end (T): when the
  // next super-tile is one, the wait is for everything outstanding and k + 2 is past the end too
  // (g is not read on that path: the grab of k + 2 was issued with no active lane).
  auto landed = [&](uint32_t& g, int k2, int nxt_tile) {
    if (nxt_tile >= T) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      return T;
    }
    int v;
    asm volatile("s_waitcnt vmcnt(20)\n\tv_readfirstlane_b32 %0, %1" : "=s"(v), "+v"(g) :: "memory");
    const int t = k2 < NS ? gw + k2 * NWS : NS * NWS + v;
    return min(max(t, nxt_tile + 1), T);
  };
  int cur = min(gw, T), nxt = min(gw + NWS, T);  // wave-uniform super-tile indices
  int k = 0;                                      // cur is the wave's super-tile number k
  uint32_t g = 0u;                                // the grab in flight

  // Prologue, copies: q rows, the new K and V rows (fused append) into this wave's terms area
  // (free until the first super-tile is processed), super-tile 0 and the grab of super-tile 2.
  // Only the first three are waited for before the q operands are built; super-tile 1 is issued
  // after them (below).
  {
    const uint32_t stage = lds_addr(&tm);
    const uint16_t* qblk = q + ((int64_t)b * Hq + hk * G) * L * D;  // the R rows, contiguous
    dma_b128<0>(qblk, (uint32_t)min(16 * lane, R * 2 * D - 16), stage);
    if (app) {
      const int64_t src = ((int64_t)b * Hkv + hk) * D;
      dma_b32<1024>(args.knew + src, 4u * (uint32_t)lane, stage);
      dma_b32<1280>(args.vnew + src, 4u * (uint32_t)lane, stage);
    }
    if constexpr (NORM) {  // norm weights behind the new rows, RoPE frequencies beside
      dma_b32<1536>(nargs.qn_w, 4u * (uint32_t)lane, stage);
      dma_b32<1792>(nargs.kn_w, 4u * (uint32_t)lane, stage);
      const int nf = nargs.rot_dims >> 1;  // wave-uniform; without rotation re-read the q weights
      dma_b32<0>(nf ? (const void*)nargs.inv_freq : (const void*)nargs.qn_w,
                 4u * (uint32_t)min(lane, max(nf, 1) - 1), lds_addr(&nsm.inv_freq[wv][0]));
    }
  }
  // The grabs are issued on every path (with no active lane when static or past the end), so
  // that the asm statement that defines g is the same on every path: its result lands in that
  // register after the statement, and a copy the compiler might insert would read it too early.
  if (cur < T) issue(cur, B0);
  grab(g, 2 >= NS && nxt < T);  // super-tile number 2: dynamic when NS == 2
  // the q and new rows have landed (super-tile 0 and the grab issued after them may be in flight)
  if (cur < T)
    asm volatile("s_waitcnt vmcnt(21)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(1)" ::: "memory");
  // ---- B operands of Q.K^T: q[rho] dims 8 s .. 8 s + 7 when this lane group's tile is mt, times
  // the workgroup's power-of-two q factor 2^kq (from the largest |q| element of its R rows). Wave
  // w converts row w (w < R) once for the workgroup into the shared fp16 rows, with the row's two
  // half sums; after a barrier every lane reads its row whole (lanes 4 apart hold all rows), the
  // lanes without an operand the zero row. The barriers wait for LDS only: the copies of
  // super-tile 0 stay in flight.
  const uint32_t* own = reinterpret_cast<const uint32_t*>(&tm);  // q rows 64 words apart
  const int rw = min(wv, R - 1);  // waves past R - 1 redo the last row and store nothing
  uint32_t xq;                    // this lane's pair (dims 2 lane, 2 lane + 1) of row rw
  float amax;                     // the largest |q| element of the R rows, in every lane
  if constexpr (NORM) {
    // Raw q row rw and the new K row -> RMSNorm + RoPE at position n - 1: each wave normalizes
    // and rotates its own staged copies, the two rows together so that their reductions
    // interleave, with the rotation's sin and cos computed once for both. The K row goes back to
    // the wave's copy for the append below; the rows' largest elements go through LDS.
    uint32_t* ownw = reinterpret_cast<uint32_t*>(&tm);
    const RopeLane rl = rope_lane(lane, &nsm.inv_freq[wv][0], nargs.rot_dims, (float)(n - 1));
    uint32_t xr[2] = {own[64 * rw + lane], own[256 + lane]};  // q row rw; K row at byte 1024
    const uint32_t wr[2] = {own[384 + lane], own[448 + lane]};  // norm weights, bytes 1536, 1792
    norm_rope_rows<2>(xr, wr, lane, nargs.norm_eps, rl, nargs.rot_dims, nargs.mscale);
    ownw[256 + lane] = xr[1];
    xq = xr[0];
    const float m = wave_max_valu(fmaxf(fabsf(bf16_lo(xq)), fabsf(bf16_hi(xq))));
    if (lane == 0) qsh.amax[wv] = m;
    lds_barrier();
    amax = qsh.amax[0];
#pragma unroll
    for (int j = 1; j < NWAVE; ++j)
      if (j < R) amax = fmaxf(amax, qsh.amax[j]);
  } else {
    xq = own[64 * rw + lane];
    amax = 0.0f;
#pragma unroll
    for (int j = 0; j < NWAVE; ++j)
      if (j < R) {
        const uint32_t w = own[64 * j + lane];
        amax = fmaxf(amax, fmaxf(fabsf(bf16_lo(w)), fabsf(bf16_hi(w))));
      }
  }
  {
    const int kq = q_pow2_exp(amax);
    const float qf = pow2f(kq);
    kscale = qk_scale_log2 * pow2f(24 - kq);
    if (wv < R) {
      const float lo = bf16_lo(xq), hi = bf16_hi(xq);
      qsh.h[wv][lane] = pack_h2(lo * qf, hi * qf);
      float sg = lo + hi;  // over dims 0-63 (lanes 0-31) and 64-127 (lanes 32-63)
      sg += dpp<DPP_QUAD_XOR1>(sg);
      sg += dpp<DPP_QUAD_XOR2>(sg);
      sg += dpp<DPP_ROW_ROR4>(sg);
      sg += dpp<DPP_ROW_ROR8>(sg);
      sg = sum_xor16(sg);
      if ((lane & 31) == 0) qsh.s[wv][lane >> 5] = sg * qk_scale_log2;
    }
    if (wv == 0) qsh.h[NWAVE][lane] = 0u;
    lds_barrier();
    const bool on = qvalid && mt == lq4;
    const half8_t* qr = reinterpret_cast<const half8_t*>(&qsh.h[on ? rho : NWAVE][0]);
#pragma unroll
    for (int st = 0; st < 16; ++st) qb[st] = qr[st];
    qsum[0] = qvalid ? qsh.s[rho][0] : 0.0f;
    qsum[1] = qvalid ? qsh.s[rho][1] : 0.0f;
  }
  // Super-tile 1 goes out only now, behind every wave's super-tile 0 (~18 MB over the chip at
  // 82,671 keys): issued together, the two landed in the same window, so the loop waited for
  // super-tile 0 until both were nearly in (37.6 -> 36.7 us per fused decode step).
  // The new K and V rows are quantized between its copy groups (the copies issue at the memory
  // pipeline's rate, ~1.2 us for a super-tile's 20 per wave with every wave's super-tile 0 in
  // flight, and the quantization's dependent divisions take ~1 us on their own).
  QPair app_k = {0u, 0, 0}, app_v = {0u, 0, 0};
  uint32_t app_w[4] = {0u, 0u, 0u, 0u};  // ks, kb, vs, vb words of the new row (group 0 low)
  bool patched = false;
  const uint8_t* st8 = reinterpret_cast<const uint8_t*>(&tm);
  auto quantize_new = [&](int j) {
    if (!app) return;
    if (j == 0) app_k = quantize_pair_q8(*reinterpret_cast<const uint32_t*>(st8 + 1024 + 4 * lane));
    if (j == 1) app_v = quantize_pair_q8(*reinterpret_cast<const uint32_t*>(st8 + 1280 + 4 * lane));
    if (j == 2) {
      const uint16_t hv[4] = {app_k.scale, app_k.bias, app_v.scale, app_v.bias};
#pragma unroll
      for (int i = 0; i < 4; ++i)
        app_w[i] = (uint32_t)__builtin_amdgcn_readlane((int)hv[i], 0) |
                   ((uint32_t)__builtin_amdgcn_readlane((int)hv[i], 32) << 16);
    }
    __builtin_amdgcn_sched_barrier(0);  // keeps the work between the copy groups
  };
  if (nxt < T) {
    issue_with(nxt, B1, quantize_new);
  } else {
    quantize_new(0);
    quantize_new(1);
    quantize_new(2);
  }
  // Overwrites row app_r of an LDS super-tile with the new row (same swizzle as the copies:
  // chunk c of row r at chunk position c ^ (r & 7); lane l holds bytes 2l, 2l+1 = chunk l / 8).
  auto patch = [&](auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    PackBuf& pb = sm.loop.buf[wv][BUF];
    const int off = app_r * D + 16 * ((lane >> 3) ^ (app_r & 7)) + 2 * (lane & 7);
    *reinterpret_cast<uint16_t*>(pb.k + off) = (uint16_t)app_k.codes;
    *reinterpret_cast<uint16_t*>(pb.v + off) = (uint16_t)app_v.codes;
    if (lane == 0) {
      pb.ks[app_r] = app_w[0];
      pb.kb[app_r] = app_w[1];
      pb.vs[app_r] = app_w[2];
      pb.vb[app_r] = app_w[3];
    }
  };

  // Unrolled by two so that each buffer's LDS offsets are constants. Step k waits for super-tile
  // k, processes it, then refills its buffer with super-tile k + 2 after the grab of super-tile
  // k + 3; once k + 2 is past the end (the tile counter ran out, so k + 3 would be too) no copies
  // are issued and the grab has no active lane, so the wave's last wait finds nothing else in
  // flight.
  for (;;) {
    if (cur >= T) break;
    int after = landed(g, k + 2, nxt);
    if (cur == app_t) {
      patch(B0);
      patched = true;
    }
    process(cur, B0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer refilled next are done
    grab(g, k + 3 >= NS && after < T);
    if (after < T) issue(after, B0);
    cur = nxt;
    nxt = after;
    ++k;
    if (cur >= T) break;
    after = landed(g, k + 2, nxt);
    if (cur == app_t) {
      patch(B1);
      patched = true;
    }
    process(cur, B1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    grab(g, k + 3 >= NS && after < T);
    if (after < T) issue(after, B1);
    cur = nxt;
    nxt = after;
    ++k;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (patched) {  // the new row goes to the cache (no copy in this kernel reads it back)
    const int64_t crow = row0 + nrow;
    *reinterpret_cast<uint16_t*>(args.kc + crow * D + 2 * lane) = (uint16_t)app_k.codes;
    *reinterpret_cast<uint16_t*>(args.vc + crow * D + 2 * lane) = (uint16_t)app_v.codes;
    if ((lane & 31) == 0) {
      const int64_t w = crow * 2 + (lane >> 5);
      args.ks[w] = app_k.scale;
      args.kb[w] = app_k.bias;
      args.vs[w] = app_v.scale;
      args.vb[w] = app_v.bias;
    }
  }

  float osc[4];  // output factors: 2^24 (codes entered as c 2^-24) over the P.V factors
  vscale_out(vsc, 16777216.0f, 1.0f, osc);
  packed_finish<NWAVE>(oacc, m_run, lsum, bsum0, bsum1, osc,
                       reinterpret_cast<float*>(&sm.loop.buf[0][0]),
                       (int)(2 * sizeof(PackBuf) / sizeof(float)), &sm.st[0][0][0], &sh_last,
                       args, plan, x, b, hk, R);
}

template <bool CAUSAL>
__global__ __launch_bounds__(NTHR) void q8_attn_packed_kernel(AttnArgs args, DecodePlan plan) {
  q8_attn_packed_body<CAUSAL, false>(args, plan, NormArgs{});
}

__global__ __launch_bounds__(NTHR) void q8_attn_norm_kernel(AttnArgs args, DecodePlan plan,
                                                           NormArgs nargs) {
  q8_attn_packed_body<false, true>(args, plan, nargs);
}

}  // namespace

QAttnFn q8_attn_fn(bool causal) {
  return causal ? q8_attn_packed_kernel<true> : q8_attn_packed_kernel<false>;
}

void launch_q8_attn_norm(unsigned S, unsigned Hkv, hipStream_t st, const AttnArgs& a,
                         const DecodePlan& plan, const NormArgs& nargs) {
  q8_attn_norm_kernel<<<dim3(S, Hkv), dim3(NTHR), 0, st>>>(a, plan, nargs);
}

}  // namespace lq
