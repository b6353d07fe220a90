// Attention over the 8-bit KV cache for more than 4 query rows per KV head -- the causal verify
// block of speculative decoding (G * L rows, L <= 16) and single-token decode with G > 4 -- and
// for up to 4 rows over a single sequence of at most 65,536 rows.
//
// Replaces, for verify blocks, the reference's unfused path (dequantize, laguna_mlx/cache.py:
// 99-100, then SDPA with the bottom-right causal mask, laguna.py:107, 183-186), and for decode
// q8_decode_attention (laguna_mlx/q8_attn.py:102-130) when G > 4.
//
// Dense MFMA layout (v_mfma_f32_16x16x32_f16): the 16 columns of an N tile are 16 query rows, so
// NT tiles serve up to 16 NT rows; the 16 rows of an M tile are 16 keys; a super-tile of 64 keys
// is 4 M tiles.
//  * Q.K^T per (M tile mt, quant group g, N tile nt): two MFMAs over the 64 dims of group g. A
//    lane of lane group q supplies dims 64 g + 16 q + 8 e + (0..7) of key 16 mt + (lane % 16) for
//    k-step e (one 16-byte LDS read per (mt, g)); codes enter the MFMA as fp16 subnormals
//    c * 2^-24 (one v_perm_b32 per two codes, exact), 2^24 folded into the K scale.
//  * The affine terms fold out per key and group: q.(s c + b) = s (q.c) + b sum_g(q); the per-key
//    terms (scaled K scale, K bias, V scale, V bias) are computed once per super-tile by one lane
//    per key and shared through LDS.
//  * After Q.K^T a lane holds, per N tile, the scores of keys 16 mt + 4 q + r (r < 4) of one
//    query row; softmax runs in that layout (row max: in-lane over mt and r, then over the 4
//    lane groups), with lazy rescaling and exp2 of scores pre-scaled by scale * log2(e).
//  * P.V: two k-steps of 32 keys (M tiles 2e and 2e+1); A = V^T (16 dims x 32 keys) from one
//    transposed 8-byte LDS read (ds_read_b64_tr_b8), B = P * V scale * 2^kv in fp16 built from the
//    lane's own weights (k-slot j of lane group q = key 16 (2e + j / 4) + 4 q + j % 4).
//  * Work: the waves of a sequence's workgroups take super-tiles gw, gw + NWS, ... (static,
//    interleaved); K, V and the word arrays of a super-tile go global -> LDS with 20 DMA copies,
//    double-buffered per wave, one fixed wait per super-tile.
//  * Fused append (k_new/v_new set): the L new rows n-L .. n-1 of each sequence (one for decode,
//    the verify block's rows for verify) are quantized at the start by the other waves of the
//    workgroup(s) whose wave owns their super-tile (the owner has the sequence's last, extra
//    super-tile and stays off this work), stored to the cache at once and staged in LDS; the
//    owner patches the staged rows into its LDS copy of the super-tile after the copies land (the
//    copies may have read the rows before or while they were stored), once an LDS count says the
//    staging waves are done. No other wave uses those rows. Same arithmetic as
//    quantize_group_kernel, so the codes agree.
//  * Partials (m, l, acc) per (workgroup, query row) go to the workspace. With MERGE (at most 8
//    rows per KV head: decode of one sequence, up to 16 splits x 8 rows x 520 B = 66 KB per head)
//    they are written with agent-scope stores and the last workgroup of (sequence, KV head) to
//    arrive merges them (merge_rows4), as the packed kernels do; otherwise decode_merge_kernel
//    merges them (at 16+ rows per KV head the partials of 32 workgroups are ~330 KB per head, too
//    much for one workgroup to merge at the end of the attention kernel).
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

// ST keys per super-tile: 64 with DW = 4 waves per workgroup, or 32 with DW = 8 (two waves per
// SIMD hide each other's MFMA, LDS and exp latency). Either way one workgroup per CU (about 150 KB
// of LDS: two tile buffers per wave).
template <int ST>
struct DenseBuf {
  uint8_t k[ST * D];
  uint8_t v[ST * D];
  uint32_t ks[ST];
  uint32_t kb[ST];
  uint32_t vs[ST];
  uint32_t vb[ST];
};

template <int ST>
struct DenseTerms {  // per key of the current super-tile
  float ks0[ST], ks1[ST], ku0[ST], ku1[ST];  // s_g * scale*log2e * 2^24, b_g
  float vs0[ST], vs1[ST], vb0[ST], vb1[ST];
};

constexpr int MAX_NEW = 16;  // rows of a fused append (verify L <= 16)
typedef uint32_t v4u32_t __attribute__((ext_vector_type(4)));

template <int NT, int ST, int DW>
struct DenseSmem {
  union {
    struct {
      DenseBuf<ST> buf[DW][2];
      DenseTerms<ST> terms[DW];
    } loop;
    f4_t acc[DW][NT * 8][64];  // wave partials in register layout (epilogue)
  };
  alignas(16) float st[DW][16 * NT][4];  // m, l, bias sum 0, bias sum 1
  alignas(16) float wgt[16 * NT][DW];    // per row: each wave's log-sum-exp weight times 2^24
  float bsw[16 * NT][2];                 // per row: the weighted bias sums of the two groups
  struct {                             // fused append: new row n - L + j, quantized
    uint8_t k[MAX_NEW][D];
    uint8_t v[MAX_NEW][D];
    uint32_t w[MAX_NEW][4];            // K scale, K bias, V scale, V bias words
    int ready;                         // staging waves done
  } stg;
};

// Global -> LDS copy of one dword per lane from a per-lane 64-bit address into lds + 4 lane
// (non-temporal, like the other copies).
__device__ __forceinline__ void dma_b32_v(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
               :: "v"(g), "s"(lds) : "memory");
}

template <int NT, bool CAUSAL, int ST, int DW, bool MERGE>
__global__ __launch_bounds__(64 * DW, 1) void q8_attn_dense_kernel(AttnArgs args, DecodePlan plan) {
  static_assert(ST == 32 || ST == 64, "super-tiles of 32 or 64 keys");
  constexpr int MT = ST / 16;  // M tiles (16 keys) per super-tile
  constexpr int EK = ST / 32;  // P.V k-steps (32 keys) per super-tile
  // copies per super-tile: K and V codes 1 KB each (8 rows), then the word arrays (four of
  // ST dwords; with ST = 32 two copies of 64 lanes, each lane addressing its own array)
  constexpr int NCOPY = ST / 4 + (ST == 64 ? 4 : 2);
  using DenseBuf = lq::DenseBuf<ST>;
  using DenseTerms = lq::DenseTerms<ST>;
  constexpr int DST = ST;
  __shared__ DenseSmem<NT, ST, DW> sm;
  __shared__ int sh_last;
  static_assert(!MERGE || (NT == 1 && DW == 8), "in-kernel merge: one N tile on 8 waves");
  const uint16_t* __restrict__ q = args.q;
  const int Hkv = args.Hkv, G = args.G, L = args.L;
  const int64_t cap = args.cap;
  const float qk_scale_log2 = args.qk_scale_log2;
  LQ_ARG_BATCH("s"(q), "s"(args.kc), "s"(args.vc), "s"(args.ks), "s"(args.kb), "s"(args.vs),
               "s"(args.vb), "s"(args.knew), "s"(args.vnew), "s"(args.pos), "s"(cap), "s"(Hkv),
               "s"(G), "s"(L), "s"(plan.nseq), "s"(plan.split_begin[1]), "s"(plan.len[0]));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  const SeqSplits sq = seq_splits(plan, x);
  const int b = sq.b;
  // rows after the append: the host's length, or (decode from device positions) pos[b] + 1
  const int n = args.pos ? (int)min(max((int64_t)args.pos[b] + 1, (int64_t)1), args.cap)
                         : sq.len;
  const int T = (n + DST - 1) / DST;
  const int NWS = sq.ns * DW;
  const int gw = (x - sq.s0) * DW + wv;
  const int R = G * L;  // query rows of this KV head, <= 16 NT
  const int Hq = Hkv * G;
  const int64_t row0 = ((int64_t)b * Hkv + hk) * cap;
  const int last_row = n - 1;

  const int lc = lane & 15;
  const int lq4 = lane >> 4;

  // B operands of Q.K^T (filled once the first super-tile is in flight): per N tile, group g,
  // k-step e: q[row 16 nt + lc] dims 64 g + 16 lq4 + 8 e + (0..7), fp16; qsum: the group's sum of
  // those fp16 values (all lanes of the column), times scale * log2(e).
  half8_t qb[NT][2][2];
  float qsum[NT][2];
  int qpos[NT];  // position i of the query row in its block (causal bound)

  f4_t oacc[NT][8];  // out^T[16 dt + 4 lq4 + r][row 16 nt + lc]
  float m_run[NT], lsum[NT], bsum[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    m_run[nt] = -INFINITY;
    lsum[nt] = 0.0f;
    bsum[nt][0] = bsum[nt][1] = 0.0f;
  }

  const uint8_t* kbase = args.kc + row0 * D;
  const uint8_t* vbase = args.vc + row0 * D;
  const uint32_t* ksw = reinterpret_cast<const uint32_t*>(args.ks + row0 * 2);
  const uint32_t* kbw = reinterpret_cast<const uint32_t*>(args.kb + row0 * 2);
  const uint32_t* vsw = reinterpret_cast<const uint32_t*>(args.vs + row0 * 2);
  const uint32_t* vbw = reinterpret_cast<const uint32_t*>(args.vb + row0 * 2);
  const int causal_base = n - L;  // query i sees keys t <= causal_base + i
  DenseTerms& tm = sm.loop.terms[wv];

  // ---- fused append: super-tiles ta .. tb (at most two) hold the new rows na .. n-1. Super-tile
  // t belongs to wave t % NWS of the sequence, i.e. to workgroup (t % NWS) / DW; that workgroup
  // stages the rows of its super-tile(s).
  const bool app = args.knew != nullptr;
  const int na = n - L;
  const int ta = na / DST, tb = (n - 1) / DST;
  const int xs = x - sq.s0;
  const bool wg_a = app && (ta % NWS) / DW == xs;
  const bool wg_b = app && tb != ta && (tb % NWS) / DW == xs;
  const int sr0 = wg_a ? na : tb * DST;  // rows staged by this workgroup: [sr0, sr1)
  const int sr1 = wg_b ? n : min(n, (ta + 1) * DST);
  const int wa = wg_a ? ta % NWS - DW * xs : -1;  // owner waves in this workgroup (or -1)
  const int wb = wg_b ? tb % NWS - DW * xs : -1;
  const int nstage = DW - (wa >= 0) - (wb >= 0);  // staging waves: the others (>= 2)
  const int si = wv - (wa >= 0 && wa < wv) - (wb >= 0 && wb < wv);  // this wave's staging rank
  const bool stager = (wg_a || wg_b) && wv != wa && wv != wb;
  if (wg_a || wg_b) {  // workgroup-uniform; before any copy is issued: nothing to wait for
    if (tid == 0) sm.stg.ready = 0;
    __syncthreads();
  }
  // Overwrites the new rows of super-tile `tile` in its LDS copy with the staged ones (same
  // swizzle as the copies: chunk c of row r at chunk position c ^ (r & 7); lane l moves bytes
  // 2l, 2l+1 = chunk l / 8).
  auto patch = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    DenseBuf& pb = sm.loop.buf[wv][BUF];
    const int t0 = tile * DST;
    for (int row = max(t0, na); row < min(t0 + DST, n); ++row) {
      const int j = row - na, r = row - t0;
      const int off = r * D + 16 * ((lane >> 3) ^ (r & 7)) + 2 * (lane & 7);
      const uint16_t kc2 = *reinterpret_cast<const uint16_t*>(&sm.stg.k[j][2 * lane]);
      const uint16_t vc2 = *reinterpret_cast<const uint16_t*>(&sm.stg.v[j][2 * lane]);
      *reinterpret_cast<uint16_t*>(pb.k + off) = kc2;
      *reinterpret_cast<uint16_t*>(pb.v + off) = vc2;
      if (lane < 4) {
        uint32_t* dst = lane == 0 ? pb.ks : lane == 1 ? pb.kb : lane == 2 ? pb.vs : pb.vb;
        dst[r] = sm.stg.w[j][lane];
      }
    }
  };

  // NCOPY copies per super-tile: ST / 8 K + ST / 8 V (1 KB each) + the word arrays. Copy u of lane
  // l moves 16 bytes of row 8 u + l / 8, chunk l % 8 to chunk position (l % 8) ^ (l / 8) of the
  // LDS row. A full super-tile issues its K and V rows in groups of four under one M0 each (the
  // rows 8 apart as immediate offsets, which move the LDS destination with them) at a 32-bit
  // per-lane offset from fixed bases; the last one clamps rows to the sequence's last row and
  // goes copy by copy, and so do super-tiles past the end (their copies land in a buffer that is
  // never read). With ST = 32 the word arrays go two per copy: lanes 0-31 read K scale (V scale)
  // words, lanes 32-63 K bias (V bias) words, into the adjacent ks/kb (vs/vb) arrays of the
  // buffer; with ST = 64 the four arrays go as one group (bases shifted back by their spacing).
  const uint32_t lds_bufs = lds_addr(&sm.loop.buf[wv][0]);
  const uint32_t col_off = (uint32_t)(16 * ((lane & 7) ^ (lane >> 3)));
  const uint32_t ro0 = (uint32_t)((lane >> 3) * D) + col_off;
  const uint32_t* wsel0 = lane < 32 ? ksw : kbw;  // ST = 32: this lane's word arrays
  const uint32_t* wsel1 = lane < 32 ? vsw : vbw;
  constexpr int WSP = ST * 4;  // bytes between the word arrays in LDS
  const uint8_t* kbase4 = kbase + 32 * D;  // ST = 64: rows 32-63 of a super-tile
  const uint8_t* vbase4 = vbase + 32 * D;
  const uint8_t* kbw_s = reinterpret_cast<const uint8_t*>(kbw) - WSP;
  const uint8_t* vsw_s = reinterpret_cast<const uint8_t*>(vsw) - 2 * WSP;
  const uint8_t* vbw_s = reinterpret_cast<const uint8_t*>(vbw) - 3 * WSP;
  auto issue = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * DST;
    const uint32_t lb = lds_bufs + (uint32_t)(BUF * sizeof(DenseBuf));
    constexpr int OK = offsetof(DenseBuf, k), OV = offsetof(DenseBuf, v);
    constexpr int OKS = offsetof(DenseBuf, ks), OKB = offsetof(DenseBuf, kb);
    constexpr int OVS = offsetof(DenseBuf, vs), OVB = offsetof(DenseBuf, vb);
    static_assert(OKB == OKS + WSP && OVS == OKS + 2 * WSP && OVB == OKS + 3 * WSP,
                  "word arrays WSP apart");
    if (t0 + DST <= n) {
      const uint32_t vo = ro0 + (uint32_t)t0 * D;
      dma4_b128<OK, 8 * D>(kbase, vo, lb);
      dma4_b128<OV, 8 * D>(vbase, vo, lb);
      if constexpr (ST == 64) {
        dma4_b128<OK + 32 * D, 8 * D>(kbase4, vo, lb);
        dma4_b128<OV + 32 * D, 8 * D>(vbase4, vo, lb);
        dma4_b32<OKS, WSP>(ksw, kbw_s, vsw_s, vbw_s, 4u * (uint32_t)(t0 + lane), lb);
      } else {
        const int wrow = t0 + (lane & 31);
        dma_b32_v(wsel0 + wrow, lb + OKS);
        dma_b32_v(wsel1 + wrow, lb + OVS);
      }
      return;
    }
    uint32_t ro[ST / 8];
#pragma unroll
    for (int u = 0; u < ST / 8; ++u)
      ro[u] = (uint32_t)min(t0 + (lane >> 3) + 8 * u, last_row) * D + col_off;
    const uint32_t wo = 4u * (uint32_t)min(t0 + lane, last_row);
    const int wrow = min(t0 + (lane & 31), last_row);
    dma_b128<OK + 0>(kbase, ro[0], lb);
    dma_b128<OK + 1024>(kbase, ro[1], lb);
    dma_b128<OK + 2048>(kbase, ro[2], lb);
    dma_b128<OK + 3072>(kbase, ro[3], lb);
    dma_b128<OV + 0>(vbase, ro[0], lb);
    dma_b128<OV + 1024>(vbase, ro[1], lb);
    dma_b128<OV + 2048>(vbase, ro[2], lb);
    dma_b128<OV + 3072>(vbase, ro[3], lb);
    if constexpr (ST == 64) {
      dma_b128<OK + 4096>(kbase, ro[4 % (ST / 8)], lb);
      dma_b128<OK + 5120>(kbase, ro[5 % (ST / 8)], lb);
      dma_b128<OK + 6144>(kbase, ro[6 % (ST / 8)], lb);
      dma_b128<OK + 7168>(kbase, ro[7 % (ST / 8)], lb);
      dma_b128<OV + 4096>(vbase, ro[4 % (ST / 8)], lb);
      dma_b128<OV + 5120>(vbase, ro[5 % (ST / 8)], lb);
      dma_b128<OV + 6144>(vbase, ro[6 % (ST / 8)], lb);
      dma_b128<OV + 7168>(vbase, ro[7 % (ST / 8)], lb);
      dma_b32<OKS>(ksw, wo, lb);
      dma_b32<OKB>(kbw, wo, lb);
      dma_b32<OVS>(vsw, wo, lb);
      dma_b32<OVB>(vbw, wo, lb);
    } else {
      dma_b32_v(wsel0 + wrow, lb + OKS);
      dma_b32_v(wsel1 + wrow, lb + OVS);
    }
  };

  // Per-key K factor: scale * log2(e) * 2^24 (codes enter the MFMA as c * 2^-24) / 2^kq (the q
  // operands' power-of-two factor, set with them below).
  float kscale = qk_scale_log2 * 16777216.0f;
  VScale vsc;  // P.V factors 2^kv of the two quant groups (set by the first tile)

  auto process = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * DST;
    const DenseBuf& pb = sm.loop.buf[wv][BUF];
    // per-key terms, one lane per key (V scales scaled by the wave's P.V factors; |scale_v| of
    // valid keys kept for their check)
    const bool kl = ST == 64 || lane < ST;
    float sv0, sv1, va0, va1;
    {
      const int kk = kl ? lane : 0;
      const uint32_t a = pb.ks[kk], c = pb.kb[kk], e = pb.vs[kk], f = pb.vb[kk];
      sv0 = bf16_lo(e);
      sv1 = bf16_hi(e);
      const bool kv = kl && t0 + lane < n;  // rows past n are clamped copies, never attended
      va0 = kv ? fabsf(sv0) : 0.0f;
      va1 = kv ? fabsf(sv1) : 0.0f;
      if (kl) {
        tm.ks0[lane] = bf16_lo(a) * kscale;
        tm.ks1[lane] = bf16_hi(a) * kscale;
        tm.ku0[lane] = bf16_lo(c);
        tm.ku1[lane] = bf16_hi(c);
        tm.vs0[lane] = sv0 * vsc.f0;
        tm.vs1[lane] = sv1 * vsc.f1;
        tm.vb0[lane] = bf16_lo(f);
        tm.vb1[lane] = bf16_hi(f);
      }
    }
    // Q.K^T: c[mt][nt][g]
    f4_t c[MT][NT][2];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int r = 16 * mt + lc;
      const uint8_t* kr = pb.k + r * D;
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const uint4 u = *reinterpret_cast<const uint4*>(kr + 16 * ((4 * g + lq4) ^ (r & 7)));
        const half8_t a0 = codes8_sub(u.x, u.y);
        const half8_t a1 = codes8_sub(u.z, u.w);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f4_t z = {0.f, 0.f, 0.f, 0.f};
          z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qb[nt][g][0], z, 0, 0, 0);
          z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qb[nt][g][1], z, 0, 0, 0);
          c[mt][nt][g] = z;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const bool vnew = vscale_check(va0, va1, vsc);  // new P.V factors: applied with N tile 0
    const bool full = t0 + DST <= n && (!CAUSAL || t0 + DST - 1 <= causal_base);
    // scores of this lane's keys 16 mt + 4 lq4 + r, per N tile (per-key terms read per M tile)
    float sc[NT][MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int k0 = 16 * mt + 4 * lq4;
      const float4 s0 = *reinterpret_cast<const float4*>(tm.ks0 + k0);
      const float4 s1 = *reinterpret_cast<const float4*>(tm.ks1 + k0);
      const float4 u0 = *reinterpret_cast<const float4*>(tm.ku0 + k0);
      const float4 u1 = *reinterpret_cast<const float4*>(tm.ku1 + k0);
      const float s0v[4] = {s0.x, s0.y, s0.z, s0.w}, s1v[4] = {s1.x, s1.y, s1.z, s1.w};
      const float u0v[4] = {u0.x, u0.y, u0.z, u0.w}, u1v[4] = {u1.x, u1.y, u1.z, u1.w};
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          sc[nt][mt][r] = fmaf(s0v[r], c[mt][nt][0][r],
                               fmaf(s1v[r], c[mt][nt][1][r],
                                    fmaf(u1v[r], qsum[nt][1], u0v[r] * qsum[nt][0])));
    }
    if (!full) {  // keys past the sequence or the row's causal bound (the last super-tiles only)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int lim = CAUSAL ? causal_base + qpos[nt] : n - 1;  // <= n - 1
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            sc[nt][mt][r] = t0 + 16 * mt + 4 * lq4 + r <= lim ? sc[nt][mt][r] : -INFINITY;
      }
    }
    uint32_t pw[NT][EK][2][4];  // P.V B operands: [nt][k-step e][group][dword]
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, sc[nt][mt][r]);
      tmax = max_xor16(tmax);
      tmax = max_xor32(tmax);
      const bool bump = tmax > m_run[nt] + RESCALE_LOG2;
      const uint64_t bumps = __builtin_amdgcn_ballot_w64(bump);
      const bool vn = nt == 0 && vnew;
      if (bumps || vn) {  // rare: a new running max, or new P.V factors
        if (bumps) {
          const float mn = bump ? tmax : m_run[nt];
          const float alpha = m_run[nt] == -INFINITY ? 0.0f : exp2_nonpos(m_run[nt] - mn);
          // while no lane has seen a key of these rows the sums are all zero
          if (__builtin_amdgcn_ballot_w64(m_run[nt] != -INFINITY)) {
            lsum[nt] *= alpha;
            bsum[nt][0] *= alpha;
            bsum[nt][1] *= alpha;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] *= alpha;
          }
          m_run[nt] = mn;
        }
        if (vn) {  // every N tile's accumulators; the V terms read below are rewritten
          vscale_apply<NT>(va0, va1, vsc, &oacc[0][0]);
          if (kl) {
            tm.vs0[lane] = sv0 * vsc.f0;
            tm.vs1[lane] = sv1 * vsc.f1;
          }
          __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
          __builtin_amdgcn_wave_barrier();
          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
      }
      const float mref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      float ls = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
      for (int e = 0; e < EK; ++e) {
        float w0[8], w1[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int mt = 2 * e + h;
          const int k0 = 16 * mt + 4 * lq4;
          const float4 vs0 = *reinterpret_cast<const float4*>(tm.vs0 + k0);
          const float4 vs1 = *reinterpret_cast<const float4*>(tm.vs1 + k0);
          const float4 vb0 = *reinterpret_cast<const float4*>(tm.vb0 + k0);
          const float4 vb1 = *reinterpret_cast<const float4*>(tm.vb1 + k0);
          const float vs0v[4] = {vs0.x, vs0.y, vs0.z, vs0.w};
          const float vs1v[4] = {vs1.x, vs1.y, vs1.z, vs1.w};
          const float vb0v[4] = {vb0.x, vb0.y, vb0.z, vb0.w};
          const float vb1v[4] = {vb1.x, vb1.y, vb1.z, vb1.w};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float p = __builtin_amdgcn_exp2f(sc[nt][mt][r] - mref);
            ls += p;
            b0 = fmaf(p, vb0v[r], b0);
            b1 = fmaf(p, vb1v[r], b1);
            w0[4 * h + r] = p * vs0v[r];
            w1[4 * h + r] = p * vs1v[r];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          pw[nt][e][0][j] = pack_h2(w0[2 * j], w0[2 * j + 1]);
          pw[nt][e][1][j] = pack_h2(w1[2 * j], w1[2 * j + 1]);
        }
      }
      lsum[nt] += ls;
      bsum[nt][0] += b0;
      bsum[nt][1] += b1;
    }
    // P.V: A = V^T tile (16 dims x 32 keys) via one transposed LDS read per dim tile. Source
    // lane s of each 16-lane group addresses key T[s/2] at column offset 8 (s % 2), so result
    // lane i receives keys T[0..7] of dim i.
#pragma unroll
    for (int e = 0; e < EK; ++e) {
      const int kslot = lc >> 1;
      const int key = 32 * e + (kslot < 4 ? 4 * lq4 + kslot : 16 + 4 * lq4 + (kslot - 4));
      const uint8_t* vrow = pb.v + key * D + 8 * (lc & 1);
      const int sw = key & 7;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const v2i_t raw =
            __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)(vrow + 16 * (dt ^ sw)));
        const half8_t a = codes8_sub((uint32_t)raw.x, (uint32_t)raw.y);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const uint32_t* w = pw[nt][e][dt >> 2];
          const half8_t bw = words_as_h8(w[0], w[1], w[2], w[3]);
          oacc[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bw, oacc[nt][dt], 0, 0, 0);
        }
      }
    }
  };

  const std::integral_constant<int, 0> B0;
  const std::integral_constant<int, 1> B1;
  // Unrolled by two so that each buffer's LDS offsets are constants. The next super-tile is
  // issued before the current one is processed, so the wait is a fixed count (the copies issued
  // after it), except at the end, where nothing past the last super-tile is issued.
  int cur = min(gw, T);
  // Prologue: the R q rows (contiguous, R * 256 <= 16 KB) go by DMA into this wave's second
  // buffer, free until super-tile 1 is issued; then the staging waves' new rows (plain loads)
  // and super-tile 0. Only the q copies and the new rows are waited for before the q operands
  // are built; super-tile 0 streams in meanwhile.
  {
    const uint16_t* qblk = q + ((int64_t)b * Hq + hk * G) * L * D;
    const int qbytes = R * 2 * D;
    const uint32_t qlds = lds_bufs + (uint32_t)sizeof(DenseBuf);
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (1024 * i < qbytes)  // wave-uniform
        dma_b128<0>(qblk, (uint32_t)min(1024 * i + 16 * lane, qbytes - 16), qlds + 1024 * i);
  }
  // staging wave: the new rows sr0 + si + nstage i (at most 8 with L <= 16), loads issued
  // together with q's. They are inline asm, in the staging waves only, so that the compiler
  // inserts no wait of its own for them: its count
  // would not include the asm copies of super-tile 0 issued after them, and its wait before the
  // first use waited for those too, i.e. the staged rows were quantized only once super-tile 0
  // had landed. The explicit wait below covers them (they are older than super-tile 0's copies),
  // and the empty statement after it takes them as in-out operands, so no use moves above it.
  uint32_t kraw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u}, vraw[8] = {0u, 0u, 0u, 0u, 0u, 0u, 0u, 0u};
  if (stager) {  // wave-uniform; a staging wave reads rows past sr1 as row sr1 - 1, unused
    const int64_t hrow = ((int64_t)b * Hkv + hk) * L - na;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = min(sr0 + si + nstage * i, sr1 - 1);
      const int64_t src = (hrow + row) * D + 2 * lane;
      asm volatile("global_load_dword %0, %1, off"
                   : "+v"(kraw[i]) : "v"(args.knew + src) : "memory");
      asm volatile("global_load_dword %0, %1, off"
                   : "+v"(vraw[i]) : "v"(args.vnew + src) : "memory");
    }
  }
  if (cur < T) issue(cur, B0);
  if (cur < T) {  // the q copies and the new rows have landed
    if constexpr (NCOPY == 20)
      asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }
  asm volatile("" : "+v"(kraw[0]), "+v"(kraw[1]), "+v"(kraw[2]), "+v"(kraw[3]), "+v"(kraw[4]),
               "+v"(kraw[5]), "+v"(kraw[6]), "+v"(kraw[7]), "+v"(vraw[0]), "+v"(vraw[1]),
               "+v"(vraw[2]), "+v"(vraw[3]), "+v"(vraw[4]), "+v"(vraw[5]), "+v"(vraw[6]),
               "+v"(vraw[7]));

  // q operands: one power-of-two factor for all rows of the wave (the largest |q| element of any
  // row in [2^14, 2^15) before the fp16 conversion); 2^-kq goes into kscale
  {
    uint32_t qwd[NT][2][8];
    uint32_t mbits = 0u;
    const uint8_t* qstage = reinterpret_cast<const uint8_t*>(&sm.loop.buf[wv][1]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int qr_i = 16 * nt + lc;
      const bool valid = qr_i < R;
      const int gh = valid ? qr_i / L : 0;
      const int i = valid ? qr_i - gh * L : 0;
      qpos[nt] = i;
      const uint8_t* qr = qstage + (gh * L + i) * 2 * D;  // row gh * L + i of the block
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const uint4 u = *reinterpret_cast<const uint4*>(qr + 2 * (64 * g + 16 * lq4));
        const uint4 v = *reinterpret_cast<const uint4*>(qr + 2 * (64 * g + 16 * lq4 + 8));
        const uint32_t w[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          qwd[nt][g][j] = valid ? w[j] : 0u;
          mbits = bf16x2_absmax_bits(mbits, qwd[nt][g][j]);
          s += bf16_lo(qwd[nt][g][j]) + bf16_hi(qwd[nt][g][j]);
        }
        qsum[nt][g] = sum_xor32(sum_xor16(s)) * qk_scale_log2;
      }
    }
    const int kq = q_pow2_exp(bf16x2_max_value(mbits));
    const float qf = pow2f(kq);
    kscale = qk_scale_log2 * pow2f(24 - kq);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const uint32_t wd = qwd[nt][g][4 * e + j];
            qb[nt][g][e][2 * j] = (_Float16)(bf16_lo(wd) * qf);
            qb[nt][g][e][2 * j + 1] = (_Float16)(bf16_hi(wd) * qf);
          }
  }

  if (stager) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int row = sr0 + si + nstage * i;
      if (row < sr1) {  // wave-uniform
        const int j = row - na;
        const int64_t crow = row0 + row;
        const QPair kq = quantize_pair_q8(kraw[i]);
        const QPair vq = quantize_pair_q8(vraw[i]);
        *reinterpret_cast<uint16_t*>(&sm.stg.k[j][2 * lane]) = (uint16_t)kq.codes;
        *reinterpret_cast<uint16_t*>(&sm.stg.v[j][2 * lane]) = (uint16_t)vq.codes;
        *reinterpret_cast<uint16_t*>(args.kc + crow * D + 2 * lane) = (uint16_t)kq.codes;
        *reinterpret_cast<uint16_t*>(args.vc + crow * D + 2 * lane) = (uint16_t)vq.codes;
        const uint16_t hv[4] = {kq.scale, kq.bias, vq.scale, vq.bias};
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const uint32_t word = (uint32_t)__builtin_amdgcn_readlane((int)hv[f], 0) |
                                ((uint32_t)__builtin_amdgcn_readlane((int)hv[f], 32) << 16);
          if (lane == f) {
            sm.stg.w[j][f] = word;
            uint16_t* dst = f == 0 ? args.ks : f == 1 ? args.kb : f == 2 ? args.vs : args.vb;
            reinterpret_cast<uint32_t*>(dst)[crow] = word;
          }
        }
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the staged rows are in LDS
    if (lane == 0)
      __hip_atomic_fetch_add(&sm.stg.ready, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  // Waits for the super-tile in process order: until only the NCOPY copies of the super-tile
  // issued after it are outstanding, or until nothing is when that one was past the end (not
  // issued).
  auto wait_tile = [&](bool next_issued) {
    if (!next_issued)
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if constexpr (NCOPY == 20)
      asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(10)" ::: "memory");
  };
  // The owner waits (bounded) for the staging waves before its first patch; they finish within
  // microseconds of the start, long before the owner reaches its last super-tiles.
  auto staged = [&]() {
    for (int spin = 0; spin < (1 << 22); ++spin) {
      const int done =
          __hip_atomic_load(&sm.stg.ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (done >= nstage) break;
      __builtin_amdgcn_s_sleep(2);
    }
  };
  for (;;) {
    if (cur >= T) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer reused next are done
    int nx = min(cur + NWS, T);
    if (nx < T) issue(nx, B1);
    wait_tile(nx < T);  // super-tile cur has landed in LDS
    if (app && (cur == ta || cur == tb)) {
      staged();
      patch(cur, B0);
    }
    process(cur, B0);
    cur = nx;
    if (cur >= T) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    nx = min(cur + NWS, T);
    if (nx < T) issue(nx, B0);
    wait_tile(nx < T);
    if (app && (cur == ta || cur == tb)) {
      staged();
      patch(cur, B1);
    }
    process(cur, B1);
    cur = nx;
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  vscale_remove<NT>(vsc, &oacc[0][0]);

  // ---- per-wave totals over the 4 lane groups that share a column
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    lsum[nt] = sum_xor32(sum_xor16(lsum[nt]));
    bsum[nt][0] = sum_xor32(sum_xor16(bsum[nt][0]));
    bsum[nt][1] = sum_xor32(sum_xor16(bsum[nt][1]));
  }
  // Wave partials go to LDS as the registers hold them (lane-contiguous 16-byte writes, no bank
  // conflicts), each wave into its own two tile buffers, which are free once its loop has ended
  // (its copies have all landed: vmcnt 0 above), so no barrier comes first and the waves that
  // end early write while the others finish: accw(w)[8 nt + dt][lane] = oacc[nt][dt] of wave w.
  static_assert(sizeof(sm.loop.buf[0]) >= sizeof(f4_t) * NT * 8 * 64, "wave partial too large");
  auto accw = [&](int w) { return reinterpret_cast<f4_t(*)[64]>(&sm.loop.buf[w][0]); };
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) accw(wv)[8 * nt + dt][lane] = oacc[nt][dt];
    if (lq4 == 0)
      *reinterpret_cast<float4*>(sm.st[wv][nt * 16 + lc]) =
          make_float4(m_run[nt], lsum[nt], bsum[nt][0], bsum[nt][1]);
  }
  __syncthreads();

  // ---- merge the waves (log-sum-exp) into the workgroup's partial: per row the waves' weights
  // against the row's largest m (times 2^24: codes entered as c 2^-24), the weighted bias sums
  // and the row's (M, l); per item (8 nt + dt, lane), dims 16 dt + 4 (lane / 16) + (0..3) of
  // query row 16 nt + lane % 16: bias sum + the weighted sum of the waves' accumulators.
  if constexpr (MERGE) {
    // One item per thread (one N tile on 8 waves: dt = wave), which computes its row's weights
    // itself (DW exp2), so that no second barrier and no serial per-row step come before the
    // sums; agent-scope partial stores, 16 bytes per item.
    const int col = lane & 15;
    if (col < R) {
      float4 stw[DW];
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        stw[w] = *reinterpret_cast<const float4*>(sm.st[w][col]);
        M = max_ieee(M, stw[w].x);
      }
      float ew[DW], bias = 0.0f;
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        ew[w] = stw[w].x == -INFINITY ? 0.0f : exp2_nonpos(stw[w].x - M);
        bias = fmaf(ew[w], wv < 4 ? stw[w].z : stw[w].w, bias);
      }
      f4_t a = {bias, bias, bias, bias};
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const f4_t v = accw(w)[wv][lane];
        const float wg = ew[w] * 16777216.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = fmaf(wg, v[r], a[r]);
      }
      const int64_t prow = (int64_t)x * Hkv * R + (int64_t)hk * R + col;
      const __amdgpu_buffer_rsrc_t rsrc =
          __builtin_amdgcn_make_buffer_rsrc(args.part_acc, 0, 0x7fffffff, 0x00020000);
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(v4u32_t, a), rsrc,
          (int)((prow * D + 16 * wv + 4 * lq4) * (int64_t)sizeof(float)), 0, 16);  // sc1
      if (tid < R) {  // wave 0, lane = row
        float l = 0.0f;
#pragma unroll
        for (int w = 0; w < DW; ++w) l += ew[w] * stw[w].y;
        st_agent2(reinterpret_cast<float*>(args.part_ml + prow), M, l);
      }
    }
  } else {
    if (tid < R) {
      const int col = tid;
      float M = -INFINITY;
#pragma unroll
      for (int w = 0; w < DW; ++w) M = max_ieee(M, sm.st[w][col][0]);
      float l = 0.0f, b0 = 0.0f, b1 = 0.0f;
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const float* st = sm.st[w][col];
        const float e = st[0] == -INFINITY ? 0.0f : exp2_nonpos(st[0] - M);
        sm.wgt[col][w] = e * 16777216.0f;
        l += e * st[1];
        b0 = fmaf(e, st[2], b0);
        b1 = fmaf(e, st[3], b1);
      }
      sm.bsw[col][0] = b0;
      sm.bsw[col][1] = b1;
      args.part_ml[(int64_t)x * Hkv * R + (int64_t)hk * R + col] = make_float2(M, l);
    }
    __syncthreads();
    for (int it = tid; it < NT * 8 * 64; it += 64 * DW) {
      const int reg = it >> 6, ln = it & 63;
      const int col = 16 * (reg >> 3) + (ln & 15);
      if (col >= R) continue;
      const int dt = reg & 7;
      float wg[DW];
#pragma unroll
      for (int w = 0; w < DW; w += 4) {
        const float4 q4 = *reinterpret_cast<const float4*>(&sm.wgt[col][w]);
        wg[w] = q4.x;
        wg[w + 1] = q4.y;
        wg[w + 2] = q4.z;
        wg[w + 3] = q4.w;
      }
      const float bias = sm.bsw[col][dt >> 2];
      f4_t a = {bias, bias, bias, bias};
#pragma unroll
      for (int w = 0; w < DW; ++w) {
        const f4_t v = accw(w)[reg][ln];
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = fmaf(wg[w], v[r], a[r]);
      }
      const int d0 = 16 * dt + 4 * (ln >> 4);
      *reinterpret_cast<f4_t*>(args.part_acc + ((int64_t)x * Hkv * R + (int64_t)hk * R + col) * D + d0) = a;
    }
  }
  if constexpr (MERGE) {
    // Every thread's partial stores have completed (vmcnt 0) before the barrier in front of the
    // arrival count; the last workgroup of (sequence, KV head) merges all splits (agent-scope
    // loads issued after its count returned) and resets the counter for the next call.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
      uint32_t* c = arrival_counter(args.counters, b * Hkv + hk);
      const uint32_t ns = (uint32_t)sq.ns;
      const uint32_t prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int last = prev + 1 == ns;
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh_last = last;
    }
    __syncthreads();
    if (!sh_last) return;
    float* red = reinterpret_cast<float*>(&sm.acc[0][0][0]);  // free: the wave partials are read
    if (R <= 4)
      merge_rows4<DW, 4>(b, hk, Hkv, R, plan, args.part_acc, args.part_ml, args.out, red);
    else
      merge_rows4<DW, 8>(b, hk, Hkv, R, plan, args.part_acc, args.part_ml, args.out, red);
  }
}

}  // namespace

// Up to 32 query rows per KV head: 32-key super-tiles on 8 waves. More rows: 64-key super-tiles
// on 4 waves (their accumulators leave no registers for a second wave per SIMD). merge: the
// in-kernel split merge (decode, at most 8 rows per KV head).
QAttnFn q8_dense_attn_fn(int nt, bool causal, bool merge) {
  if (merge) return nt == 1 && !causal ? q8_attn_dense_kernel<1, false, 32, 8, true> : nullptr;
  if (causal) {
    switch (nt) {
      case 1: return q8_attn_dense_kernel<1, true, 32, 8, false>;
      case 2: return q8_attn_dense_kernel<2, true, 32, 8, false>;
      case 3: return q8_attn_dense_kernel<3, true, 64, 4, false>;
      case 4: return q8_attn_dense_kernel<4, true, 64, 4, false>;
    }
  } else {
    switch (nt) {
      case 1: return q8_attn_dense_kernel<1, false, 32, 8, false>;
      case 2: return q8_attn_dense_kernel<2, false, 32, 8, false>;
      case 3: return q8_attn_dense_kernel<3, false, 64, 4, false>;
      case 4: return q8_attn_dense_kernel<4, false, 64, 4, false>;
    }
  }
  return nullptr;
}

int q8_dense_threads(int nt) { return nt <= 2 ? 512 : 256; }

}  // namespace lq
