// Single-token decode attention over a plain bf16 KV cache (the bandwidth reference of the
// quantized paths; the reference's plain cache + SDPA, laguna_mlx/laguna.py:107, 209-214,
// scripts/micro_kv_decode.py:41).
//
// Same plan and structure as the packed 8-bit kernel (qattn.hip), with what bf16 changes:
//  * Two waves per workgroup: a 64-key super-tile of bf16 K and V is 32 KB, double-buffered per
//    wave, so two waves fill the LDS (128 KB).
//  * K rows are the Q.K^T A operand as they are (v_mfma_f32_16x16x32_bf16, q in bf16 is exact);
//    the 16-byte chunk c of row r sits at chunk position c ^ (r & 15).
//  * V^T comes from the LDS tile with ds_read_b64_tr_b16: four source lanes per key row (16
//    dims) give every lane one dim of four keys, two reads make an 8-key A operand.
//  * P enters the bf16 MFMA as a high and a low bf16 part (p = hi + lo to ~16 bits), two MFMAs
//    per operand, so the weights keep fp16-like precision.
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

constexpr int BW = 2;          // waves per workgroup
constexpr int BTHR = 64 * BW;
constexpr int BPST = 64;       // keys per super-tile
constexpr int BROW = D * 2;    // bytes per bf16 row

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

struct Bf16Buf {
  uint8_t k[BPST * BROW];
  uint8_t v[BPST * BROW];
};

struct Bf16Smem {
  Bf16Buf buf[BW][2];  // a wave's two also hold its partial rows after its loop
  alignas(16) float st[BW][4][6];
  alignas(16) uint8_t qstage[BW][4 * D * 2];  // each wave's copy of the (<= 4) q rows
};

__device__ __forceinline__ bf16x8_t u4_as_bf8(uint4 u) { return __builtin_bit_cast(bf16x8_t, u); }
__device__ __forceinline__ uint32_t bf16_bits(float x) { return (uint32_t)f32_to_bf16(x); }

template <bool CAUSAL>
__global__ __launch_bounds__(BTHR) void bf16_attn_packed_kernel(AttnArgs args, DecodePlan plan) {
  __shared__ Bf16Smem sm;
  __shared__ int sh_last;

  const uint16_t* __restrict__ q = args.q;
  const uint8_t* __restrict__ kc = args.kc;
  const uint8_t* __restrict__ vc = args.vc;
  const int Hkv = args.Hkv, G = args.G, L = args.L;
  const int64_t cap = args.cap;
  const float qk_scale_log2 = args.qk_scale_log2;
  LQ_ARG_BATCH("s"(q), "s"(kc), "s"(vc), "s"(cap), "s"(Hkv), "s"(G), "s"(L), "s"(plan.nseq),
               "s"(plan.chunk), "s"(plan.split_begin[1]), "s"(plan.len[0]));

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
  const int sub = (c_end - c_begin + BW - 1) / BW;
  const int w_begin = min(c_begin + wv * sub, c_end);
  const int w_end = min(w_begin + sub, c_end);
  const int nst = (w_end - w_begin + BPST - 1) / BPST;
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

  bf16x8_t qb[16];
  f4_t oacc[8];
  float m_run = -INFINITY, lsum = 0.f;
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) oacc[dt] = f4_t{0.f, 0.f, 0.f, 0.f};

  const uint8_t* kbase = kc + row0 * BROW;
  const uint8_t* vbase = vc + row0 * BROW;

  // 32 copies per super-tile: copy u of lane l moves 16 bytes of row 4u + l / 16, chunk
  // (l % 16) ^ (row & 15), to chunk position l % 16 of that LDS row.
  const uint32_t lds_bufs = lds_addr(&sm.buf[wv][0]);
  uint32_t row_off[16];
#pragma unroll
  for (int u = 0; u < 16; ++u) {
    const int r = 4 * u + (lane >> 4);
    row_off[u] = (uint32_t)(r * BROW + 16 * ((lane & 15) ^ (r & 15)));
  }
  auto issue = [&](int si, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    constexpr int OK = offsetof(Bf16Buf, k), OV = offsetof(Bf16Buf, v);
    const int t0 = w_begin + si * BPST;
    const uint32_t lb = lds_bufs + (uint32_t)(BUF * sizeof(Bf16Buf));
    const uint8_t* kb0 = kbase;
    const uint8_t* vb0 = vbase;
    uint32_t ro[16];
    if (t0 + BPST <= w_end) {
      kb0 += (int64_t)t0 * BROW;
      vb0 += (int64_t)t0 * BROW;
#pragma unroll
      for (int u = 0; u < 16; ++u) ro[u] = row_off[u];
    } else {
      const int last = max(w_end - 1, 0);
#pragma unroll
      for (int u = 0; u < 16; ++u) {
        const int r = 4 * u + (lane >> 4);
        ro[u] = (uint32_t)min(t0 + r, last) * BROW + 16 * ((lane & 15) ^ (r & 15));
      }
    }
#define LQ_BF16_COPY(u)                          \
    dma_b128<OK + 1024 * (u)>(kb0, ro[u], lb);   \
    dma_b128<OV + 1024 * (u)>(vb0, ro[u], lb);
    LQ_BF16_COPY(0) LQ_BF16_COPY(1) LQ_BF16_COPY(2) LQ_BF16_COPY(3)
    LQ_BF16_COPY(4) LQ_BF16_COPY(5) LQ_BF16_COPY(6) LQ_BF16_COPY(7)
    LQ_BF16_COPY(8) LQ_BF16_COPY(9) LQ_BF16_COPY(10) LQ_BF16_COPY(11)
    LQ_BF16_COPY(12) LQ_BF16_COPY(13) LQ_BF16_COPY(14) LQ_BF16_COPY(15)
#undef LQ_BF16_COPY
  };

  // P.V B-operand halves: key tile 2e in slots 0-3, 2e+1 in slots 4-7 (this lane's tile is mt)
  const uint32_t sel_lo0 = mt == 0 ? ~0u : 0u, sel_hi0 = mt == 1 ? ~0u : 0u;
  const uint32_t sel_lo1 = mt == 2 ? ~0u : 0u, sel_hi1 = mt == 3 ? ~0u : 0u;
  // V^T reads: source lane lc of group lq4 addresses key 4 lq4 + lc / 4 of a key tile, dims
  // 16 dt + 4 (lc % 4) .. + 3 (chunk 2 dt + (lc % 4) / 2, half lc % 2 of it)
  const int vkey = 4 * lq4 + (lc >> 2);
  const int vsw = vkey & 15;

  auto process = [&](int si, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = w_begin + si * BPST;
    const Bf16Buf& pb = sm.buf[wv][BUF];
    // Q.K^T: A = key row lc of tile lq4, 16 steps of 8 dims, two independent chains
    f4_t c0 = {0.f, 0.f, 0.f, 0.f}, c1 = {0.f, 0.f, 0.f, 0.f};
    {
      const int r = 16 * lq4 + lc;
      const uint8_t* kr = pb.k + r * BROW;
#pragma unroll
      for (int s = 0; s < 16; s += 2) {
        const uint4 a = *reinterpret_cast<const uint4*>(kr + 16 * (s ^ (r & 15)));
        const uint4 a2 = *reinterpret_cast<const uint4*>(kr + 16 * ((s + 1) ^ (r & 15)));
        c0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(u4_as_bf8(a), qb[s], c0, 0, 0, 0);
        c1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(u4_as_bf8(a2), qb[s + 1], c1, 0, 0, 0);
      }
    }
    const int k0 = 16 * mt + 4 * lq4;
    float sc[4];
    float tmax = -INFINITY;
    const bool full = t0 + BPST <= w_end && (!CAUSAL || t0 + BPST - 1 <= n - L);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = (c0[r] + c1[r]) * qk_scale_log2;
      if (!full) {
        const int t = t0 + k0 + r;
        bool ok = t < w_end;
        if (CAUSAL) ok = ok && t <= causal_bound;
        v = ok ? v : -INFINITY;
      }
      sc[r] = v;
      tmax = fmaxf(tmax, v);
    }
    tmax = max_ieee(tmax, dpp<DPP_ROW_ROR4>(tmax));
    tmax = max_ieee(tmax, dpp<DPP_ROW_ROR8>(tmax));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    const bool bump = tmax > m_run + RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(bump)) {
      const float mn = bump ? tmax : m_run;
      const float alpha = m_run == -INFINITY ? 0.0f : exp2_nonpos(m_run - mn);
      // while no lane has seen a key (the wave's first super-tile) the sums are all zero
      if (__builtin_amdgcn_ballot_w64(m_run != -INFINITY)) {
        lsum *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
      }
      m_run = mn;
    }
    const float mref = m_run == -INFINITY ? 0.0f : m_run;
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float p = __builtin_amdgcn_exp2f(sc[r] - mref);
      lsum += p;
      ph[r] = bf16_bits(p);
      pl[r] = bf16_bits(p - __uint_as_float(ph[r] << 16));
    }
    const uint32_t h01 = ph[0] | (ph[1] << 16), h23 = ph[2] | (ph[3] << 16);
    const uint32_t l01 = pl[0] | (pl[1] << 16), l23 = pl[2] | (pl[3] << 16);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t slo = e == 0 ? sel_lo0 : sel_lo1, shi = e == 0 ? sel_hi0 : sel_hi1;
      const bf16x8_t bh = u4_as_bf8(make_uint4(h01 & slo, h23 & slo, h01 & shi, h23 & shi));
      const bf16x8_t bl = u4_as_bf8(make_uint4(l01 & slo, l23 & slo, l01 & shi, l23 & shi));
      const uint8_t* v0 = pb.v + (32 * e + vkey) * BROW + 8 * (lc & 1);
      const uint8_t* v1 = v0 + 16 * BROW;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const int cpos = 16 * ((2 * dt + ((lc & 3) >> 1)) ^ vsw);
        const v4s_t r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t*)(v0 + cpos));
        const v4s_t r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t*)(v1 + cpos));
        const uint4 au = make_uint4(__builtin_bit_cast(uint2, r0).x, __builtin_bit_cast(uint2, r0).y,
                                    __builtin_bit_cast(uint2, r1).x, __builtin_bit_cast(uint2, r1).y);
        const bf16x8_t a = u4_as_bf8(au);
        oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, oacc[dt], 0, 0, 0);
        oacc[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, oacc[dt], 0, 0, 0);
      }
    }
  };

  const std::integral_constant<int, 0> B0;
  const std::integral_constant<int, 1> B1;
  // Prologue: the R q rows (contiguous, <= 1 KB) by DMA into this wave's staging area, then
  // super-tile 0; only the q copy is waited for before the q operands are built. Nothing is
  // issued for super-tiles past the wave's range.
  {
    const uint16_t* qblk = q + ((int64_t)b * Hq + hk * G) * L * D;
    dma_b128<0>(qblk, (uint32_t)min(16 * lane, R * 2 * D - 16), lds_addr(&sm.qstage[wv][0]));
  }
  if (nst > 0) issue(0, B0);
  if (nst > 0)
    asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
  else
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // q as block-diagonal bf16 B operands: q[rho] dims 8 s .. 8 s + 7 when lane group lq4 == mt
  {
    const bool on = qvalid && mt == lq4;
    const uint8_t* qr = &sm.qstage[wv][0] + (gh * L + qi) * 2 * D;
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      const uint4 u = *reinterpret_cast<const uint4*>(qr + 16 * s);
      qb[s] = u4_as_bf8(on ? u : make_uint4(0u, 0u, 0u, 0u));
    }
  }

  // Step si issues super-tile si + 1 (if in range), waits for si (all but the copies of si + 1),
  // processes it.
  for (int si = 0; si < nst; si += 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer refilled next are done
    if (si + 1 < nst) issue(si + 1, B1);
    if (si + 1 < nst)
      asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    process(si, B0);
    if (si + 1 >= nst) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (si + 2 < nst) issue(si + 2, B0);
    if (si + 2 < nst)
      asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    process(si + 1, B1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const float osc[4] = {1.0f, 1.0f, 1.0f, 1.0f};
  static_assert(sizeof(sm.buf[0]) >= sizeof(float) * (6 * 128 + 256), "wave buffers hold the finish rows");
  packed_finish<BW>(oacc, m_run, lsum, 0.0f, 0.0f, osc, reinterpret_cast<float*>(&sm.buf[0][0]),
                    (int)(2 * sizeof(Bf16Buf) / sizeof(float)), &sm.st[0][0][0], &sh_last, args,
                    plan, x, b, hk, R);
}

}  // namespace

QAttnFn bf16_attn_fn(bool causal) {
  return causal ? bf16_attn_packed_kernel<true> : bf16_attn_packed_kernel<false>;
}

}  // namespace lq
