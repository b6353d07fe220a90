// Causal attention of a prefill chunk straight off the 8-bit KV cache: the L query rows of each
// head are the chunk's positions n-L .. n-1, whose K/V are already the last L of the first n
// cache rows, and row i sees keys 0 .. n-L+i. Replaces, for prefill chunks, the reference's path
// of dequantizing the whole cache (laguna_mlx/cache.py:99-100) and running SDPA with the causal
// mask (laguna.py:107); tests/test_cache.py:79-93 is the reference's guard that the quantized
// prefill never materializes the score matrix, and neither does this kernel.
//
// Work: one workgroup of 8 waves per (sequence, KV head, block of 256 query rows), the rows
// being PB = 256 / G positions of all G query heads of the KV head; wave w takes 32 rows (two
// MFMA N tiles of 16) of one head. The workgroup walks the 128-key tiles up to its last row's
// causal bound; each tile is brought into LDS once for all 8 waves and dequantized once:
//  * the raw tile (K and V codes, 128 B per key each, and the four bf16 word arrays) is copied
//    global -> LDS by DMA two tiles ahead (two raw slots, 5 copies per thread per tile);
//  * the tile is dequantized (scale * code + bias in fp32, rounded to fp16) into K [128 keys][128
//    dims] and V^T [128 dims][128 keys], both XOR-swizzled by 16-byte chunk so that the MFMA
//    operand reads are conflict-free;
//  * each wave runs Q.K^T (v_mfma_f32_16x16x32_f16: M = 16 keys, N = 16 rows, K = 32 dims; q
//    pre-scaled by scale * log2(e) in fp16; each K fragment read once for both N tiles), the
//    online softmax with lazy rescaling (a lane holds keys 16 mt + 4 q + r of one row; scores
//    relative to the running maximum, which the accumulators start from), and P.V (M = 16 dims,
//    N = 16 rows, K = 32 keys; the lane's own 8 probabilities are its k-slots: key 32 e + 16 h +
//    4 q + r of k-step e is slot 8 q + 4 h + r, and V^T stores the keys in that slot order).
// Ping-pong: a SIMD holds one wave of each half of the workgroup (waves 0-3: group A, 4-7: group
// B), and the two halves run the same per-tile phases one phase apart, so that one wave's matrix
// phase (Q.K^T or P.V: MFMA and LDS reads) overlaps the other's vector phase (softmax, or its
// share of the dequantization: K by group A, V by group B). Four barrier-separated slots per tile:
//
//   slot    group A                  group B
//   4t      Q.K^T(t)                 dequantize V(t)
//   4t+1    softmax(t)               Q.K^T(t)
//   4t+2    P.V(t)                   softmax(t)
//   4t+3    dequantize K(t+1)        P.V(t)
//
// K(t+1) overwrites K(t) after both halves' Q.K^T(t), V(t) overwrites V(t-1) after both halves'
// P.V(t-1), so one fp16 K and one V^T buffer suffice. Raw tile t+2 is issued in slot 4t+1 (its
// slot held raw t, whose K was dequantized in slot 4t-1 and V in slot 4t) and waited for two
// tiles later.
// Tiles past a wave's last row are skipped by that wave (it keeps its copy and dequantization
// duties); tiles straddling its rows' bounds are masked per row. Rows past L (a ragged last block)
// read no q and store nothing. Keys past n-1 are never read: copies clamp their rows to n-1.
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

// Codes 2 h, 2 h + 1 of a word as the fp16 pair 1024 + c (exponent 10: the code is the mantissa),
// one v_perm_b32; scale * (1024 + c) + (bias - 1024 scale) then dequantizes in one
// v_fma_mix (fp32 arithmetic, rounded once to fp16).
__device__ __forceinline__ half2_t codes_1024(uint32_t w, int h) {
  return __builtin_bit_cast(half2_t,
                            __builtin_amdgcn_perm(0x64646464u, w, h ? 0x04030402u : 0x04010400u));
}

constexpr int PW = 8;       // waves per workgroup
constexpr int PROWS = 256;  // query rows per workgroup
constexpr int PT = 128;     // keys per tile
constexpr int PMT = PT / 16;  // M tiles (16 keys) per tile
constexpr int PE = PT / 32;   // P.V k-steps (32 keys) per tile

struct PrefillRaw {
  alignas(16) uint8_t k[PT * D];  // row-major [key][128 B]
  uint8_t v[PT * D];
  uint32_t w[4][PT];              // K scale, K bias, V scale, V bias words (two bf16 groups each)
};

struct PrefillSmem {
  PrefillRaw raw[2];
  alignas(16) _Float16 k[PT * D];   // [key][dim], 16-byte chunk j of key r at chunk j ^ (r & 15)
  alignas(16) _Float16 vt[D * PT];  // [dim][slot], 16-byte chunk j of dim d at chunk j ^ (d & 15)
};

__global__ __launch_bounds__(64 * PW, 1) void q8_prefill_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ ks, const uint16_t* __restrict__ kb,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vs,
    const uint16_t* __restrict__ vb, uint16_t* __restrict__ out, int64_t cap, int n, int L,
    int Hkv, int G, int npb, float qk_scale_log2) {
  __shared__ PrefillSmem sm;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool grp_a = wv < PW / 2;  // wave-uniform
  const int lc = lane & 15;
  const int lq4 = lane >> 4;
  const int x = blockIdx.x;
  const int hk = x % Hkv;  // consecutive workgroups (consecutive XCDs) take consecutive KV heads
  // last position blocks first: they see the most keys, so the dispatch order is longest first
  const int pb = npb - 1 - (x / Hkv) % npb;
  const int b = x / (Hkv * npb);
  const int PB = PROWS / G;  // positions per workgroup
  const int Hq = Hkv * G;
  const int base = n - L;    // row i sees keys <= base + i

  // this wave's rows: head gh, positions p0 .. p0 + 31 (row 16 nt + lc of the wave: p0 + 16 nt + lc)
  const int gh = (32 * wv) / PB;
  const int p0 = pb * PB + (32 * wv) % PB;
  const int lim_lo = base + p0;                                  // bound of the wave's first row
  const int lim_hi = p0 < L ? base + min(p0 + 31, L - 1) : -1;  // of its last valid row
  const int wg_last = min(pb * PB + PB - 1, L - 1);  // the workgroup's last valid position
  const int T = (base + wg_last) / PT + 1;           // tiles the workgroup needs

  const int64_t row0 = ((int64_t)b * Hkv + hk) * cap;
  const int last_row = n - 1;

  // ---- raw tile copies, per thread: two 16-byte K copies (wave wv: keys 16 wv .. 16 wv + 15),
  // two V copies, one word (wave wv: word array wv / 2, keys 64 (wv % 2) + lane)
  const uint32_t lds_raw = lds_addr(&sm.raw[0]);
  const int ck = 16 * wv + (lane >> 3);  // key of this lane's first K / V copy (second: + 8)
  const uint32_t cofs = 16u * (uint32_t)(lane & 7);
  const uint32_t cofs_v = 16u * (uint32_t)((lane & 7) ^ (lane >> 3));  // V: chunk c of row r at c ^ (r & 7)
  const int wa = wv >> 1;
  const uint16_t* warr = wa == 0 ? ks : wa == 1 ? kb : wa == 2 ? vs : vb;
  const int wkey = 64 * (wv & 1) + lane;
  auto issue = [&](int t, int slot) {
    const int t0 = PT * min(t, T - 1);
    const uint32_t lb = lds_raw + (uint32_t)slot * (uint32_t)sizeof(PrefillRaw);
    // M0 operands: wave-uniform values, made explicit so that they live in SGPRs
    const uint32_t mk = __builtin_amdgcn_readfirstlane(lb + offsetof(PrefillRaw, k) + 2048u * wv);
    const uint32_t mv = __builtin_amdgcn_readfirstlane(lb + offsetof(PrefillRaw, v) + 2048u * wv);
    const uint32_t mw = __builtin_amdgcn_readfirstlane(
        lb + offsetof(PrefillRaw, w) + 4u * (uint32_t)(PT * wa + 64 * (wv & 1)));
    const int64_t kr0 = row0 + min(t0 + ck, last_row);
    const int64_t kr1 = row0 + min(t0 + ck + 8, last_row);
    const int64_t wr = row0 + min(t0 + wkey, last_row);
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(kc + kr0 * D + cofs), "s"(mk) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(kc + kr1 * D + cofs), "s"(mk + 1024u) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(vc + kr0 * D + cofs_v), "s"(mv) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(vc + kr1 * D + cofs_v), "s"(mv + 1024u) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
                 :: "v"(warr + wr * 2), "s"(mw) : "memory");
  };

  // ---- dequantization shares: K of a tile by group A (256 threads, 4 chunks of 16 codes each),
  // V^T by group B (16 slot groups, 4 per wave)
  const int ta = tid & 255;  // thread index within the group
  // (the thread index is re-read through an empty asm in each call, so that the compiler
  // recomputes these addresses in the slot instead of holding them in registers across the loop)
  auto dequant_k = [&](const PrefillRaw& rw) {
    int tr = ta;
    asm volatile("" : "+v"(tr));
    const int dc = tr & 7;  // 16 codes of key (tr >> 3) + 32 i, dims 16 dc .. 16 dc + 15
    const uint32_t gsel = (dc >> 2) ? SEL_HI : SEL_LO;
    uint4 c4[4];
    uint32_t sw[4], zw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {  // all reads first: one LDS round trip
      const int dk = (tr >> 3) + 32 * i;
      c4[i] = *reinterpret_cast<const uint4*>(rw.k + dk * D + 16 * dc);
      sw[i] = rw.w[0][dk];
      zw[i] = rw.w[1][dk];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int dk = (tr >> 3) + 32 * i;
      const float s = bf16_pick(sw[i], gsel);
      const float z = fmaf(-1024.0f, s, bf16_pick(zw[i], gsel));  // bias - 1024 scale
      const uint32_t cw[4] = {c4[i].x, c4[i].y, c4[i].z, c4[i].w};
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const half2_t c01 = codes_1024(cw[j], 0), c23 = codes_1024(cw[j], 1);
        h[2 * j] = pack_h2(fmaf(s, (float)c01.x, z), fmaf(s, (float)c01.y, z));
        h[2 * j + 1] = pack_h2(fmaf(s, (float)c23.x, z), fmaf(s, (float)c23.y, z));
      }
      uint4* kd = reinterpret_cast<uint4*>(sm.k + dk * D);
      kd[(2 * dc) ^ (dk & 15)] = make_uint4(h[0], h[1], h[2], h[3]);
      kd[(2 * dc + 1) ^ (dk & 15)] = make_uint4(h[4], h[5], h[6], h[7]);
    }
  };
  // V^T chunk (dim d, k-step e, lane group q) = the 8 keys T[j] = 32 e + 16 (j / 4) + 4 q + j % 4
  // of dim d, in that slot order. Group B wave e, lane group q: one transposed read
  // (ds_read_b64_tr_b8) per 16-dim window w gives lane (q, i) the codes of T[0..7] at dim 16 w + i
  // (source lane s addresses key T[s / 2], bytes 8 (s % 2) of the window; the raw V rows are
  // stored with 16-byte chunk c of row r at chunk c ^ (r & 7)).
  auto dequant_v = [&](const PrefillRaw& rw) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const int e = wv - PW / 2, qg = ln >> 4, i = ln & 15;
    const int k0 = 32 * e + 4 * qg;  // T[0..3] = k0 .. k0 + 3, T[4..7] = k0 + 16 .. k0 + 19
    const int skey = k0 + 16 * (i >> 3) + ((i >> 1) & 3);  // T[i / 2]: this lane's source key
    const uint8_t* src = rw.v + skey * D + 8 * (i & 1);
    const int ssw = skey & 7;
    const uint4 s03 = *reinterpret_cast<const uint4*>(&rw.w[2][k0]);
    const uint4 s47 = *reinterpret_cast<const uint4*>(&rw.w[2][k0 + 16]);
    const uint4 z03 = *reinterpret_cast<const uint4*>(&rw.w[3][k0]);
    const uint4 z47 = *reinterpret_cast<const uint4*>(&rw.w[3][k0 + 16]);
    const uint32_t sw[8] = {s03.x, s03.y, s03.z, s03.w, s47.x, s47.y, s47.z, s47.w};
    const uint32_t zw[8] = {z03.x, z03.y, z03.z, z03.w, z47.x, z47.y, z47.z, z47.w};
#pragma unroll
    for (int g = 0; g < 2; ++g) {  // dims 64 g .. 64 g + 63: quant group g, windows 4 g .. 4 g + 3
      v2i_t raw[4];
#pragma unroll
      for (int w = 0; w < 4; ++w)
        raw[w] = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)(src + 16 * ((4 * g + w) ^ ssw)));
      float sj[8], zj[8];  // scale and bias - 1024 scale of key T[j], group g
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        sj[j] = g ? bf16_hi(sw[j]) : bf16_lo(sw[j]);
        zj[j] = fmaf(-1024.0f, sj[j], g ? bf16_hi(zw[j]) : bf16_lo(zw[j]));
      }
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        const int d = 16 * (4 * g + w) + i;
        float v[8];
#pragma unroll
        for (int hw = 0; hw < 2; ++hw) {  // keys T[4 hw .. 4 hw + 3]
          const uint32_t word = hw ? (uint32_t)raw[w].y : (uint32_t)raw[w].x;
          const half2_t c01 = codes_1024(word, 0), c23 = codes_1024(word, 1);
          v[4 * hw + 0] = fmaf(sj[4 * hw + 0], (float)c01.x, zj[4 * hw + 0]);
          v[4 * hw + 1] = fmaf(sj[4 * hw + 1], (float)c01.y, zj[4 * hw + 1]);
          v[4 * hw + 2] = fmaf(sj[4 * hw + 2], (float)c23.x, zj[4 * hw + 2]);
          v[4 * hw + 3] = fmaf(sj[4 * hw + 3], (float)c23.y, zj[4 * hw + 3]);
        }
        reinterpret_cast<uint4*>(sm.vt + d * PT)[(4 * e + qg) ^ i] =
            make_uint4(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]),
                       pack_h2(v[6], v[7]));
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  issue(0, 0);
  issue(1, 1);

  // ---- q of the wave's rows as MFMA B operands, pre-scaled (fp16), while the tiles fly
  half8_t qb[2][4];
  int lim[2];  // causal bound of this lane's row per N tile (-1: not a row of the chunk)
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const int i = p0 + 16 * nt + lc;
    const bool valid = i < L;
    lim[nt] = valid ? base + i : -1;
    const uint16_t* qr = q + (((int64_t)b * Hq + hk * G + gh) * L + (valid ? i : 0)) * D;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const uint4 u = *reinterpret_cast<const uint4*>(qr + 32 * kk + 8 * lq4);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qb[nt][kk][2 * j] = valid ? (_Float16)(bf16_lo(w[j]) * qk_scale_log2) : (_Float16)0.0f;
        qb[nt][kk][2 * j + 1] = valid ? (_Float16)(bf16_hi(w[j]) * qk_scale_log2) : (_Float16)0.0f;
      }
    }
  }

  f4_t oacc[2][8];
  f4_t lacc[2];  // row sums of P (MFMA layout: all four values of a lane hold its row's sum)
  float m_run[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    lacc[nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    m_run[nt] = -INFINITY;
  }
  half8_t ones8;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones8[j] = (_Float16)1.0f;

  // ---- per-tile phases of one wave
  // MFMA A fragments: K key 16 mt + lc, dims 32 kk + 8 lq4 .. + 7 at kfrag[kk] + 256 mt (uint4
  // units); V^T dim 16 dt + lc, slots 32 e + 8 lq4 .. + 7 at vfrag[e] + 256 dt
  const uint4* kfrag[4];
  const uint4* vfrag[PE];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    kfrag[j] = reinterpret_cast<const uint4*>(sm.k) + 16 * lc + ((4 * j + lq4) ^ lc);
    vfrag[j] = reinterpret_cast<const uint4*>(sm.vt) + 16 * lc + ((4 * j + lq4) ^ lc);
  }
  f4_t c[2][PMT];     // scores, c[nt][mt]: keys 16 mt + 4 lq4 + r of row 16 nt + lc (log2 units)
  half8_t pw[2][PE];  // P in fp16, per N tile and k-step
  // Q.K^T of both N tiles from one read of each K fragment, relative to the rows' running
  // maxima (0 before the first): the accumulators start at -mref
  auto qk = [&]() {
    f4_t cinit[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      const float mref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      cinit[nt] = f4_t{-mref, -mref, -mref, -mref};
    }
    // fragments one M tile ahead of the MFMAs that use them (the scheduling barriers keep the
    // reads of M tile mt + 1 issued before the MFMAs of M tile mt)
    uint4 fa[2][4];
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) fa[0][kk] = kfrag[kk][0];
#pragma unroll
    for (int mt = 0; mt < PMT; ++mt) {
      if (mt + 1 < PMT) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) fa[(mt + 1) & 1][kk] = kfrag[kk][256 * (mt + 1)];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const uint4 a = fa[mt & 1][kk];  // key 16 mt + lc
        const half8_t ah = words_as_h8(a.x, a.y, a.z, a.w);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)  // each chain starts from the shared -mref tuple
          c[nt][mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, qb[nt][kk],
                                                             kk == 0 ? cinit[nt] : c[nt][mt], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // softmax per N tile: masking, lazy rescale, P in fp16 (its row sums are taken by P.V)
  auto softmax = [&](int t0, bool full) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      if (!full) {
#pragma unroll
        for (int mt = 0; mt < PMT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            c[nt][mt][r] = t0 + 16 * mt + 4 * lq4 + r <= lim[nt] ? c[nt][mt][r] : -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < PMT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, c[nt][mt][r]);
      tmax = max_xor16(tmax);
      tmax = max_xor32(tmax);
      // a new running maximum: the tile's exceeds it by more than RESCALE_LOG2 (any finite one
      // the first time)
      const bool bump = tmax > (m_run[nt] == -INFINITY ? -INFINITY : RESCALE_LOG2);
      if (__builtin_amdgcn_ballot_w64(bump)) {
        const float mref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
        const float mn = bump ? mref + tmax : m_run[nt];
        const float alpha = m_run[nt] == -INFINITY ? 0.0f : exp2_nonpos(m_run[nt] - mn);
        m_run[nt] = mn;
        lacc[nt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] *= alpha;
        const float shift = bump ? tmax : 0.0f;  // new reference minus the one the scores hold
#pragma unroll
        for (int mt = 0; mt < PMT; ++mt) c[nt][mt] -= shift;
      }
#pragma unroll
      for (int e = 0; e < PE; ++e) {
        half2_t ph[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int hh = j >> 1, r = 2 * (j & 1);
          ph[j] = half2_t{(_Float16)__builtin_amdgcn_exp2f(c[nt][2 * e + hh][r]),
                          (_Float16)__builtin_amdgcn_exp2f(c[nt][2 * e + hh][r + 1])};
        }
        pw[nt][e] = __builtin_bit_cast(half8_t, ph);
      }
    }
  };
  // P.V of both N tiles from one read of each V^T fragment, and the rows' sums of P:
  // out^T[16 dt + 4 lq4 + r][row 16 nt + lc] += V^T[dims][slots] P^T[slots][rows]
  auto pv = [&]() {
    // fragments four dims tiles ahead (half a k-step), as in qk: step u = (k-step u / 2, dim
    // tiles 4 (u % 2) .. + 3)
    uint4 fv[2][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fv[0][j] = vfrag[0][256 * j];
#pragma unroll
    for (int u = 0; u < 2 * PE; ++u) {
      if (u + 1 < 2 * PE) {
        const int e1 = (u + 1) >> 1, d1 = 4 * ((u + 1) & 1);
#pragma unroll
        for (int j = 0; j < 4; ++j) fv[(u + 1) & 1][j] = vfrag[e1][256 * (d1 + j)];
      }
      __builtin_amdgcn_sched_barrier(0);
      const int e = u >> 1, d0 = 4 * (u & 1);
      if (u & 1) {  // row sums of this k-step's P: a ones A operand (every output row the sum)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          lacc[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones8, pw[nt][e], lacc[nt], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint4 a = fv[u & 1][j];  // dim 16 (d0 + j) + lc
        const half8_t ah = words_as_h8(a.x, a.y, a.z, a.w);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
          oacc[nt][d0 + j] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, pw[nt][e], oacc[nt][d0 + j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // ---- prologue: raw tile 0 landed (only tile 1's copies outstanding), K(0) dequantized
  asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
  __syncthreads();
  if (grp_a) dequant_k(sm.raw[0]);
  __syncthreads();

  // The two halves run their own loops (wave-uniform branch): each wave passes the same four
  // barriers per tile. Tiles 0 .. Tact - 1 hold keys visible to the wave's rows; past them the
  // wave keeps only its copy and dequantization duties. (Two loops rather than a condition per
  // phase, so that the scores and P are not live across the loop's back edge.)
  const int Tact = lim_hi < 0 ? 0 : min(T, lim_hi / PT + 1);
  if (grp_a) {
    int t = 0;
    for (; t < Tact; ++t) {
      const int t0 = PT * t;
      qk();                                            // slot 4t
      __syncthreads();
      issue(t + 2, t & 1);                             // slot 4t + 1: raw t + 2 into t's slot
      softmax(t0, t0 + PT - 1 <= lim_lo);
      __syncthreads();
      pv();                                            // slot 4t + 2
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");  // raw tile t + 1 landed
      __syncthreads();
      if (t + 1 < T) dequant_k(sm.raw[(t + 1) & 1]);  // slot 4t + 3
      __syncthreads();
    }
    for (; t < T; ++t) {
      __syncthreads();
      issue(t + 2, t & 1);
      __syncthreads();
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      __syncthreads();
      if (t + 1 < T) dequant_k(sm.raw[(t + 1) & 1]);
      __syncthreads();
    }
  } else {
    int t = 0;
    for (; t < Tact; ++t) {
      const int t0 = PT * t;
      dequant_v(sm.raw[t & 1]);                        // slot 4t
      __syncthreads();
      issue(t + 2, t & 1);                             // slot 4t + 1
      qk();
      __syncthreads();
      softmax(t0, t0 + PT - 1 <= lim_lo);              // slot 4t + 2
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      __syncthreads();
      pv();                                            // slot 4t + 3
      __syncthreads();
    }
    for (; t < T; ++t) {
      dequant_v(sm.raw[t & 1]);
      __syncthreads();
      issue(t + 2, t & 1);
      __syncthreads();
      asm volatile("s_waitcnt vmcnt(5)" ::: "memory");
      __syncthreads();
      __syncthreads();
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the end

  // ---- output rows: acc / l
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    const float l = lacc[nt][0];
    const int i = p0 + 16 * nt + lc;
    if (lim[nt] < 0) continue;
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
    uint16_t* orow = out + (((int64_t)b * Hq + hk * G + gh) * L + i) * D;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const f4_t o = oacc[nt][dt];
      const uint32_t lo = (uint32_t)f32_to_bf16(o[0] * inv) | ((uint32_t)f32_to_bf16(o[1] * inv) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(o[2] * inv) | ((uint32_t)f32_to_bf16(o[3] * inv) << 16);
      *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * lq4) = make_uint2(lo, hi);
    }
  }
}

}  // namespace
}  // namespace lq

extern "C" int lq_q8_prefill_attn(const uint16_t* q, const uint8_t* kc, const uint16_t* ks,
                                  const uint16_t* kb, const uint8_t* vc, const uint16_t* vs,
                                  const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv,
                                  int64_t L, int64_t D, int64_t cap, int64_t n, float scale,
                                  uint16_t* out, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(D == 128, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "Hq=%lld must be a multiple of Hkv=%lld",
               (long long)Hq, (long long)Hkv);
  const int64_t G = Hq / Hkv;
  LQ_CHECK_ARG(G == 1 || G == 2 || G == 4 || G == 8,
               "prefill kernel takes 1, 2, 4 or 8 query heads per KV head (got %lld)", (long long)G);
  LQ_CHECK_ARG(B >= 1 && L >= 1 && L <= n && n <= cap && cap <= (1 << 24),
               "need 1 <= L=%lld <= n=%lld <= cap=%lld <= 2^24", (long long)L, (long long)n,
               (long long)cap);
  LQ_CHECK_ARG(q && kc && ks && kb && vc && vs && vb && out, "null pointer");
  const int64_t npb = (L + PROWS / G - 1) / (PROWS / G);
  const int64_t wgs = B * Hkv * npb;
  LQ_CHECK_ARG(wgs <= (int64_t)INT32_MAX, "too many workgroups");
  q8_prefill_kernel<<<dim3((unsigned)wgs), dim3(64 * PW), 0, (hipStream_t)stream>>>(
      q, kc, ks, kb, vc, vs, vb, out, cap, (int)n, (int)L, (int)Hkv, (int)G, (int)npb,
      scale * 1.4426950408889634f);
  LQ_CHECK_LAUNCH("q8_prefill_kernel");
  return LQ_OK;
}
