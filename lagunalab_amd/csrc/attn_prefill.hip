// Causal attention of a prefill chunk straight off the 8-bit KV cache: the L query rows of each
// head are the chunk's positions n-L .. n-1, whose K/V are already the last L of the first n
// cache rows, and row i sees keys 0 .. n-L+i. Replaces, for prefill chunks, the reference's path
// of dequantizing the whole cache (laguna_mlx/cache.py:99-100) and running SDPA with the causal
// mask (laguna.py:107); tests/test_cache.py:79-93 is the reference's guard that the quantized
// prefill never materializes the score matrix, and neither does this kernel.
//
// Work: one workgroup of 8 waves per (sequence, KV head, block of 256 query rows), the rows
// being PB = 256 / G positions of all G query heads of the KV head; wave w takes 32 rows (two
// MFMA N tiles of 16) of one head. The workgroup walks the 64-key tiles up to its last row's
// causal bound (128-key tiles), and each tile is brought into LDS once for all 8 waves:
//  * the raw tile (K and V codes, 128 B per key each, and the four bf16 word arrays) is copied
//    global -> LDS by DMA one tile ahead (two raw slots, 5 copies per thread per tile), landing
//    while the current tile is dequantized and computed;
//  * the workgroup dequantizes it once (scale * code + bias in fp32, rounded to fp16) into K [128
//    keys][128 dims] and V^T [128 dims][128 keys], both XOR-swizzled by 16-byte chunk so that the
//    MFMA operand reads are conflict-free;
//  * each wave then runs Q.K^T (v_mfma_f32_16x16x32_f16: M = 16 keys, N = 16 rows, K = 32 dims;
//    q pre-scaled by scale * log2(e) in fp16), the online softmax with lazy rescaling (a lane
//    holds keys 16 mt + 4 q + r of one row), and P.V (M = 16 dims, N = 16 rows, K = 32 keys; the
//    lane's own 8 probabilities are its k-slots: key 32 e + 16 h + 4 q + r of k-step e is slot
//    8 q + 4 h + r, and V^T stores the keys in that slot order).
// Tiles past a wave's last row are skipped by that wave; tiles straddling its rows' bounds are
// masked per row. Rows past L (a ragged last block) read no q and store nothing. Keys past n-1
// are never read: copies clamp their rows to n-1.
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

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
                 :: "v"(vc + kr0 * D + cofs), "s"(mv) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :: "v"(vc + kr1 * D + cofs), "s"(mv + 1024u) : "memory");
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
                 :: "v"(warr + wr * 2), "s"(mw) : "memory");
  };

  issue(0, 0);

  // ---- q of the wave's rows as MFMA B operands, pre-scaled (fp16), while the tile flies
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
  float m_run[2], lsum[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    m_run[nt] = -INFINITY;
    lsum[nt] = 0.0f;
  }

  for (int t = 0; t < T; ++t) {
    const int slot = t & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // tile t landed
    __syncthreads();  // every wave's copies of tile t, and every wave done with tile t - 1
    issue(t + 1, slot ^ 1);  // lands while tile t is dequantized and computed
    const PrefillRaw& rw = sm.raw[slot];
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // K: 16 codes of key dk, dims 16 dc .. 16 dc + 15
      const int u = tid + 512 * i;
      const int dk = u >> 3, dc = u & 7;
      const uint4 c4 = *reinterpret_cast<const uint4*>(rw.k + dk * D + 16 * dc);
      const int g = dc >> 2;
      const float s = g ? bf16_hi(rw.w[0][dk]) : bf16_lo(rw.w[0][dk]);
      const float z = g ? bf16_hi(rw.w[1][dk]) : bf16_lo(rw.w[1][dk]);
      const uint32_t cw[4] = {c4.x, c4.y, c4.z, c4.w};
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t c = cw[j];
        h[2 * j] = pack_h2(fmaf(s, (float)(c & 0xff), z), fmaf(s, (float)((c >> 8) & 0xff), z));
        h[2 * j + 1] = pack_h2(fmaf(s, (float)((c >> 16) & 0xff), z), fmaf(s, (float)(c >> 24), z));
      }
      uint4* kd = reinterpret_cast<uint4*>(sm.k + dk * D);
      kd[(2 * dc) ^ (dk & 15)] = make_uint4(h[0], h[1], h[2], h[3]);
      kd[(2 * dc + 1) ^ (dk & 15)] = make_uint4(h[4], h[5], h[6], h[7]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {  // V: slot group wv + 8 i (k-step ve, lane group vq), dims 2 lane, +1
      const int grp = wv + 8 * i;
      const int ve = grp >> 2, vq = grp & 3;
      const int g = lane >> 5;
      float lo[8], hi[8];
#pragma unroll
      for (int hh = 0; hh < 2; ++hh)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = 32 * ve + 16 * hh + 4 * vq + r;
          const uint32_t c2 = *reinterpret_cast<const uint16_t*>(rw.v + key * D + 2 * lane);
          const float s = g ? bf16_hi(rw.w[2][key]) : bf16_lo(rw.w[2][key]);
          const float z = g ? bf16_hi(rw.w[3][key]) : bf16_lo(rw.w[3][key]);
          lo[4 * hh + r] = fmaf(s, (float)(c2 & 0xff), z);
          hi[4 * hh + r] = fmaf(s, (float)(c2 >> 8), z);
        }
      const int d0 = 2 * lane;
      const int chunk = 4 * ve + vq;  // slots 32 ve + 8 vq .. + 7
      reinterpret_cast<uint4*>(sm.vt + d0 * PT)[chunk ^ (d0 & 15)] =
          make_uint4(pack_h2(lo[0], lo[1]), pack_h2(lo[2], lo[3]), pack_h2(lo[4], lo[5]),
                     pack_h2(lo[6], lo[7]));
      reinterpret_cast<uint4*>(sm.vt + (d0 + 1) * PT)[chunk ^ ((d0 + 1) & 15)] =
          make_uint4(pack_h2(hi[0], hi[1]), pack_h2(hi[2], hi[3]), pack_h2(hi[4], hi[5]),
                     pack_h2(hi[6], hi[7]));
    }
    __syncthreads();

    const int t0 = PT * t;
    if (t0 > lim_hi) continue;  // wave-uniform: no key of this tile is visible to its rows
    const bool full = t0 + PT - 1 <= lim_lo;

    // Per N tile: Q.K^T, softmax, P.V. The N tiles' chains are independent, so the second
    // tile's MFMAs can run while the first tile's softmax (VALU, exp) issues.
    // c: keys 16 mt + 4 lq4 + r of row 16 nt + lc (log2 units)
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
      f4_t c[PMT];
#pragma unroll
      for (int mt = 0; mt < PMT; ++mt) {
        const int key = 16 * mt + lc;
        const uint4* kr = reinterpret_cast<const uint4*>(sm.k + key * D);
        c[mt] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const uint4 a = kr[(4 * kk + lq4) ^ lc];
          c[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(words_as_h8(a.x, a.y, a.z, a.w),
                                                         qb[nt][kk], c[mt], 0, 0, 0);
        }
      }
      if (!full) {
#pragma unroll
        for (int mt = 0; mt < PMT; ++mt)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            c[mt][r] = t0 + 16 * mt + 4 * lq4 + r <= lim[nt] ? c[mt][r] : -INFINITY;
      }
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < PMT; ++mt)
#pragma unroll
        for (int r = 0; r < 4; ++r) tmax = fmaxf(tmax, c[mt][r]);
      tmax = max_xor16(tmax);
      tmax = max_xor32(tmax);
      const bool bump = tmax > m_run[nt] + RESCALE_LOG2;
      if (__builtin_amdgcn_ballot_w64(bump)) {
        const float mn = bump ? tmax : m_run[nt];
        const float alpha = m_run[nt] == -INFINITY ? 0.0f : exp2_nonpos(m_run[nt] - mn);
        m_run[nt] = mn;
        lsum[nt] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] *= alpha;
      }
      const float mref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];
      float ls = 0.0f;
#pragma unroll
      for (int e = 0; e < PE; ++e) {
        float p[8];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            p[4 * hh + r] = __builtin_amdgcn_exp2f(c[2 * e + hh][r] - mref);
            ls += p[4 * hh + r];
          }
        const half8_t pb = words_as_h8(pack_h2(p[0], p[1]), pack_h2(p[2], p[3]),
                                       pack_h2(p[4], p[5]), pack_h2(p[6], p[7]));
        // P.V: out^T[16 dt + 4 lq4 + r][row 16 nt + lc] += V^T[dims][slots] P^T[slots][rows]
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
          const int d = 16 * dt + lc;
          const uint4 a = reinterpret_cast<const uint4*>(sm.vt + d * PT)[(4 * e + lq4) ^ (d & 15)];
          oacc[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(words_as_h8(a.x, a.y, a.z, a.w),
                                                                pb, oacc[nt][dt], 0, 0, 0);
        }
      }
      lsum[nt] += ls;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the clamped copies past the end

  // ---- output rows: acc / l (the row's partial sums of its four lane groups added)
#pragma unroll
  for (int nt = 0; nt < 2; ++nt) {
    float l = sum_xor32(sum_xor16(lsum[nt]));
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
