// Fused attention over the 8-bit KV cache on MFMA: single-token decode and the multi-query
// causal verify block of speculative decoding.
//
// Replaces q8_decode_attention (laguna_mlx/q8_attn.py:102-130: the Metal kernel at :17-99 and
// the block merge at :126-130) and, for verify blocks, the reference's unfused path
// (dequantize, cache.py:99-100, then SDPA with the bottom-right causal mask, laguna.py:107,
// 183-186).
//
// Design (CDNA4, gfx950):
//  * Grid (split, kv head): each workgroup owns a contiguous key range of one sequence and one
//    KV head and serves every query row of that KV head (G heads x L positions), so each K/V
//    byte is read from HBM once. The four waves of a workgroup split its range and run fully
//    independently (no workgroup barrier in the key loop); their partials meet once at the end.
//  * Per wave, keys stream in tiles of 32 rows with a one-tile prefetch. K and V codes and the
//    four scale/bias word arrays go straight from global memory to LDS (global_load_lds),
//    double-buffered, so nothing in flight holds a VGPR and the only wait is one fixed vmcnt.
//  * Q.K^T: v_mfma_f32_16x16x32_f16. A = 16 key rows x 32 dims of (1024 + code) fp16 pairs (one
//    v_perm_b32 per pair), B = 32 dims x 16 query rows of q in fp16, one accumulator per quant
//    group so the affine terms fold out: q.(s c + b) = s (q.(1024 + c)) + (b - 1024 s) sum(q).
//  * Softmax in the MFMA result layout: a lane holds 8 keys of one query row; the column max is
//    two cross-lane exchanges; p = exp2(s - m) with scale*log2(e) folded into the scores.
//  * P.V: v_mfma_f32_16x16x32_f16 with A = V^T (16 dims x 32 keys) read from the LDS tile with
//    ds_read_b64_tr_b8 (one 8-byte transposed read per operand) and B = P * scale_v in fp16.
//    The keys of B's k-slots are ordered exactly as the lane already holds them after Q.K^T,
//    so P never leaves registers. Bias and 1024-offset terms are per-row sums, not per element.
//  * Partials (m, l, acc[128]) per (split, query row) go to the workspace. The packed kernel
//    merges them itself (the last workgroup of each sequence and KV head to finish, counted with
//    one atomic per workgroup); after the general kernel decode_merge_kernel does the merge.
#include "attn_dev.h"

namespace lq {
namespace {

using namespace attn;

constexpr int WT = 32;       // key rows per wave tile
constexpr int NWAVE = 4;
constexpr int NTHR = 64 * NWAVE;

// Per wave, per buffer: K and V codes (32 rows x 128 B each; the 16-byte chunk c of row r sits at
// chunk position c ^ (r & 7) to spread the column reads over the LDS banks) and the scale/bias
// word arrays ks, kb, vs, vb (32 each).
struct WaveBuf {
  uint8_t k[WT * D];
  uint8_t v[WT * D];
  uint32_t ks[WT];
  uint32_t kb[WT];
  uint32_t vs[WT];
  uint32_t vb[WT];
};

template <int NT>
struct QSmem {
  union {
    WaveBuf buf[NWAVE][2];
    struct {
      float acc[NWAVE][16 * NT][D];  // wave partials, final merge
    } fin;
  };
  float st[NWAVE][16 * NT][6];  // m, l, wsum0, wsum1, bsum0, bsum1
};

__device__ __forceinline__ half8_t codes8_as_h8(uint32_t w0, uint32_t w1) {
  half8_t r;
  const half2_t a = codes_as_h2(w0, SEL_B01), b = codes_as_h2(w0, SEL_B23);
  const half2_t c = codes_as_h2(w1, SEL_B01), d = codes_as_h2(w1, SEL_B23);
  r[0] = a[0]; r[1] = a[1]; r[2] = b[0]; r[3] = b[1];
  r[4] = c[0]; r[5] = c[1]; r[6] = d[0]; r[7] = d[1];
  return r;
}

template <int NT, bool CAUSAL>
__global__ __launch_bounds__(NTHR) void q8_attn_mfma_kernel(
    AttnArgs args, DecodePlan plan) {
  __shared__ QSmem<NT> sm;
  const uint16_t* __restrict__ q = args.q;
  const uint8_t* __restrict__ kc = args.kc;
  const uint16_t* __restrict__ ks = args.ks;
  const uint16_t* __restrict__ kb = args.kb;
  const uint8_t* __restrict__ vc = args.vc;
  const uint16_t* __restrict__ vs = args.vs;
  const uint16_t* __restrict__ vb = args.vb;
  float* __restrict__ part_acc = args.part_acc;
  float2* __restrict__ part_ml = args.part_ml;
  const int Hkv = args.Hkv, G = args.G, L = args.L;
  const int64_t cap = args.cap;
  const float qk_scale_log2 = args.qk_scale_log2;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  int b;
  find_seq(plan, x, b);
  const int n = plan.len[b];
  const int c_begin = (x - plan.split_begin[b]) * plan.chunk;
  const int c_end = min(c_begin + plan.chunk, n);
  const int sub = (c_end - c_begin + NWAVE - 1) / NWAVE;
  const int w_begin = min(c_begin + wv * sub, c_end);
  const int w_end = min(w_begin + sub, c_end);
  const int ntiles = (w_end - w_begin + WT - 1) / WT;
  const int R = G * L;            // query rows of this KV head
  const int Hq = Hkv * G;
  const int64_t row0 = ((int64_t)b * Hkv + hk) * cap;

  const int lc = lane & 15;       // MFMA column (query row within an N tile)
  const int lq4 = lane >> 4;      // lane group 0..3

  // ---- B operands of Q.K^T: per N tile, group g, half e: 8 dims per lane (fp16)
  // k-slot j of lane group lq4 in step (g, e) is dim 64 g + 16 lq4 + 8 e + j
  half8_t qb[NT][2][2];
  float qsum[NT][2];  // sum over the group's 64 dims of the fp16 q (scaled by qk_scale_log2)
  int qpos[NT];       // query position i of this lane's column (causal bound)
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int qi = nt * 16 + lc;
    const bool valid = qi < R;
    const int gh = valid ? qi / L : 0;
    const int i = valid ? qi - gh * L : 0;
    qpos[nt] = i;
    const uint16_t* qr = q + (((int64_t)b * Hq + hk * G + gh) * L + i) * D;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float s = 0.0f;
      const uint4 u = *reinterpret_cast<const uint4*>(qr + 64 * g + 16 * lq4);
      const uint4 v = *reinterpret_cast<const uint4*>(qr + 64 * g + 16 * lq4 + 8);
      const uint32_t w[8] = {u.x, u.y, u.z, u.w, v.x, v.y, v.z, v.w};
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t wd = w[4 * e + j];
          const _Float16 lo = valid ? (_Float16)bf16_to_f32((uint16_t)(wd & 0xffffu)) : (_Float16)0.0f;
          const _Float16 hi = valid ? (_Float16)bf16_to_f32((uint16_t)(wd >> 16)) : (_Float16)0.0f;
          qb[nt][g][e][2 * j] = lo;
          qb[nt][g][e][2 * j + 1] = hi;
          s += (float)lo + (float)hi;
        }
      s += shfl_xor_f(s, 16);
      s += shfl_xor_f(s, 32);
      qsum[nt][g] = s * qk_scale_log2;
    }
  }

  f4_t oacc[NT][8];  // out^T[16 dt + 4 lq4 + r][column]
  float m_run[NT], lsum[NT], wsum[NT][2], bsum[NT][2];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] = f4_t{0.f, 0.f, 0.f, 0.f};
    m_run[nt] = -INFINITY;
    lsum[nt] = 0.0f;
    wsum[nt][0] = wsum[nt][1] = bsum[nt][0] = bsum[nt][1] = 0.0f;
  }

  const uint8_t* kbase = kc + row0 * D;
  const uint8_t* vbase = vc + row0 * D;
  const uint32_t* ksw = reinterpret_cast<const uint32_t*>(ks + row0 * 2);
  const uint32_t* kbw = reinterpret_cast<const uint32_t*>(kb + row0 * 2);
  const uint32_t* vsw = reinterpret_cast<const uint32_t*>(vs + row0 * 2);
  const uint32_t* vbw = reinterpret_cast<const uint32_t*>(vb + row0 * 2);
  const int causal_base = n - L;  // query i sees keys t <= causal_base + i

  // Issue tile `jt`'s loads straight into LDS buffer jt & 1 (10 loads per lane): K and V codes
  // with the chunk swizzle applied on the global side, and the four scale/bias word arrays.
  auto issue = [&](int jt) {
    const int t0 = w_begin + jt * WT;
    const int last = max(w_end - 1, 0);
    WaveBuf& wb = sm.buf[wv][jt & 1];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = (lane >> 3) + 8 * u;
      const int64_t t = min(t0 + row, last);
      const int chunk = (lane & 7) ^ (row & 7);
      g2l_b128(kbase + t * D + 16 * chunk, wb.k + 1024 * u);
      g2l_b128(vbase + t * D + 16 * chunk, wb.v + 1024 * u);
    }
    const int64_t ts = min(t0 + (lane & 31), last);
    g2l_b32(lane < 32 ? (const void*)(ksw + ts) : (const void*)(kbw + ts), wb.ks);
    g2l_b32(lane < 32 ? (const void*)(vsw + ts) : (const void*)(vbw + ts), wb.vs);
  };

  // Process tile `jt` (its loads complete): scores, softmax, P.V.
  auto process = [&](int jt) {
    const int t0 = w_begin + jt * WT;
    const WaveBuf& wb = sm.buf[wv][jt & 1];
    // Q.K^T per (row tile mt, N tile nt, group g)
    f4_t sacc[2][NT][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int r = 16 * mt + lc;  // A row = key; 16 bytes = dims 64 g + 16 lq4 + (0..15)
        const uint4 c =
            *reinterpret_cast<const uint4*>(wb.k + r * D + 16 * ((lq4 + 4 * g) ^ (r & 7)));
        const half8_t a0 = codes8_as_h8(c.x, c.y);
        const half8_t a1 = codes8_as_h8(c.z, c.w);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          f4_t z = {0.f, 0.f, 0.f, 0.f};
          z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, qb[nt][g][0], z, 0, 0, 0);
          z = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, qb[nt][g][1], z, 0, 0, 0);
          sacc[mt][nt][g] = z;
        }
      }
    half8_t wbo[NT][2];  // P.V B operands per N tile and quant group
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float sc[2][4];
      float tmax = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        // scale/bias words of this lane's keys 16 mt + 4 lq4 + r
        const uint4 ksr = *reinterpret_cast<const uint4*>(wb.ks + 16 * mt + 4 * lq4);
        const uint4 kbr = *reinterpret_cast<const uint4*>(wb.kb + 16 * mt + 4 * lq4);
        const uint32_t kw[4] = {ksr.x, ksr.y, ksr.z, ksr.w};
        const uint32_t bw[4] = {kbr.x, kbr.y, kbr.z, kbr.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = t0 + 16 * mt + 4 * lq4 + r;
          const float s0 = bf16_to_f32((uint16_t)(kw[r] & 0xffffu));
          const float s1 = bf16_to_f32((uint16_t)(kw[r] >> 16));
          const float b0 = bf16_to_f32((uint16_t)(bw[r] & 0xffffu));
          const float b1 = bf16_to_f32((uint16_t)(bw[r] >> 16));
          float v = (s0 * qk_scale_log2) * sacc[mt][nt][0][r] + (b0 - 1024.0f * s0) * qsum[nt][0];
          v += (s1 * qk_scale_log2) * sacc[mt][nt][1][r] + (b1 - 1024.0f * s1) * qsum[nt][1];
          bool ok = t < w_end;
          if (CAUSAL) ok = ok && t <= causal_base + qpos[nt];
          v = ok ? v : -INFINITY;
          sc[mt][r] = v;
          tmax = fmaxf(tmax, v);
        }
      }
      tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
      tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
      // Lazy rescaling: the reference max m_run only moves when a tile's max exceeds it by more
      // than RESCALE_LOG2 (so p <= 2^RESCALE_LOG2); the accumulators are rescaled only then.
      const bool bump = tmax > m_run[nt] + RESCALE_LOG2;
      float alpha = 1.0f;
      if (__builtin_amdgcn_ballot_w64(bump)) {
        const float mn = bump ? tmax : m_run[nt];
        alpha = m_run[nt] == -INFINITY ? 0.0f : exp2f(m_run[nt] - mn);
        m_run[nt] = mn;
        lsum[nt] *= alpha;
        wsum[nt][0] *= alpha;
        wsum[nt][1] *= alpha;
        bsum[nt][0] *= alpha;
        bsum[nt][1] *= alpha;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) oacc[nt][dt] *= alpha;
      }
      const float mref = m_run[nt] == -INFINITY ? 0.0f : m_run[nt];  // no valid key yet
      // P and the P.V B operands (k-slot j: key 4 lq4 + j for j < 4, 16 + 4 lq4 + j - 4 else)
      float ls = 0.f, ws0 = 0.f, ws1 = 0.f, bs0 = 0.f, bs1 = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const uint4 vsr = *reinterpret_cast<const uint4*>(wb.vs + 16 * mt + 4 * lq4);
        const uint4 vbr = *reinterpret_cast<const uint4*>(wb.vb + 16 * mt + 4 * lq4);
        const uint32_t sw[4] = {vsr.x, vsr.y, vsr.z, vsr.w};
        const uint32_t bw[4] = {vbr.x, vbr.y, vbr.z, vbr.w};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float p = exp2f(sc[mt][r] - mref);
          const _Float16 w0 = (_Float16)(p * bf16_to_f32((uint16_t)(sw[r] & 0xffffu)));
          const _Float16 w1 = (_Float16)(p * bf16_to_f32((uint16_t)(sw[r] >> 16)));
          wbo[nt][0][4 * mt + r] = w0;
          wbo[nt][1][4 * mt + r] = w1;
          ls += p;
          ws0 += (float)w0;
          ws1 += (float)w1;
          bs0 += p * bf16_to_f32((uint16_t)(bw[r] & 0xffffu));
          bs1 += p * bf16_to_f32((uint16_t)(bw[r] >> 16));
        }
      }
      lsum[nt] += ls;
      wsum[nt][0] += ws0;
      wsum[nt][1] += ws1;
      bsum[nt][0] += bs0;
      bsum[nt][1] += bs1;
    }
    // P.V: A = V^T tile (16 dims x 32 keys) via one transposed LDS read per dim tile. Source
    // lane s of each 16-lane group addresses key T[s/2] at column offset 8 (s % 2), so result
    // lane i receives keys T[0..7] of dim i.
    const int kslot = lc >> 1;
    const int key = kslot < 4 ? 4 * lq4 + kslot : 16 + 4 * lq4 + (kslot - 4);
    const uint8_t* vrow = wb.v + key * D + 8 * (lc & 1);
    const int vsw7 = key & 7;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const v2i_t raw =
          __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i_t*)(vrow + 16 * (dt ^ vsw7)));
      const half8_t a = codes8_as_h8((uint32_t)raw.x, (uint32_t)raw.y);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        oacc[nt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, wbo[nt][dt >> 2], oacc[nt][dt],
                                                               0, 0, 0);
    }
  };

  // Tile jt + 1's loads are always issued before tile jt is processed (past the last tile they
  // clamp to one cached row and are never used), so the wait is a fixed count: 10 loads.
  issue(0);
  for (int jt = 0; jt < ntiles; ++jt) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer reused next are done
    issue(jt + 1);
    asm volatile("s_waitcnt vmcnt(10)" ::: "memory");   // tile jt has landed in LDS
    process(jt);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // ---- per-wave totals over the 4 lane groups that share a column
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float v[5] = {lsum[nt], wsum[nt][0], wsum[nt][1], bsum[nt][0], bsum[nt][1]};
#pragma unroll
    for (int k = 0; k < 5; ++k) {
      v[k] += shfl_xor_f(v[k], 16);
      v[k] += shfl_xor_f(v[k], 32);
    }
    lsum[nt] = v[0];
    wsum[nt][0] = v[1];
    wsum[nt][1] = v[2];
    bsum[nt][0] = v[3];
    bsum[nt][1] = v[4];
  }
  __syncthreads();  // every wave is done with its LDS tiles before they are reused below
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int col = nt * 16 + lc;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.fin.acc[wv][col][16 * dt + 4 * lq4 + r] = oacc[nt][dt][r];
    if (lq4 == 0) {
      float* st = sm.st[wv][col];
      st[0] = m_run[nt];
      st[1] = lsum[nt];
      st[2] = wsum[nt][0];
      st[3] = wsum[nt][1];
      st[4] = bsum[nt][0];
      st[5] = bsum[nt][1];
    }
  }
  __syncthreads();

  // ---- merge the four waves (log-sum-exp) into the workgroup's partial
  for (int o = tid; o < R * D; o += NTHR) {
    const int col = o / D;
    const int d = o - col * D;
    const int g = d >> 6;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, sm.st[w][col][0]);
    float a = 0.0f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float* st = sm.st[w][col];
      const float e = st[0] == -INFINITY ? 0.0f : exp2f(st[0] - M);
      a += e * ((sm.fin.acc[w][col][d] - 1024.0f * st[2 + g]) + st[4 + g]);
    }
    part_acc[((int64_t)x * Hkv * R + (int64_t)hk * R + col) * D + d] = a;
  }
  if (tid < R) {
    const int col = tid;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) M = fmaxf(M, sm.st[w][col][0]);
    float l = 0.0f;
#pragma unroll
    for (int w = 0; w < NWAVE; ++w) {
      const float* st = sm.st[w][col];
      l += st[0] == -INFINITY ? 0.0f : exp2f(st[0] - M) * st[1];
    }
    part_ml[(int64_t)x * Hkv * R + (int64_t)hk * R + col] = make_float2(M, l);
  }
}

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
  union {
    struct {
      PackBuf buf[NWAVE][2];
      PackTerms terms[NWAVE];
    } loop;
    alignas(16) float acc[NWAVE][4][D];  // wave partials, final merge
  };
  alignas(16) float st[NWAVE][4][6];
};

template <bool CAUSAL>
__global__ __launch_bounds__(NTHR) void q8_attn_packed_kernel(
    AttnArgs args, DecodePlan plan) {
  __shared__ PackSmem sm;
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

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar loop control
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  int b;
  find_seq(plan, x, b);
  const int n = plan.len[b];
  // Work in super-tiles of PST keys. The NWS waves of the sequence's workgroups take about 80%
  // of them statically (wave gw: super-tiles gw + k NWS for k < NS), the rest one at a time from
  // the (sequence, KV head) tile counter, two super-tiles ahead. Waves that started late or sit
  // on busier parts of the chip (XCDs start up to ~3 us apart and differ by ~10% in the
  // bandwidth they get) then take fewer of the dynamic super-tiles.
  const int T = (n + PST - 1) / PST;
  const int NWS = (plan.split_begin[b + 1] - plan.split_begin[b]) * NWAVE;
  const int gw = (x - plan.split_begin[b]) * NWAVE + wv;
  const int NS = max(2, (4 * T) / (5 * NWS));  // static super-tiles per wave
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
  // swizzle read back in process). A full super-tile uses the scalar row base t0 and per-lane
  // offsets that never change; the last one clamps rows to the sequence's last row, and so do
  // super-tiles past the end (their copies land in a buffer that is never read).
  const uint32_t lds_bufs = lds_addr(&sm.loop.buf[wv][0]);
  const uint32_t col_off = (uint32_t)(16 * ((lane & 7) ^ (lane >> 3)));
  uint32_t row_off[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) row_off[u] = (uint32_t)(((lane >> 3) + 8 * u) * D) + col_off;
  auto issue = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * PST;
    const uint32_t lb = lds_bufs + (uint32_t)(BUF * sizeof(PackBuf));
    constexpr int OK = offsetof(PackBuf, k), OV = offsetof(PackBuf, v);
    constexpr int OKS = offsetof(PackBuf, ks), OKB = offsetof(PackBuf, kb);
    constexpr int OVS = offsetof(PackBuf, vs), OVB = offsetof(PackBuf, vb);
    const uint8_t* kb0 = kbase;
    const uint8_t* vb0 = vbase;
    const uint32_t *w0 = ksw, *w1 = kbw, *w2 = vsw, *w3 = vbw;
    uint32_t ro[8], wo;
    if (t0 + PST <= n) {
      kb0 += (int64_t)t0 * D;
      vb0 += (int64_t)t0 * D;
      w0 += t0;
      w1 += t0;
      w2 += t0;
      w3 += t0;
#pragma unroll
      for (int u = 0; u < 8; ++u) ro[u] = row_off[u];
      wo = 4u * (uint32_t)lane;
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u)
        ro[u] = (uint32_t)min(t0 + (lane >> 3) + 8 * u, last_row) * D + col_off;
      wo = 4u * (uint32_t)min(t0 + lane, last_row);
    }
    dma_b128<OK + 0>(kb0, ro[0], lb);
    dma_b128<OV + 0>(vb0, ro[0], lb);
    dma_b128<OK + 1024>(kb0, ro[1], lb);
    dma_b128<OV + 1024>(vb0, ro[1], lb);
    dma_b128<OK + 2048>(kb0, ro[2], lb);
    dma_b128<OV + 2048>(vb0, ro[2], lb);
    dma_b128<OK + 3072>(kb0, ro[3], lb);
    dma_b128<OV + 3072>(vb0, ro[3], lb);
    dma_b128<OK + 4096>(kb0, ro[4], lb);
    dma_b128<OV + 4096>(vb0, ro[4], lb);
    dma_b128<OK + 5120>(kb0, ro[5], lb);
    dma_b128<OV + 5120>(vb0, ro[5], lb);
    dma_b128<OK + 6144>(kb0, ro[6], lb);
    dma_b128<OV + 6144>(vb0, ro[6], lb);
    dma_b128<OK + 7168>(kb0, ro[7], lb);
    dma_b128<OV + 7168>(vb0, ro[7], lb);
    dma_b32<OKS>(w0, wo, lb);
    dma_b32<OKB>(w1, wo, lb);
    dma_b32<OVS>(w2, wo, lb);
    dma_b32<OVB>(w3, wo, lb);
  };

  // Lane masks selecting the P.V B-operand half of K-step e (key tile 2e in slots 0-3, 2e+1 in
  // slots 4-7): this lane's own key tile is mt.
  const uint32_t sel_lo0 = mt == 0 ? ~0u : 0u, sel_hi0 = mt == 1 ? ~0u : 0u;
  const uint32_t sel_lo1 = mt == 2 ? ~0u : 0u, sel_hi1 = mt == 3 ? ~0u : 0u;
  const float kscale = qk_scale_log2 * 16777216.0f;  // 2^24: codes enter the MFMA as c * 2^-24

  auto process = [&](int tile, auto bufc) {
    constexpr int BUF = decltype(bufc)::value;
    const int t0 = tile * PST;
    const PackBuf& pb = sm.loop.buf[wv][BUF];
    // per-key terms, one lane per key: K scale * scale * log2(e) * 2^24, K bias, V scale, V bias
    {
      const uint32_t a = pb.ks[lane], c = pb.kb[lane], e = pb.vs[lane], f = pb.vb[lane];
      tm.ks0[lane] = bf16_lo(a) * kscale;
      tm.ks1[lane] = bf16_hi(a) * kscale;
      tm.ku0[lane] = bf16_lo(c);
      tm.ku1[lane] = bf16_hi(c);
      tm.vs0[lane] = bf16_lo(e);
      tm.vs1[lane] = bf16_hi(e);
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
    tmax = fmaxf(tmax, dpp<DPP_ROW_ROR4>(tmax));
    tmax = fmaxf(tmax, dpp<DPP_ROW_ROR8>(tmax));
    tmax = max_xor16(tmax);
    tmax = max_xor32(tmax);
    const bool bump = tmax > m_run + RESCALE_LOG2;
    if (__builtin_amdgcn_ballot_w64(bump)) {
      const float mn = bump ? tmax : m_run;
      const float alpha = m_run == -INFINITY ? 0.0f : exp2f(m_run - mn);
      m_run = mn;
      lsum *= alpha;
      bsum0 *= alpha;
      bsum1 *= alpha;
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) oacc[dt] *= alpha;
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
    // P * scale_v in fp16, two keys per dword, per quant group
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
  // below keep fixed counts), the old value in lane 0 of the returned VGPR. Inline asm like the
  // copies, so that the compiler inserts no wait for it: `landed` reads it in the same statement
  // as the explicit s_waitcnt that covers it (vector memory operations complete in issue order;
  // each step issues the grab, then the 20 copies of the next super-tile, then waits until only
  // those 20 are outstanding).
  auto grab = [&](bool dyn) {
    uint32_t old;
    uint64_t sv;
    const uint32_t mask = __builtin_amdgcn_readfirstlane(dyn ? 1u : 0u);
    asm volatile("s_mov_b64 %1, exec\n\ts_mov_b32 exec_lo, %5\n\ts_mov_b32 exec_hi, 0\n\t"
                 "global_atomic_add %0, %2, %3, %4 sc0\n\ts_mov_b64 exec, %1"
                 : "=&v"(old), "=&s"(sv)
                 : "v"(ctr_off), "v"(1u), "s"(args.counters), "s"(mask)
                 : "memory");
    return old;
  };
  // Waits for the current super-tile's copies and the grab issued after them (before the next
  // super-tile's copies); returns the index of the wave's super-tile number k2 (that after nxt):
  // static below NS, else the grabbed value past the static ones, clamped to (nxt, T] so that the
  // loop always advances and every copy address stays inside the sequence.
  auto landed = [&](uint32_t g, int k2, int nxt_tile) {
    int v;
    asm volatile("s_waitcnt vmcnt(20)\n\tv_readfirstlane_b32 %0, %1" : "=s"(v) : "v"(g) : "memory");
    const int t = k2 < NS ? gw + k2 * NWS : NS * NWS + v;
    return min(max(t, nxt_tile + 1), T);
  };
  int cur = min(gw, T), nxt = min(gw + NWS, T);  // wave-uniform super-tile indices
  int k = 0;                                      // cur is the wave's super-tile number k
  issue(cur, B0);  // the first super-tile streams in while q is loaded and converted

  // ---- B operands of Q.K^T: q[rho] dims 8 s .. 8 s + 7 when this lane group's tile is mt
  {
    const bool on = qvalid && mt == lq4;
    const uint16_t* qr = q + (((int64_t)b * Hq + hk * G + gh) * L + qi) * D;
    float sg[2] = {0.f, 0.f};
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const uint4 u = *reinterpret_cast<const uint4*>(qr + 8 * st);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const _Float16 lo = (_Float16)bf16_to_f32((uint16_t)(w[j] & 0xffffu));
        const _Float16 hi = (_Float16)bf16_to_f32((uint16_t)(w[j] >> 16));
        qb[st][2 * j] = on ? lo : (_Float16)0.0f;
        qb[st][2 * j + 1] = on ? hi : (_Float16)0.0f;
        sg[st >> 3] += (float)lo + (float)hi;
      }
    }
    qsum[0] = qvalid ? sg[0] * qk_scale_log2 : 0.0f;
    qsum[1] = qvalid ? sg[1] * qk_scale_log2 : 0.0f;
  }
  QPair app_k = {0u, 0, 0}, app_v = {0u, 0, 0};
  uint32_t app_w[4] = {0u, 0u, 0u, 0u};  // ks, kb, vs, vb words of the new row (group 0 low)
  bool patched = false;
  if (app) {
    const int64_t src = ((int64_t)b * Hkv + hk) * D + 2 * lane;
    app_k = quantize_pair_q8(*reinterpret_cast<const uint32_t*>(args.knew + src));
    app_v = quantize_pair_q8(*reinterpret_cast<const uint32_t*>(args.vnew + src));
    const uint16_t hv[4] = {app_k.scale, app_k.bias, app_v.scale, app_v.bias};
#pragma unroll
    for (int j = 0; j < 4; ++j)
      app_w[j] = (uint32_t)__builtin_amdgcn_readlane((int)hv[j], 0) |
                 ((uint32_t)__builtin_amdgcn_readlane((int)hv[j], 32) << 16);
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

  // Unrolled by two so that each buffer's LDS offsets are constants. The next super-tile is
  // always issued before the current one is processed (past the end the copies clamp to the last
  // row and are never read), so the wait is a fixed count: the 20 copies of the next super-tile,
  // issued after the current one's copies and after the grab of the one after next.
  for (;;) {
    if (cur >= T) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // reads of the buffer reused next are done
    uint32_t grabbed = grab(k + 2 >= NS);
    issue(nxt, B1);
    int after = landed(grabbed, k + 2, nxt);  // super-tile cur and the grab have landed
    if (cur == app_t) {
      patch(B0);
      patched = true;
    }
    process(cur, B0);
    cur = nxt;
    nxt = after;
    ++k;
    if (cur >= T) break;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    grabbed = grab(k + 2 >= NS);
    issue(nxt, B0);
    after = landed(grabbed, k + 2, nxt);
    if (cur == app_t) {
      patch(B1);
      patched = true;
    }
    process(cur, B1);
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

  __syncthreads();  // every wave is done with its LDS tiles before they are reused below
  packed_finish<NWAVE>(oacc, m_run, lsum, bsum0, bsum1, 16777216.0f, &sm.acc[0][0][0],
                       &sm.st[0][0][0], &sh_last, args, plan, x, b, hk, R);
}

}  // namespace

QAttnFn q8_attn_fn(int nt, bool causal) {
  if (nt == 0) return causal ? q8_attn_packed_kernel<true> : q8_attn_packed_kernel<false>;
  if (causal) {
    switch (nt) {
      case 1: return q8_attn_mfma_kernel<1, true>;
      case 2: return q8_attn_mfma_kernel<2, true>;
      case 3: return q8_attn_mfma_kernel<3, true>;
      case 4: return q8_attn_mfma_kernel<4, true>;
    }
  } else {
    switch (nt) {
      case 1: return q8_attn_mfma_kernel<1, false>;
      case 2: return q8_attn_mfma_kernel<2, false>;
      case 3: return q8_attn_mfma_kernel<3, false>;
      case 4: return q8_attn_mfma_kernel<4, false>;
    }
  }
  return nullptr;
}

}  // namespace lq
