// Fused single-token decode attention over the quantized KV cache (split-K flash-decoding).
//
// Replaces q8_decode_attention (laguna_mlx/q8_attn.py:102-130): the Metal kernel that reads the
// packed cache once, dequantizes in registers and keeps an online softmax per block of keys
// (:17-99), and the log-sum-exp merge of the block partials (:126-130).
//
// CDNA4 design (not a translation of the Metal kernel's lane layout):
//  * Grid (split, kv head). Each workgroup (4 wave64s) owns a contiguous range of `chunk` keys of
//    one sequence and one KV head and serves all G query heads of that KV head, so every K/V
//    byte is read from HBM exactly once. `chunk` is chosen so that the grid fills every CU with
//    as many resident workgroups as the occupancy allows (one wave of workgroups, no tail).
//  * Inside a workgroup two producer waves compute the scores of key tile j (128 rows) while two
//    consumer waves run the softmax and P.V of tile j-1; the score tiles are double-buffered in
//    LDS, one barrier per tile. Splitting the roles keeps either role's registers (q in the
//    producers, the output accumulator in the consumers) out of the other's wave.
//  * Producers: 4 lanes per key row, each lane loads its 32 codes with two 128-bit loads and
//    computes the G partial dot products with v_dot2_f32_f16 on (1024 + code) fp16 pairs built
//    with one v_perm_b32 per pair. The affine terms are folded out of the inner loop:
//    q.(s c + b) = s (q.(1024 + c)) + (b - 1024 s) sum(q); the 4-lane sum is two DPP adds.
//    Scores are stored already multiplied by scale * log2(e).
//  * Consumers: each consumer wave keeps its own running max over its 64 rows of every tile
//    (wave-wide DPP max), p = exp2(s - m), and stores the V weights p * scale_v as fp16 pairs of
//    two rows in wave-private LDS. P.V: 8 lanes per row pair (16 dims each), one v_perm
//    interleave per 4-byte word pair and one v_perm per (row pair, dim), then v_dot2_f32_f16 for
//    the G heads; the bias term sum p * bias_v and the 1024 offset are accumulated per row, not
//    per element.
//  * The two consumer waves are merged by log-sum-exp at the end; partials (m, l, acc[128]) per
//    (split, query head) go to the workspace and a second kernel does the per-sequence merge.
#include "common.h"

namespace lq {
namespace {

constexpr int D = 128;
constexpr int NT = 256;       // threads per workgroup
constexpr int MIN_CHUNK = 128;

struct DecodePlan {
  int32_t nseq;
  int32_t chunk;
  int32_t split_begin[LQ_MAX_SEQS + 1];  // first global split of each sequence
  int32_t len[LQ_MAX_SEQS];
};

__device__ __forceinline__ void find_seq(const DecodePlan& plan, int x, int& b) {
  b = 0;
  for (int i = 1; i < plan.nseq; ++i)
    if (x >= plan.split_begin[i]) b = i;
}

// ----------------------------------------------------------------------------------------------
// q8 split kernel: 2 producer waves (K scores) + 2 consumer waves (softmax, P.V), pipelined over
// tiles of 128 key rows through double-buffered LDS score tiles.
// ----------------------------------------------------------------------------------------------

constexpr int KT = 128;  // key rows per pipeline tile (64 per wave of each role)

template <int G>
struct Q8Smem {
  float s[2][KT][G];            // scores (log2 domain), double buffered
  half2_t w[2][32][2][G];       // per consumer wave: [row pair][group][head] = (w_row0, w_row1)
  float fin[2][G][D];           // consumer-wave partial acc, summed over its rows
  float fsum[2][G][6];          // consumer-wave m, l, wsum[2], bsum[2]
};

template <int G>
__global__ __launch_bounds__(NT) void q8_decode_split_kernel(
    const uint16_t* __restrict__ q, const uint8_t* __restrict__ kc,
    const uint16_t* __restrict__ ks, const uint16_t* __restrict__ kb,
    const uint8_t* __restrict__ vc, const uint16_t* __restrict__ vs,
    const uint16_t* __restrict__ vb, int Hkv, int64_t cap, float qk_scale_log2,
    DecodePlan plan, float* __restrict__ part_acc, float2* __restrict__ part_ml) {
  __shared__ Q8Smem<G> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;          // 0,1: producers; 2,3: consumers
  const int x = blockIdx.x;
  const int hk = blockIdx.y;
  int b;
  find_seq(plan, x, b);
  const int n = plan.len[b];
  const int t_begin = (x - plan.split_begin[b]) * plan.chunk;
  const int t_end = min(t_begin + plan.chunk, n);
  const int ntiles = (t_end - t_begin + KT - 1) / KT;
  const int Hq = Hkv * G;
  const int64_t bh = (int64_t)b * Hkv + hk;
  const int64_t row0 = bh * cap;  // cache row of token 0

  if (wv < 2) {
    // ================================ producer: K scores ====================================
    // 4 lanes per key row; lane owns dims [32*rl, 32*rl+32), all in group rl/2.
    const int rl = lane & 3;
    const int rsub = lane >> 2;
    const int kgrp = rl >> 1;
    half2_t qh[G][16];
    float qsum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const uint4* q4 =
          reinterpret_cast<const uint4*>(q + ((int64_t)b * Hq + hk * G + h) * D + 32 * rl);
      float a = 0.0f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const uint4 u = q4[v];
        const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const _Float16 lo = (_Float16)bf16_to_f32((uint16_t)(wd[j] & 0xffffu));
          const _Float16 hi = (_Float16)bf16_to_f32((uint16_t)(wd[j] >> 16));
          qh[h][4 * v + j] = half2_t{lo, hi};
          a += (float)lo + (float)hi;
        }
      }
      qsum[h] = a;
    }
    const uint8_t* kbase = kc + row0 * D + 32 * rl;
    // scale/bias of both groups of a row as one 32-bit word (group kgrp picked at use)
    const uint32_t* ksw = reinterpret_cast<const uint32_t*>(ks + row0 * 2);
    const uint32_t* kbw = reinterpret_cast<const uint32_t*>(kb + row0 * 2);
    const int kshift = 16 * kgrp;

    // Branch-free loads (rows past the tile end are clamped to its last row and masked later),
    // issued one tile ahead of their use so every wave keeps a tile of loads in flight.
    uint4 ca[4], cb[4];
    uint32_t sraw[4], braw[4];
    auto load_tile = [&](int jt, uint4* xa, uint4* xb, uint32_t* xs, uint32_t* xbias) {
      const int t0 = t_begin + jt * KT;
      const int last = min(KT, t_end - t0) - 1;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = t0 + min(64 * wv + 16 * i + rsub, last);
        xs[i] = ksw[t];
        xbias[i] = kbw[t];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = t0 + min(64 * wv + 16 * i + rsub, last);
        const uint4* p = reinterpret_cast<const uint4*>(kbase + t * D);
        xa[i] = p[0];
        xb[i] = p[1];
      }
    };
    load_tile(0, ca, cb, sraw, braw);

    // One pipeline step: prefetch tile j+1 into (xa..), score tile j from (ya..), barrier.
    auto step = [&](int j, const uint4* ya, const uint4* yb, const uint32_t* ys,
                    const uint32_t* ybias, uint4* xa, uint4* xb, uint32_t* xs, uint32_t* xbias) {
      if (j + 1 < ntiles) load_tile(j + 1, xa, xb, xs, xbias);
      if (j < ntiles) {
        const int t0 = t_begin + j * KT;
        const int rows = min(KT, t_end - t0);
        float(*S)[G] = sm.s[j & 1];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 64 * wv + 16 * i + rsub;
          const uint32_t wd[8] = {ya[i].x, ya[i].y, ya[i].z, ya[i].w,
                                  yb[i].x, yb[i].y, yb[i].z, yb[i].w};
          float dacc[G];
#pragma unroll
          for (int h = 0; h < G; ++h) dacc[h] = 0.0f;
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            const half2_t lo = codes_as_h2(wd[k], SEL_B01);
            const half2_t hi = codes_as_h2(wd[k], SEL_B23);
#pragma unroll
            for (int h = 0; h < G; ++h) {
              dacc[h] = dot2(qh[h][2 * k], lo, dacc[h]);
              dacc[h] = dot2(qh[h][2 * k + 1], hi, dacc[h]);
            }
          }
          // q.(s c + b) = s (q.(1024 + c)) + (b - 1024 s) sum(q), times scale*log2(e)
          const float sc = bf16_to_f32((uint16_t)(ys[i] >> kshift));
          const float bi = bf16_to_f32((uint16_t)(ybias[i] >> kshift));
          const float s1 = sc * qk_scale_log2;
          const float u1 = (bi - 1024.0f * sc) * qk_scale_log2;
#pragma unroll
          for (int h = 0; h < G; ++h) {
            const float part = quad_sum(s1 * dacc[h] + u1 * qsum[h]);
            if ((h & 3) == rl) S[r][h] = r < rows ? part : -INFINITY;
          }
        }
      }
      __syncthreads();
    };
    uint4 na[4], nb[4];
    uint32_t ns[4], nbias[4];
    for (int j = 0; j <= ntiles; j += 2) {
      step(j, ca, cb, sraw, braw, na, nb, ns, nbias);
      if (j + 1 <= ntiles) step(j + 1, na, nb, ns, nbias, ca, cb, sraw, braw);
    }
  } else {
    // ================================ consumer: softmax + P.V ==============================
    const int cw = wv - 2;  // consumer wave: rows [64*cw, 64*cw+64) of each tile
    // P.V role: 8 lanes per row pair, lane owns dims [16*vl, 16*vl+16)
    const int vl = lane & 7;
    const int rs = lane >> 3;
    const int vgrp = vl >> 2;
    // softmax role: lane -> (row pair sp, group sg)
    const int sp = lane >> 1;
    const int sg = lane & 1;
    const int sr0 = 64 * cw + 16 * (sp >> 3) + (sp & 7);
    const int sr1 = sr0 + 8;

    float acc[G][16];
    float m_run[G], lsum[G], wsum[G], bsum[G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int d = 0; d < 16; ++d) acc[h][d] = 0.0f;
      m_run[h] = -INFINITY;
      lsum[h] = wsum[h] = bsum[h] = 0.0f;
    }
    const uint8_t* vbase = vc + row0 * D + 16 * vl;
    const uint32_t* vsw = reinterpret_cast<const uint32_t*>(vs + row0 * 2);
    const uint32_t* vbw = reinterpret_cast<const uint32_t*>(vb + row0 * 2);
    const int vshift = 16 * sg;
    half2_t(*W)[2][G] = sm.w[cw];

    // V codes of 4 row pairs per lane plus the softmax rows' V scale/bias, loaded branch-free
    // (rows clamped to the tile's last row) one tile ahead of their use.
    uint4 ca[4], cb[4];
    uint32_t vraw[4];  // scale and bias words (both groups) of rows sr0, sr1
    auto load_tile = [&](int jt, uint4* xa, uint4* xb, uint32_t* xr) {
      const int t0 = t_begin + jt * KT;
      const int last = min(KT, t_end - t0) - 1;
      const int64_t u0 = t0 + min(sr0, last), u1 = t0 + min(sr1, last);
      xr[0] = vsw[u0];
      xr[1] = vsw[u1];
      xr[2] = vbw[u0];
      xr[3] = vbw[u1];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r0 = min(64 * cw + 16 * i + rs, last);
        const int r1 = min(64 * cw + 16 * i + rs + 8, last);
        xa[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)(t0 + r0) * D);
        xb[i] = *reinterpret_cast<const uint4*>(vbase + (int64_t)(t0 + r1) * D);
      }
    };
    if (ntiles > 0) load_tile(0, ca, cb, vraw);

    // One pipeline step: prefetch tile j into (xa..), softmax + P.V of tile j-1 from (ya..).
    auto step = [&](int j, const uint4* ya, const uint4* yb, const uint32_t* yr, uint4* xa,
                    uint4* xb, uint32_t* xr) {
      if (j >= 1) {
        const int jt = j - 1;
        const int t0 = t_begin + jt * KT;
        const int rows = min(KT, t_end - t0);
        if (j < ntiles) load_tile(j, xa, xb, xr);
        // softmax over this wave's 64 rows
        const float(*S)[G] = sm.s[jt & 1];
        const bool ok0 = sr0 < rows, ok1 = sr1 < rows;
        const float vs0 = ok0 ? bf16_to_f32((uint16_t)(yr[0] >> vshift)) : 0.0f;
        const float vs1 = ok1 ? bf16_to_f32((uint16_t)(yr[1] >> vshift)) : 0.0f;
        const float vb0 = ok0 ? bf16_to_f32((uint16_t)(yr[2] >> vshift)) : 0.0f;
        const float vb1 = ok1 ? bf16_to_f32((uint16_t)(yr[3] >> vshift)) : 0.0f;
        float alpha[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
          const float s0 = S[sr0][h];
          const float s1 = S[sr1][h];
          const float mn = fmaxf(m_run[h], wave_max(fmaxf(s0, s1)));
          const float mref = mn == -INFINITY ? 0.0f : mn;  // a wave with no valid row yet
          alpha[h] = exp2f(m_run[h] - mref);
          m_run[h] = mn;
          const float p0 = exp2f(s0 - mref);
          const float p1 = exp2f(s1 - mref);
          const half2_t w = half2_t{(_Float16)(p0 * vs0), (_Float16)(p1 * vs1)};
          W[sp][sg][h] = w;
          lsum[h] = alpha[h] * lsum[h] + (sg == 0 ? p0 + p1 : 0.0f);
          wsum[h] = alpha[h] * wsum[h] + ((float)w.x + (float)w.y);
          bsum[h] = alpha[h] * bsum[h] + (p0 * vb0 + p1 * vb1);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int h = 0; h < G; ++h)
#pragma unroll
          for (int d = 0; d < 16; ++d) acc[h][d] *= alpha[h];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // rows past the tile end carry weight 0 (their scores are -inf)
          half2_t wt[G];
#pragma unroll
          for (int h = 0; h < G; ++h) wt[h] = W[8 * i + rs][vgrp][h];
          const uint32_t w0[4] = {ya[i].x, ya[i].y, ya[i].z, ya[i].w};
          const uint32_t w1[4] = {yb[i].x, yb[i].y, yb[i].z, yb[i].w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            // interleave two rows' bytes: xl = (a0, b0, a1, b1), xh = (a2, b2, a3, b3)
            const uint32_t xl = __builtin_amdgcn_perm(w1[k], w0[k], 0x05010400u);
            const uint32_t xh = __builtin_amdgcn_perm(w1[k], w0[k], 0x07030602u);
            const half2_t c0 = codes_as_h2(xl, SEL_B01);
            const half2_t c1 = codes_as_h2(xl, SEL_B23);
            const half2_t c2 = codes_as_h2(xh, SEL_B01);
            const half2_t c3 = codes_as_h2(xh, SEL_B23);
#pragma unroll
            for (int h = 0; h < G; ++h) {
              acc[h][4 * k + 0] = dot2(wt[h], c0, acc[h][4 * k + 0]);
              acc[h][4 * k + 1] = dot2(wt[h], c1, acc[h][4 * k + 1]);
              acc[h][4 * k + 2] = dot2(wt[h], c2, acc[h][4 * k + 2]);
              acc[h][4 * k + 3] = dot2(wt[h], c3, acc[h][4 * k + 3]);
            }
          }
        }
      }
      __syncthreads();
    };
    uint4 na[4], nb[4];
    uint32_t nr[4];
    // iteration j consumes the buffer tile j-1 was loaded into: tile t lives in (ca..) for even
    // t and in (na..) for odd t
    for (int j = 0; j <= ntiles; j += 2) {
      step(j, na, nb, nr, ca, cb, vraw);  // j even: consumes tile j-1 (odd), loads tile j (even)
      if (j + 1 <= ntiles) step(j + 1, ca, cb, vraw, na, nb, nr);
    }

    // ---- consumer wave partial: sum acc over the 8 row slots, the softmax sums over lanes
#pragma unroll
    for (int h = 0; h < G; ++h)
#pragma unroll
      for (int d = 0; d < 16; ++d) {
        float v = acc[h][d];
        v += dpp<DPP_ROW_ROR8>(v);
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        acc[h][d] = v;
      }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      const float l = wave_sum(lsum[h]);
      // wsum/bsum: even lanes hold group 0, odd lanes group 1; sum over lanes of equal parity
      float ws = wsum[h], bs = bsum[h];
      ws += dpp<DPP_QUAD_XOR2>(ws);
      bs += dpp<DPP_QUAD_XOR2>(bs);
      ws += dpp<DPP_ROW_ROR4>(ws);
      bs += dpp<DPP_ROW_ROR4>(bs);
      ws += dpp<DPP_ROW_ROR8>(ws);
      bs += dpp<DPP_ROW_ROR8>(bs);
      ws += __shfl_xor(ws, 16, 64);
      bs += __shfl_xor(bs, 16, 64);
      ws += __shfl_xor(ws, 32, 64);
      bs += __shfl_xor(bs, 32, 64);
      if (lane < 2) {
        sm.fsum[cw][h][2 + lane] = ws;
        sm.fsum[cw][h][4 + lane] = bs;
      }
      if (lane == 0) {
        sm.fsum[cw][h][0] = m_run[h];
        sm.fsum[cw][h][1] = l;
      }
    }
    if (rs == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h)
#pragma unroll
        for (int d = 0; d < 16; ++d) sm.fin[cw][h][16 * vl + d] = acc[h][d];
    }
  }
  __syncthreads();

  // ---- merge the two consumer waves (log-sum-exp) into the split's partial:
  //   acc[d] = sum_t w_t (1024 + c_td) - 1024 sum_t w_t + sum_t p_t bias_t   (group of d)
  for (int o = tid; o < G * D; o += NT) {
    const int h = o / D;
    const int d = o - h * D;
    const int g = d >> 6;
    const float m0 = sm.fsum[0][h][0], m1 = sm.fsum[1][h][0];
    const float M = fmaxf(m0, m1);
    const float e0 = exp2f(m0 - M), e1 = exp2f(m1 - M);
    const float v0 = (sm.fin[0][h][d] - 1024.0f * sm.fsum[0][h][2 + g]) + sm.fsum[0][h][4 + g];
    const float v1 = (sm.fin[1][h][d] - 1024.0f * sm.fsum[1][h][2 + g]) + sm.fsum[1][h][4 + g];
    part_acc[((int64_t)x * Hq + hk * G + h) * D + d] = e0 * v0 + e1 * v1;
  }
  if (tid < G) {
    const int h = tid;
    const float m0 = sm.fsum[0][h][0], m1 = sm.fsum[1][h][0];
    const float M = fmaxf(m0, m1);
    part_ml[(int64_t)x * Hq + hk * G + h] =
        make_float2(M, exp2f(m0 - M) * sm.fsum[0][h][1] + exp2f(m1 - M) * sm.fsum[1][h][1]);
  }
}

// ----------------------------------------------------------------------------------------------
// merge kernel: one workgroup per (sequence, query head), one thread per dim
// ----------------------------------------------------------------------------------------------

__global__ __launch_bounds__(D) void decode_merge_kernel(const float* __restrict__ part_acc,
                                                         const float2* __restrict__ part_ml,
                                                         int Hq, DecodePlan plan,
                                                         uint16_t* __restrict__ out) {
  constexpr int MAXS = 1024;  // splits merged per pass through LDS
  __shared__ float wsh[MAXS];
  __shared__ float red[2];
  const int bq = blockIdx.x;
  const int b = bq / Hq;
  const int hq = bq - b * Hq;
  const int d = threadIdx.x;
  const int s0 = plan.split_begin[b], s1 = plan.split_begin[b + 1];
  // global max over the sequence's splits: all threads load (m, l) in parallel
  float M = -INFINITY;
  for (int s = s0 + d; s < s1; s += D) M = fmaxf(M, part_ml[(int64_t)s * Hq + hq].x);
  M = wave_max(M);
  if ((d & 63) == 0) red[d >> 6] = M;
  __syncthreads();
  M = fmaxf(red[0], red[1]);
  float num = 0.0f, den = 0.0f;
  for (int c0 = s0; c0 < s1; c0 += MAXS) {
    const int c1 = min(s1, c0 + MAXS);
    __syncthreads();
    for (int s = c0 + d; s < c1; s += D) {
      const float2 ml = part_ml[(int64_t)s * Hq + hq];
      const float w = exp2f(ml.x - M);
      wsh[s - c0] = w;
      den += w * ml.y;
    }
    __syncthreads();
    const float* pa = part_acc + ((int64_t)c0 * Hq + hq) * D + d;
    const int cnt = c1 - c0;
    int s = 0;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    for (; s + 4 <= cnt; s += 4) {
      a0 += wsh[s] * pa[(int64_t)s * Hq * D];
      a1 += wsh[s + 1] * pa[(int64_t)(s + 1) * Hq * D];
      a2 += wsh[s + 2] * pa[(int64_t)(s + 2) * Hq * D];
      a3 += wsh[s + 3] * pa[(int64_t)(s + 3) * Hq * D];
    }
    for (; s < cnt; ++s) a0 += wsh[s] * pa[(int64_t)s * Hq * D];
    num += (a0 + a1) + (a2 + a3);
  }
  // den: each thread summed a strided subset of the splits
  den = wave_sum(den);
  __syncthreads();
  if ((d & 63) == 0) red[d >> 6] = den;
  __syncthreads();
  den = red[0] + red[1];
  out[((int64_t)b * Hq + hq) * D + d] = f32_to_bf16(num / den);
}

// ----------------------------------------------------------------------------------------------
// host side
// ----------------------------------------------------------------------------------------------

typedef void (*SplitFn)(const uint16_t*, const uint8_t*, const uint16_t*, const uint16_t*,
                        const uint8_t*, const uint16_t*, const uint16_t*, int, int64_t, float,
                        DecodePlan, float*, float2*);

SplitFn q8_split_fn(int G) {
  switch (G) {
    case 1: return q8_decode_split_kernel<1>;
    case 2: return q8_decode_split_kernel<2>;
    case 3: return q8_decode_split_kernel<3>;
    case 4: return q8_decode_split_kernel<4>;
    case 5: return q8_decode_split_kernel<5>;
    case 6: return q8_decode_split_kernel<6>;
    case 7: return q8_decode_split_kernel<7>;
    case 8: return q8_decode_split_kernel<8>;
  }
  return nullptr;
}

// Resident workgroups per CU for a split kernel (cached; queried once per kernel).
int split_occupancy(SplitFn fn) {
  static SplitFn fns[16];
  static int occ[16];
  static int nf = 0;
  for (int i = 0; i < nf; ++i)
    if (fns[i] == fn) return occ[i];
  int k = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&k, reinterpret_cast<const void*>(fn), NT, 0) !=
          hipSuccess ||
      k < 1)
    k = 2;
  if (nf < 16) {
    fns[nf] = fn;
    occ[nf] = k;
    ++nf;
  }
  return k;
}

// Builds the split plan. Returns total splits, or -1 on bad lengths.
int64_t make_plan(int64_t B, int64_t Hkv, int64_t n, const int32_t* lens, int64_t cap,
                  int wgs_target, DecodePlan& plan) {
  if (B < 1 || B > LQ_MAX_SEQS) return -1;
  int64_t total = 0;
  for (int64_t b = 0; b < B; ++b) {
    const int64_t l = lens ? lens[b] : n;
    if (l < 1 || (cap > 0 && l > cap)) return -1;
    plan.len[b] = (int32_t)l;
    total += l;
  }
  const int64_t per_head = std::max<int64_t>(1, wgs_target / Hkv);
  int64_t chunk = (total + per_head - 1) / per_head;
  chunk = std::max<int64_t>(chunk, MIN_CHUNK);
  chunk = (chunk + 15) / 16 * 16;
  plan.nseq = (int32_t)B;
  plan.chunk = (int32_t)chunk;
  int64_t s = 0;
  for (int64_t b = 0; b < B; ++b) {
    plan.split_begin[b] = (int32_t)s;
    s += (plan.len[b] + chunk - 1) / chunk;
  }
  plan.split_begin[B] = (int32_t)s;
  return s;
}

int wgs_target_for(int G) {
  SplitFn fn = q8_split_fn(G);
  return split_occupancy(fn) * device_cu_count();
}

}  // namespace
}  // namespace lq

extern "C" int64_t lq_decode_workspace_bytes(int kind, int64_t B, int64_t Hq, int64_t Hkv,
                                             int64_t D, int64_t n, const int32_t* lens_host) {
  using namespace lq;
  clear_error();
  if (kind != LQ_KV_Q8 || D != 128 || Hkv < 1 || Hq % Hkv || Hq / Hkv > 8) {
    set_error("unsupported decode configuration");
    return -1;
  }
  DecodePlan plan;
  const int64_t S = make_plan(B, Hkv, n, lens_host, 0, wgs_target_for((int)(Hq / Hkv)), plan);
  if (S < 0) {
    set_error("bad sequence lengths");
    return -1;
  }
  return S * Hq * (int64_t)(D * sizeof(float) + sizeof(float2));
}

extern "C" int lq_decode_attn(int kind, const uint16_t* q, const void* kc, const uint16_t* ks,
                              const uint16_t* kb, const void* vc, const uint16_t* vs,
                              const uint16_t* vb, int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                              int64_t cap, int64_t n, const int32_t* lens_host, float scale,
                              uint16_t* out, void* workspace, int64_t workspace_bytes,
                              void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(kind == LQ_KV_Q8, "kv kind %d not supported", kind);
  LQ_CHECK_ARG(D == 128, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(Hkv >= 1 && Hq >= Hkv && Hq % Hkv == 0, "Hq=%lld must be a multiple of Hkv=%lld",
               (long long)Hq, (long long)Hkv);
  LQ_CHECK_ARG(Hq / Hkv <= 8, "at most 8 query heads per KV head (got %lld)", (long long)(Hq / Hkv));
  LQ_CHECK_ARG(B >= 1 && B <= LQ_MAX_SEQS, "batch %lld outside [1, %d]", (long long)B, LQ_MAX_SEQS);
  LQ_CHECK_ARG(cap >= 1 && cap <= INT32_MAX, "bad capacity %lld", (long long)cap);
  LQ_CHECK_ARG(q && kc && ks && kb && vc && vs && vb && out, "null pointer");
  const int G = (int)(Hq / Hkv);
  DecodePlan plan;
  const int64_t S = make_plan(B, Hkv, n, lens_host, cap, wgs_target_for(G), plan);
  LQ_CHECK_ARG(S > 0, "sequence lengths must be in [1, cap=%lld]", (long long)cap);
  const int64_t need = S * Hq * (int64_t)(D * sizeof(float) + sizeof(float2));
  if (!workspace || workspace_bytes < need) {
    set_error("workspace of %lld bytes is smaller than the %lld needed", (long long)workspace_bytes,
              (long long)need);
    return LQ_EWORKSPACE;
  }
  float* part_acc = reinterpret_cast<float*>(workspace);
  float2* part_ml = reinterpret_cast<float2*>(part_acc + S * Hq * D);
  hipStream_t st = (hipStream_t)stream;
  const float qk = scale * 1.4426950408889634f;
  SplitFn fn = q8_split_fn(G);
  hipLaunchKernelGGL(fn, dim3((unsigned)S, (unsigned)Hkv), dim3(NT), 0, st, q,
                     (const uint8_t*)kc, ks, kb, (const uint8_t*)vc, vs, vb, (int)Hkv, cap, qk,
                     plan, part_acc, part_ml);
  LQ_CHECK_LAUNCH("q8_decode_split_kernel");
  decode_merge_kernel<<<dim3((unsigned)(B * Hq)), dim3(D), 0, st>>>(part_acc, part_ml, (int)Hq,
                                                                      plan, out);
  LQ_CHECK_LAUNCH("decode_merge_kernel");
  return LQ_OK;
}
