// The decoder-layer operations around the cache in the attention block of a full-attention layer
// (laguna_mlx/laguna.py:94-111): q/k RMSNorm + RoPE at the cache offset before update_and_fetch,
// and the softplus output gate after attention.
//
// lq_qk_norm_rope replaces q_norm/k_norm (nn.RMSNorm over head_dim, laguna.py:89-90,97-98) and
// the rope calls (laguna.py:100-101; mlx-lm's initialize_rope: default or YaRN frequencies,
// partial rotary): one wave per (head, row), lane l holding dims 2l and 2l + 1 (head_dim 128).
// The normalized row is rounded to bf16 before the rotation, as the reference's two separate
// ops round between them. The rotation is the non-interleaved form on the first `rot_dims` dims:
// dim i pairs with dim i + rot_dims / 2, angle (position) * inv_freq[i]; the partner value sits
// rot_dims / 4 lanes away. `mscale` (YaRN's attention factor) scales the rotated dims.
//
// lq_gate_heads replaces `out.transpose(0, 2, 1, 3) * softplus(g_proj(x))` (laguna.py:108-110):
// the gate in fp32, rounded to bf16 like the reference's astype, the product rounded to bf16, and
// the result written in o_proj's [B, L, Hq, D] layout (the transpose folded into the store).
#include "common.h"

namespace lq {
namespace {

constexpr int ND = 128;  // head_dim

__global__ __launch_bounds__(256) void qk_norm_rope_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out, const uint16_t* __restrict__ q_w,
    const uint16_t* __restrict__ k_w, int64_t B, int Hq, int Hkv, int64_t L, float eps,
    const float* __restrict__ inv_freq, int rot_dims, float mscale, int64_t offset,
    const int32_t* __restrict__ offsets) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // over B (Hq + Hkv) L
  const int64_t per_b = (int64_t)(Hq + Hkv) * L;
  if (row >= B * per_b) return;  // wave-uniform
  const int64_t b = row / per_b;
  const int64_t r = row - b * per_b;
  const bool is_q = r < (int64_t)Hq * L;
  const int64_t hr = is_q ? r : r - (int64_t)Hq * L;  // head * L + l within q or k
  const int64_t l = hr % L;
  const int64_t src_row = (b * (is_q ? Hq : Hkv)) * L + hr;
  const uint16_t* in = (is_q ? q : k) + src_row * ND;
  uint16_t* out = (is_q ? q_out : k_out) + src_row * ND;
  const uint16_t* w = is_q ? q_w : k_w;
  const float pos = (float)((offsets ? (int64_t)offsets[b] : offset) + l);
  reinterpret_cast<uint32_t*>(out)[lane] =
      norm_rope_lane(reinterpret_cast<const uint32_t*>(in)[lane],
                     reinterpret_cast<const uint32_t*>(w)[lane], lane, eps, inv_freq, rot_dims,
                     mscale, pos);
}

// softplus(x) = log(1 + e^x), written as max(x, 0) + log1p(e^-|x|) (no overflow for large x)
__device__ __forceinline__ float softplus_f(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

// One thread per 8 dims of one (b, h, l) row of attn [B, Hq, L, D]; gate g is [B, L, Hq] (per
// head) or [B, L, Hq, D] (per dim).
__global__ __launch_bounds__(256) void gate_heads_kernel(const uint16_t* __restrict__ attn,
                                                         const uint16_t* __restrict__ g,
                                                         uint16_t* __restrict__ out, int64_t B,
                                                         int Hq, int64_t L, int per_dim) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = B * Hq * L * (ND / 8);
  if (t >= total) return;
  const int c = (int)(t % (ND / 8));
  const int64_t rowi = t / (ND / 8);  // (b, h, l) in attn order
  const int64_t l = rowi % L;
  const int64_t bh = rowi / L;
  const int h = (int)(bh % Hq);
  const int64_t b = bh / Hq;
  const uint4 a = reinterpret_cast<const uint4*>(attn + rowi * ND)[c];
  const int64_t orow = (b * L + l) * Hq + h;  // row of out [B, L, Hq, D] and of a per-dim gate
  uint32_t aw[4] = {a.x, a.y, a.z, a.w}, ow[4];
  if (per_dim) {
    const uint4 gv = reinterpret_cast<const uint4*>(g + orow * ND)[c];
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float g0 = bf16_to_f32(f32_to_bf16(softplus_f(bf16_lo(gw[j]))));
      const float g1 = bf16_to_f32(f32_to_bf16(softplus_f(bf16_hi(gw[j]))));
      ow[j] = (uint32_t)f32_to_bf16(bf16_lo(aw[j]) * g0) |
              ((uint32_t)f32_to_bf16(bf16_hi(aw[j]) * g1) << 16);
    }
  } else {
    const float gate = bf16_to_f32(f32_to_bf16(softplus_f(bf16_to_f32(g[orow]))));
#pragma unroll
    for (int j = 0; j < 4; ++j)
      ow[j] = (uint32_t)f32_to_bf16(bf16_lo(aw[j]) * gate) |
              ((uint32_t)f32_to_bf16(bf16_hi(aw[j]) * gate) << 16);
  }
  reinterpret_cast<uint4*>(out + orow * ND)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
}

// Residual add + RMSNorm over rows of C (<= 8192, multiple of 8) bf16 values, one workgroup per
// row, 8 values per thread: h_out = bf16(h + d) (d may be null: h_out = h), y = bf16(rms(h_out) w).
__global__ __launch_bounds__(256) void add_rms_norm_kernel(const uint16_t* h,
                                                           const uint16_t* __restrict__ d,
                                                           const uint16_t* __restrict__ w,
                                                           uint16_t* h_out,  // may alias h
                                                           uint16_t* __restrict__ y, int C,
                                                           float eps) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const int chunks = C / 8;
  float v[4][8];
  float ss = 0.0f;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = tid + 256 * it;
    if (c < chunks) {
      const uint4 a = reinterpret_cast<const uint4*>(h + row * C)[c];
      uint4 bb = make_uint4(0u, 0u, 0u, 0u);
      if (d) bb = reinterpret_cast<const uint4*>(d + row * C)[c];
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {bb.x, bb.y, bb.z, bb.w};
      uint32_t ow[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint16_t lo = d ? f32_to_bf16(bf16_lo(aw[j]) + bf16_lo(bw[j])) : (uint16_t)(aw[j] & 0xffffu);
        const uint16_t hi = d ? f32_to_bf16(bf16_hi(aw[j]) + bf16_hi(bw[j])) : (uint16_t)(aw[j] >> 16);
        v[it][2 * j] = bf16_to_f32(lo);
        v[it][2 * j + 1] = bf16_to_f32(hi);
        ow[j] = (uint32_t)lo | ((uint32_t)hi << 16);
        ss += v[it][2 * j] * v[it][2 * j] + v[it][2 * j + 1] * v[it][2 * j + 1];
      }
      if (d) reinterpret_cast<uint4*>(h_out + row * C)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)C + eps);
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int c = tid + 256 * it;
    if (c < chunks) {
      const uint4 wv = reinterpret_cast<const uint4*>(w)[c];
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t ow[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ow[j] = (uint32_t)f32_to_bf16(v[it][2 * j] * inv * bf16_lo(ww[j])) |
                ((uint32_t)f32_to_bf16(v[it][2 * j + 1] * inv * bf16_hi(ww[j])) << 16);
      reinterpret_cast<uint4*>(y + row * C)[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    }
  }
}

// y[n] = W[n, :] . x for one input row (the projections of a decode step): weights bf16 [N, K]
// row-major, read once with 16-byte loads (HBM-bound); each wave takes RPW consecutive rows, lane
// l the 8-element chunks l, l + 64, ... of each, fp32 products and sums, a wave reduction, bf16
// out. K a multiple of 8.
template <int RPW>
__global__ __launch_bounds__(256) void gemv_bf16_kernel(const uint16_t* __restrict__ W,
                                                        const uint16_t* __restrict__ x,
                                                        uint16_t* __restrict__ y, int N, int K) {
  const int lane = threadIdx.x & 63;
  const int r0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * RPW;
  if (r0 >= N) return;  // wave-uniform
  const int chunks = K >> 3;
  float acc[RPW];
#pragma unroll
  for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll 4
  for (int c = lane; c < chunks; c += 64) {
    const uint4 xv = reinterpret_cast<const uint4*>(x)[c];
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int row = min(r0 + r, N - 1);  // rows past N repeat the last one; not written
      const uint4 wv = reinterpret_cast<const uint4*>(W + (int64_t)row * K)[c];
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      float a = acc[r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a = fmaf(bf16_lo(ww[j]), bf16_lo(xw[j]), a);
        a = fmaf(bf16_hi(ww[j]), bf16_hi(xw[j]), a);
      }
      acc[r] = a;
    }
  }
#pragma unroll
  for (int r = 0; r < RPW; ++r) {
    const float a = wave_sum(acc[r]);
    if (lane == r && r0 + r < N) y[r0 + r] = f32_to_bf16(a);
  }
}

// The GEMVs of a decode step (one input row), with their neighbours fused in:
//  * IN == 0: y = W x;
//  * IN == 1 (input projection): x = RMSNorm(h) * w_in, the layer's input norm, each value
//    rounded to bf16 as the separate norm would;
//  * IN == 2 / 3 (output projection): x[k] = attn[k] * gate of k's head (IN 2: aux = gate logits
//    [H]) or of k itself (IN 3: aux [K]), the gate softplus(logit) rounded to bf16, the product
//    rounded to bf16 -- the gated attention output;
//  * with `res`: y[n] = bf16(res[n] + bf16(W[n] . x)), the residual add (y may alias res).
// Each thread first loads its input chunks (thread t: chunks t + 256 i) and their aux values,
// then every wave issues all its weight loads (RPW rows; lane l owns chunks l + 64 i, i < NL),
// and while those are in flight the workgroup builds the input vector once into LDS
// (the norm's sum of squares reduced over the workgroup); each wave then takes it from there.
// No load sits under a branch: an index past the end is clamped to a valid address and its value
// left unused (a branch around a load makes the compiler wait for every load in flight at the
// join). NC > 0: K == 512 NC exactly; NC == 0: any K up to 512 NLM, with run-time bounds.
//
// With EPI (input projection only, two rows per wave): the first `heads` x 128 outputs are the q
// and k heads, and each head is normalized and rotated in place (norm_rope_lane) by the last of
// its 16 workgroups to finish. Those workgroups store the head's rows with agent-scope stores
// (written through to the device-coherent level), wait for them, then count their arrival on the
// head's counter; the last arrival resets the counter to zero, and after an acquire fence its
// first wave reads the head back and rewrites it.
constexpr int MAXC = 16;  // K <= 512 MAXC = 8192 (Laguna's 48-head o_proj: 6144)
struct HeadEpilogue {
  const uint16_t* q_w;      // q_norm weights [128]
  const uint16_t* k_w;      // k_norm weights [128]
  const float* inv_freq;    // [rot_dims / 2]
  const int32_t* offsets;   // device position (one sequence), or null: `offset`
  uint32_t* counters;       // one per q/k head, zero between launches
  int64_t offset;
  int heads;                // Hq + Hkv
  int q_heads;              // Hq
  int rot_dims;
  float eps, mscale;
};

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// a + w . x over the 8 bf16 of one chunk
__device__ __forceinline__ float dot8(const uint4 w, const uint4 x, float a) {
  const uint32_t ww[4] = {w.x, w.y, w.z, w.w}, xw[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    a = fmaf(bf16_lo(ww[j]), bf16_lo(xw[j]), a);
    a = fmaf(bf16_hi(ww[j]), bf16_hi(xw[j]), a);
  }
  return a;
}

template <int RPW, int IN, bool EPI, int NC, int NLM>
__global__ __launch_bounds__(256) void gemv_fused_kernel(const uint16_t* W, const uint16_t* x,
                                                         const uint16_t* aux,
                                                         const uint16_t* res, uint16_t* y, int N,
                                                         int K, float eps, HeadEpilogue epi) {
  static_assert(!EPI || (RPW == 2 && IN == 1), "the head epilogue runs on the input projection");
  constexpr int NL = NC ? NC : NLM;  // weight chunks per lane per row
  constexpr int XIN = (64 * NL + 255) / 256;  // input chunks per thread
  static_assert(NL <= MAXC, "input wider than the staging buffer");
  __shared__ uint4 xs[64 * NL];
  __shared__ float red[4];
  __shared__ int sh_last;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int r0 = (blockIdx.x * 4 + (tid >> 6)) * RPW;
  const bool live = r0 < N;  // wave-uniform; every wave joins the barriers below
  const int chunks = NC ? 64 * NC : K >> 3;
  const uint4* x4 = reinterpret_cast<const uint4*>(x);
  const uint4* a4 = reinterpret_cast<const uint4*>(aux);

  uint4 xin[XIN], ain[XIN];
  uint16_t gin[XIN];
#pragma unroll
  for (int i = 0; i < XIN; ++i) {
    const int cc = min(tid + 256 * i, chunks - 1);
    xin[i] = x4[cc];
    if (IN == 1 || IN == 3) ain[i] = a4[cc];
    if (IN == 2) gin[i] = aux[(8 * cc) / ND];
  }
  // Keep the issue order: input loads, then weight loads, then the code that waits for the input
  // (vmcnt counts in order, so the input is waited for with the weights still in flight). The
  // pointers are not __restrict__, so no load moves across these memory barriers.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
  uint4 wreg[RPW][NL];
#pragma unroll
  for (int i = 0; i < NL; ++i) {
    const int cc = min(lane + 64 * i, chunks - 1);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      const int row = min(r0 + r, N - 1);  // rows past N repeat the last one; not written
      wreg[r][i] = reinterpret_cast<const uint4*>(W + (int64_t)row * K)[cc];
    }
  }
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);

  float inv = 1.0f;
  if (IN == 1) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XIN; ++i) {
      const uint32_t xw[4] = {xin[i].x, xin[i].y, xin[i].z, xin[i].w};
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s += bf16_lo(xw[j]) * bf16_lo(xw[j]) + bf16_hi(xw[j]) * bf16_hi(xw[j]);
      ss += tid + 256 * i < chunks ? s : 0.0f;
    }
    ss = wave_sum(ss);
    if (lane == 0) red[tid >> 6] = ss;
    __syncthreads();
    inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)K + eps);
  }
#pragma unroll
  for (int i = 0; i < XIN; ++i) {
    const uint32_t xw[4] = {xin[i].x, xin[i].y, xin[i].z, xin[i].w};
    const uint32_t aw[4] = {ain[i].x, ain[i].y, ain[i].z, ain[i].w};
    uint32_t ow[4];
    if (IN == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) ow[j] = xw[j];
    } else if (IN == 1) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        ow[j] = pack_bf16(bf16_lo(xw[j]) * inv * bf16_lo(aw[j]),
                          bf16_hi(xw[j]) * inv * bf16_hi(aw[j]));
    } else if (IN == 2) {
      const float gate = bf16_to_f32(f32_to_bf16(softplus_f(bf16_to_f32(gin[i]))));
#pragma unroll
      for (int j = 0; j < 4; ++j) ow[j] = pack_bf16(bf16_lo(xw[j]) * gate, bf16_hi(xw[j]) * gate);
    } else {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float g0 = bf16_to_f32(f32_to_bf16(softplus_f(bf16_lo(aw[j]))));
        const float g1 = bf16_to_f32(f32_to_bf16(softplus_f(bf16_hi(aw[j]))));
        ow[j] = pack_bf16(bf16_lo(xw[j]) * g0, bf16_hi(xw[j]) * g1);
      }
    }
    const int c = tid + 256 * i;
    if (c < chunks) xs[c] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
  __syncthreads();

  const bool head_rows = EPI && blockIdx.x * 4 * RPW < 128 * epi.heads;  // workgroup-uniform
  if (live) {
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = lane + 64 * i;
      const uint4 v = xs[min(c, chunks - 1)];
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        const float a = dot8(wreg[r][i], v, acc[r]);
        acc[r] = NC || c < chunks ? a : acc[r];
      }
    }
    uint16_t o[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      o[r] = f32_to_bf16(wave_sum(acc[r]));
    }
    if (head_rows) {  // rows r0, r0 + 1 of one q/k head (r0 even): one agent-scope word
      if (lane == 0)
        __hip_atomic_store(reinterpret_cast<uint32_t*>(y + r0),
                           (uint32_t)o[0] | ((uint32_t)o[RPW - 1] << 16), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    } else {
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        if (lane == r && r0 + r < N) {
          uint16_t v = o[r];
          if (res) v = f32_to_bf16(bf16_to_f32(res[r0 + r]) + bf16_to_f32(v));
          y[r0 + r] = v;
        }
      }
    }
  }
  if (!head_rows) return;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  const int head = (int)(blockIdx.x * 4 * RPW / 128);
  if (tid == 0) {
    const uint32_t prev =
        __hip_atomic_fetch_add(epi.counters + head, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev + 1 == 128 / (4 * RPW);
    if (last) __hip_atomic_store(epi.counters + head, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    sh_last = last;
  }
  __syncthreads();
  if (!sh_last || tid >= 64) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  uint32_t* row = reinterpret_cast<uint32_t*>(y + (int64_t)head * 128);
  const uint32_t x2 = __hip_atomic_load(row + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool is_q = head < epi.q_heads;
  const uint32_t w2 = reinterpret_cast<const uint32_t*>(is_q ? epi.q_w : epi.k_w)[lane];
  const float pos = (float)(epi.offsets ? (int64_t)epi.offsets[0] : epi.offset);
  row[lane] = norm_rope_lane(x2, w2, lane, epi.eps, epi.inv_freq, epi.rot_dims, epi.mscale, pos);
}

// Launches gemv_fused_kernel for (N, K): two rows per wave once there are enough rows to fill the
// chip with them (always with the head epilogue), exact-width variants for K = 2048, 4096 and
// 6144, else the narrowest run-time-bounded one (up to 2048, 4096 or 8192).
template <int IN, bool EPI>
void launch_gemv(const uint16_t* W, const uint16_t* x, const uint16_t* aux, const uint16_t* res,
                 uint16_t* y, int64_t N, int64_t K, float eps, const HeadEpilogue& epi,
                 hipStream_t st) {
  const bool two = EPI || N >= 4 * 2 * 2 * device_cu_count();
  const unsigned grid = (unsigned)(((two ? (N + 1) / 2 : N) + 3) / 4);
#define LQ_GEMV(RPW, NC, NLM)                                                            \
  gemv_fused_kernel<RPW, IN, EPI, NC, NLM><<<grid, 256, 0, st>>>(W, x, aux, res, y, (int)N,  \
                                                                (int)K, eps, epi)
#define LQ_GEMV_K(RPW)                                 \
  do {                                                 \
    if (K == 2048) LQ_GEMV(RPW, 4, 4);                 \
    else if (K == 4096) LQ_GEMV(RPW, 8, 8);            \
    else if (K == 6144) LQ_GEMV(RPW, 12, 12);          \
    else if (K <= 2048) LQ_GEMV(RPW, 0, 4);            \
    else if (K <= 4096) LQ_GEMV(RPW, 0, 8);            \
    else LQ_GEMV(RPW, 0, MAXC);                        \
  } while (0)
  if (two || EPI) {
    LQ_GEMV_K(2);
  } else if constexpr (!EPI) {
    LQ_GEMV_K(1);
  }
#undef LQ_GEMV_K
#undef LQ_GEMV
}

}  // namespace
}  // namespace lq

extern "C" int lq_gemv_fused(const uint16_t* W, const uint16_t* x, const uint16_t* aux,
                             const uint16_t* res, uint16_t* y, int64_t N, int64_t K, int mode,
                             float eps, int per_dim, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(N >= 1 && N <= (1 << 26) && K >= 8 && K <= 512 * MAXC && K % 8 == 0,
               "bad fused GEMV shape N=%lld K=%lld (K a multiple of 8, at most %d)", (long long)N,
               (long long)K, 512 * MAXC);
  LQ_CHECK_ARG(mode == 1 || (mode == 2 && K % ND == 0), "mode must be 1 (RMSNorm input) or 2 "
               "(gated attention input, K a multiple of 128)");
  LQ_CHECK_ARG(W && x && aux && y, "null pointer");
  LQ_CHECK_ARG(!res || res == y || (res + N <= y || y + N <= res), "res and y overlap partly");
  hipStream_t st = (hipStream_t)stream;
  const HeadEpilogue none{};
  if (mode == 1)
    launch_gemv<1, false>(W, x, aux, res, y, N, K, eps, none, st);
  else if (per_dim)
    launch_gemv<3, false>(W, x, aux, res, y, N, K, eps, none, st);
  else
    launch_gemv<2, false>(W, x, aux, res, y, N, K, eps, none, st);
  LQ_CHECK_LAUNCH("gemv_fused_kernel");
  return LQ_OK;
}

extern "C" int lq_gemv_norm_rope(const uint16_t* W, const uint16_t* x, const uint16_t* norm_w,
                                 uint16_t* y, int64_t N, int64_t K, float eps,
                                 const uint16_t* q_norm_w, const uint16_t* k_norm_w, int64_t Hq,
                                 int64_t Hkv, float head_eps, const float* inv_freq,
                                 int64_t rot_dims, float mscale, int64_t offset,
                                 const int32_t* offsets, uint32_t* counters, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(K >= 8 && K <= 512 * MAXC && K % 8 == 0,
               "bad input width K=%lld (a multiple of 8, at most %d)", (long long)K, 512 * MAXC);
  LQ_CHECK_ARG(Hq >= 1 && Hkv >= 1 && Hq <= 1024 && Hkv <= 1024, "bad head counts");
  LQ_CHECK_ARG(N >= ND * (Hq + Hkv) && N <= (1 << 26),
               "N=%lld must hold the %lld q/k head rows", (long long)N,
               (long long)(ND * (Hq + Hkv)));
  LQ_CHECK_ARG(rot_dims >= 0 && rot_dims <= ND && rot_dims % 4 == 0,
               "rot_dims must be a multiple of 4 in [0, 128] (got %lld)", (long long)rot_dims);
  LQ_CHECK_ARG(offset >= 0, "negative offset");
  LQ_CHECK_ARG(W && x && norm_w && y && q_norm_w && k_norm_w && counters &&
               (inv_freq || rot_dims == 0), "null pointer");
  HeadEpilogue epi{q_norm_w, k_norm_w, inv_freq, offsets, counters, offset, (int)(Hq + Hkv),
                   (int)Hq, (int)rot_dims, head_eps, mscale};
  launch_gemv<1, true>(W, x, norm_w, nullptr, y, N, K, eps, epi, (hipStream_t)stream);
  LQ_CHECK_LAUNCH("gemv_fused_kernel");
  return LQ_OK;
}


extern "C" int lq_gemv_bf16(const uint16_t* W, const uint16_t* x, uint16_t* y, int64_t N,
                            int64_t K, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(N >= 1 && N <= (1 << 26) && K >= 8 && K <= (1 << 20) && K % 8 == 0,
               "bad GEMV shape N=%lld K=%lld (K a multiple of 8)", (long long)N, (long long)K);
  LQ_CHECK_ARG(W && x && y, "null pointer");
  hipStream_t st = (hipStream_t)stream;
  if (K <= 512 * MAXC) {  // the staged-input kernel
    launch_gemv<0, false>(W, x, nullptr, nullptr, y, N, K, 0.0f, HeadEpilogue{}, st);
    LQ_CHECK_LAUNCH("gemv_fused_kernel");
    return LQ_OK;
  }
  // two rows per wave once there are enough rows to fill the chip with them
  if (N >= 4 * 2 * 2 * device_cu_count()) {
    const int64_t waves = (N + 1) / 2;
    gemv_bf16_kernel<2><<<dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st>>>(W, x, y, (int)N,
                                                                                  (int)K);
  } else {
    gemv_bf16_kernel<1><<<dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st>>>(W, x, y, (int)N,
                                                                              (int)K);
  }
  LQ_CHECK_LAUNCH("gemv_bf16_kernel");
  return LQ_OK;
}

extern "C" int lq_add_rms_norm(const uint16_t* h, const uint16_t* d, const uint16_t* w,
                               uint16_t* h_out, uint16_t* y, int64_t rows, int64_t C, float eps,
                               void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(C >= 8 && C <= 8192 && C % 8 == 0, "row size %lld must be a multiple of 8 in "
               "[8, 8192]", (long long)C);
  LQ_CHECK_ARG(rows >= 1 && rows <= INT32_MAX, "bad row count %lld", (long long)rows);
  LQ_CHECK_ARG(h && w && y && (!d || h_out), "null pointer");
  hipStream_t st = (hipStream_t)stream;
  add_rms_norm_kernel<<<dim3((unsigned)rows), dim3(256), 0, st>>>(h, d, w, h_out, y, (int)C, eps);
  LQ_CHECK_LAUNCH("add_rms_norm_kernel");
  return LQ_OK;
}

extern "C" int lq_qk_norm_rope(const uint16_t* q, const uint16_t* k, uint16_t* q_out,
                               uint16_t* k_out, const uint16_t* q_norm_w,
                               const uint16_t* k_norm_w, int64_t B, int64_t Hq, int64_t Hkv,
                               int64_t L, int64_t D, float eps, const float* inv_freq,
                               int64_t rot_dims, float mscale, int64_t offset,
                               const int32_t* offsets, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(D == ND, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(B >= 1 && Hq >= 1 && Hkv >= 1 && L >= 1 && Hq <= 1024 && Hkv <= 1024,
               "bad shape B=%lld Hq=%lld Hkv=%lld L=%lld", (long long)B, (long long)Hq,
               (long long)Hkv, (long long)L);
  LQ_CHECK_ARG(rot_dims >= 0 && rot_dims <= D && rot_dims % 4 == 0,
               "rot_dims must be a multiple of 4 in [0, 128] (got %lld)", (long long)rot_dims);
  LQ_CHECK_ARG(offset >= 0, "negative offset");
  LQ_CHECK_ARG(q && k && q_out && k_out && q_norm_w && k_norm_w && (inv_freq || rot_dims == 0),
               "null pointer");
  const int64_t rows = B * (Hq + Hkv) * L;
  LQ_CHECK_ARG(rows / 4 < (int64_t)INT32_MAX, "too many rows");
  hipStream_t st = (hipStream_t)stream;
  qk_norm_rope_kernel<<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st>>>(
      q, k, q_out, k_out, q_norm_w, k_norm_w, B, (int)Hq, (int)Hkv, L, eps, inv_freq,
      (int)rot_dims, mscale, offset, offsets);
  LQ_CHECK_LAUNCH("qk_norm_rope_kernel");
  return LQ_OK;
}

extern "C" int lq_gate_heads(const uint16_t* attn, const uint16_t* gate, uint16_t* out, int64_t B,
                             int64_t Hq, int64_t L, int64_t D, int per_dim, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(D == ND, "head_dim must be 128 (got %lld)", (long long)D);
  LQ_CHECK_ARG(B >= 1 && Hq >= 1 && L >= 1, "bad shape");
  LQ_CHECK_ARG(attn && gate && out && attn != out, "null or aliased pointer");
  const int64_t total = B * Hq * L * (ND / 8);
  LQ_CHECK_ARG(total / 256 < (int64_t)INT32_MAX, "too many rows");
  hipStream_t st = (hipStream_t)stream;
  gate_heads_kernel<<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st>>>(
      attn, gate, out, B, (int)Hq, L, per_dim ? 1 : 0);
  LQ_CHECK_LAUNCH("gate_heads_kernel");
  return LQ_OK;
}
