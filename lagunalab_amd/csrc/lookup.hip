// Prompt-lookup draft search and greedy acceptance of a verified block.
//
// lq_ngram_propose replaces NgramIndex.propose (laguna_mlx/dflash.py:164-167) for a history that
// lives on the device. The reference keeps a host dict of g-gram -> most recent start; on the
// GPU the same answer is one parallel scan: every candidate start s <= T-g-1 is compared with the
// final g ids, each workgroup keeps its largest matching s, and a one-workgroup finisher takes
// the maximum and copies the continuation hist[s+g : min(s+g+n, T)].
//
// lq_greedy_accept replaces the argmax + longest-prefix loop of generate_lookup
// (dflash.py:195-198): a chunked argmax (first index wins ties) over each verify row, then a
// one-workgroup finisher computes k and the next token pred[k].
#include "common.h"

namespace lq {
namespace {

constexpr int NG_CHUNK = 512;   // candidate starts per workgroup (256 threads x 2): ~160
                                // workgroups at T = 82,671, each one load round trip
constexpr int AC_CHUNK = 4096;  // logits per workgroup (256 threads x 16)

__global__ __launch_bounds__(256) void ngram_scan_kernel(const int32_t* __restrict__ hist,
                                                         int64_t T, int g,
                                                         int32_t* __restrict__ best) {
  __shared__ int32_t key[16];
  __shared__ int32_t wbest[4];
  const int tid = threadIdx.x;
  if (tid < g) key[tid] = hist[T - g + tid];
  __syncthreads();
  const int64_t S = T - g;  // candidates s in [0, S)
  const int64_t base = (int64_t)blockIdx.x * NG_CHUNK;
  int32_t mine = -1;
#pragma unroll
  for (int k = 0; k < NG_CHUNK / 256; ++k) {
    const int64_t s = base + (int64_t)k * 256 + tid;
    if (s < S) {
      bool ok = true;
      for (int j = 0; j < g; ++j) ok = ok && (hist[s + j] == key[j]);
      if (ok) mine = (int32_t)s;  // increasing s per thread: the last hit is the largest
    }
  }
  // workgroup max
  for (int off = 32; off >= 1; off >>= 1) mine = max(mine, __shfl_xor(mine, off, 64));
  if ((tid & 63) == 0) wbest[tid >> 6] = mine;
  __syncthreads();
  if (tid == 0) best[blockIdx.x] = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
}

__global__ __launch_bounds__(256) void ngram_finish_kernel(const int32_t* __restrict__ hist,
                                                           int64_t T, int g, int n, int nchunks,
                                                           const int32_t* __restrict__ best,
                                                           int32_t* __restrict__ out) {
  __shared__ int32_t wbest[4];
  const int tid = threadIdx.x;
  int32_t m = -1;
  for (int i = tid; i < nchunks; i += 256) m = max(m, best[i]);
  for (int off = 32; off >= 1; off >>= 1) m = max(m, __shfl_xor(m, off, 64));
  if ((tid & 63) == 0) wbest[tid >> 6] = m;
  __syncthreads();
  const int32_t s = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
  int count = 0;
  if (s >= 0) count = (int)min<int64_t>((int64_t)n, T - (s + g));
  if (tid == 0) {
    out[0] = count;
    out[1] = s;
  }
  if (tid < count) out[2 + tid] = hist[s + g + tid];
}

// (value, index) with ties to the smaller index
__device__ __forceinline__ void argmax_merge(float& v, int32_t& i, float v2, int32_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

__global__ __launch_bounds__(256) void argmax_chunk_kernel(const float* __restrict__ logits,
                                                           int64_t V, int nchunks,
                                                           float2* __restrict__ part) {
  __shared__ float sv[4];
  __shared__ int32_t si[4];
  const int tid = threadIdx.x;
  const int row = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * AC_CHUNK;
  const float* r = logits + (int64_t)row * V;
  float bv = -INFINITY;
  int32_t bi = INT32_MAX;
  if ((V & 3) == 0) {
#pragma unroll
    for (int k = 0; k < AC_CHUNK / 1024; ++k) {
      const int64_t i = base + (int64_t)k * 1024 + 4 * tid;
      if (i < V) {
        const float4 x = *reinterpret_cast<const float4*>(r + i);
        argmax_merge(bv, bi, x.x, (int32_t)i);
        argmax_merge(bv, bi, x.y, (int32_t)i + 1);
        argmax_merge(bv, bi, x.z, (int32_t)i + 2);
        argmax_merge(bv, bi, x.w, (int32_t)i + 3);
      }
    }
  } else {
    for (int k = 0; k < AC_CHUNK / 256; ++k) {
      const int64_t i = base + (int64_t)k * 256 + tid;
      if (i < V) argmax_merge(bv, bi, r[i], (int32_t)i);
    }
  }
  for (int off = 32; off >= 1; off >>= 1) {
    const float v2 = __shfl_xor(bv, off, 64);
    const int32_t i2 = __shfl_xor(bi, off, 64);
    argmax_merge(bv, bi, v2, i2);
  }
  if ((tid & 63) == 0) {
    sv[tid >> 6] = bv;
    si[tid >> 6] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    for (int w = 1; w < 4; ++w) argmax_merge(bv, bi, sv[w], si[w]);
    part[(int64_t)row * nchunks + blockIdx.x] = make_float2(bv, __int_as_float(bi));
  }
}

// One workgroup: the 32 lanes of a row group reduce that row's chunk partials (all rows'
// loads in one round trip for L <= 8), then k and the next token.
__global__ __launch_bounds__(256) void accept_finish_kernel(const float2* __restrict__ part,
                                                            int L, int nchunks,
                                                            const int32_t* __restrict__ drafts,
                                                            int m, int32_t* __restrict__ out) {
  __shared__ int32_t pred[64];
  const int tid = threadIdx.x;
  const int sub = tid & 31;  // lane within the row's 32-lane group
  for (int row = tid >> 5; row < L; row += 8) {
    float bv = -INFINITY;
    int32_t bi = INT32_MAX;
    for (int c = sub; c < nchunks; c += 32) {
      const float2 p = part[(int64_t)row * nchunks + c];
      argmax_merge(bv, bi, p.x, __float_as_int(p.y));
    }
    for (int off = 16; off >= 1; off >>= 1) {
      const float v2 = __shfl_xor(bv, off, 64);
      const int32_t i2 = __shfl_xor(bi, off, 64);
      argmax_merge(bv, bi, v2, i2);
    }
    if (sub == 0) pred[row] = bi;
  }
  __syncthreads();
  if (tid == 0) {
    int k = 0;
    while (k < m && drafts[k] == pred[k]) ++k;
    out[0] = k;
    out[1] = pred[k];
  }
  for (int row = tid; row < L; row += 256) out[2 + row] = pred[row];
}

}  // namespace
}  // namespace lq

extern "C" int64_t lq_ngram_workspace_bytes(int64_t T) {
  if (T < 1) return 4;
  return std::max<int64_t>(1, (T + lq::NG_CHUNK - 1) / lq::NG_CHUNK) * (int64_t)sizeof(int32_t);
}

extern "C" int lq_ngram_propose(const int32_t* hist, int64_t T, int g, int n, int32_t* out,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(g >= 1 && g <= 16, "g must be in [1, 16] (got %d)", g);
  LQ_CHECK_ARG(n >= 1 && n <= 64, "n must be in [1, 64] (got %d)", n);
  LQ_CHECK_ARG(T >= 0 && T <= INT32_MAX, "bad history length %lld", (long long)T);
  LQ_CHECK_ARG(out && (hist || T == 0), "null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int64_t S = T - g;  // number of candidate starts
  const int nchunks = S > 0 ? (int)((S + NG_CHUNK - 1) / NG_CHUNK) : 0;
  if (nchunks > 0) {
    if (!workspace || workspace_bytes < (int64_t)nchunks * 4) {
      set_error("workspace too small for the n-gram scan");
      return LQ_EWORKSPACE;
    }
    ngram_scan_kernel<<<dim3(nchunks), dim3(256), 0, st>>>(hist, T, g, (int32_t*)workspace);
    LQ_CHECK_LAUNCH("ngram_scan_kernel");
  }
  ngram_finish_kernel<<<dim3(1), dim3(256), 0, st>>>(hist, T, g, n, nchunks,
                                                     (const int32_t*)workspace, out);
  LQ_CHECK_LAUNCH("ngram_finish_kernel");
  return LQ_OK;
}

extern "C" int64_t lq_accept_workspace_bytes(int64_t L, int64_t V) {
  if (L < 1 || V < 1) return 8;
  return L * ((V + lq::AC_CHUNK - 1) / lq::AC_CHUNK) * (int64_t)sizeof(float2);
}

extern "C" int lq_greedy_accept(const float* logits, int64_t L, int64_t V, const int32_t* drafts,
                                int64_t m, int32_t* out, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(L >= 1 && L <= 64, "verify rows L must be in [1, 64] (got %lld)", (long long)L);
  LQ_CHECK_ARG(V >= 1 && V <= INT32_MAX, "bad vocabulary size %lld", (long long)V);
  LQ_CHECK_ARG(m >= 0 && m <= L - 1, "drafts m=%lld must be <= L-1=%lld", (long long)m,
               (long long)(L - 1));
  LQ_CHECK_ARG(logits && out && (drafts || m == 0), "null pointer");
  const int nchunks = (int)((V + AC_CHUNK - 1) / AC_CHUNK);
  if (!workspace || workspace_bytes < L * nchunks * (int64_t)sizeof(float2)) {
    set_error("workspace too small for greedy accept");
    return LQ_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  float2* part = (float2*)workspace;
  argmax_chunk_kernel<<<dim3(nchunks, (unsigned)L), dim3(256), 0, st>>>(logits, V, nchunks, part);
  LQ_CHECK_LAUNCH("argmax_chunk_kernel");
  accept_finish_kernel<<<dim3(1), dim3(256), 0, st>>>(part, (int)L, nchunks, drafts, (int)m, out);
  LQ_CHECK_LAUNCH("accept_finish_kernel");
  return LQ_OK;
}
