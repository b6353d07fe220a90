// Quantize-on-append and dequantize for the affine group-quantized KV cache.
//
// lq_quantize_append replaces mx.quantize as called by mlx-lm QuantizedKVCache.update_and_fetch
// from DequantKVCache.update_and_fetch (laguna_mlx/cache.py:89-90). One wave64 owns one group
// (32, 64 or 128 values): the group min/max are wave reductions, then every lane derives the same
// scale/bias with IEEE fp32 arithmetic (correctly rounded division, round-half-away), writes its
// codes, and lane 0 writes the bf16 scale and bias. The arithmetic is bit-for-bit the MLX affine
// quantizer restated in oracle/quantize.py.
//
// lq_dequantize replaces mx.dequantize on the unfused path (cache.py:99-100):
// bf16(fp32(scale) * code + fp32(bias)) with an unfused multiply then add.
#include "common.h"

namespace lq {
namespace {

constexpr int kWaves = 4;  // waves (groups) per 256-thread block

// EPL: elements per lane (group_size / 64, at least 1). BITS: 4 or 8.
// Groups [0, ngroups) go to target a, groups [ngroups, 2 ngroups) to target b when `two` (K and
// V of one update in a single launch).
template <int EPL, int BITS>
__global__ __launch_bounds__(256) void quantize_append_kernel(
    AppendTarget a, AppendTarget b, int two, int64_t ngroups, int gs, int groups_per_row,
    int64_t L, int64_t cap, int64_t offset) {
  const int lane = threadIdx.x & 63;
  int64_t gi = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (gi >= (two ? 2 * ngroups : ngroups)) return;  // whole wave exits together (wave-uniform)
  const bool second = gi >= ngroups;
  if (second) gi -= ngroups;
  const uint16_t* __restrict__ src = second ? b.src : a.src;
  uint8_t* __restrict__ codes = second ? b.codes : a.codes;
  uint16_t* __restrict__ scales = second ? b.scales : a.scales;
  uint16_t* __restrict__ biases = second ? b.biases : a.biases;

  const bool has = lane * EPL < gs;
  float x[EPL];
  float lo = INFINITY, hi = -INFINITY;
  const uint16_t* g = src + gi * gs;
#pragma unroll
  for (int e = 0; e < EPL; ++e) {
    x[e] = has ? bf16_to_f32(g[lane * EPL + e]) : 0.0f;
    if (has) {
      lo = fminf(lo, x[e]);
      hi = fmaxf(hi, x[e]);
    }
  }
  const float w_min = wave_min(lo);
  const float w_max = wave_max(hi);

  const AffineParams p = affine_params<BITS>(w_min, w_max);
  const float scale = p.scale, bias = p.bias;

  uint32_t c[EPL];
#pragma unroll
  for (int e = 0; e < EPL; ++e) c[e] = affine_code<BITS>(x[e], p);

  // destination row in the cache
  const int64_t row = gi / groups_per_row;
  const int gr = (int)(gi - row * groups_per_row);
  const int64_t bh = row / L;
  const int64_t l = row - bh * L;
  const int64_t drow = bh * cap + offset + l;
  const int64_t row_bytes = (int64_t)groups_per_row * gs * BITS / 8;
  uint8_t* dst = codes + drow * row_bytes + (int64_t)gr * (gs * BITS / 8);

  if (BITS == 8) {
    if (has) {
      if (EPL == 1) {
        dst[lane] = (uint8_t)c[0];
      } else {  // EPL == 2
        *reinterpret_cast<uint16_t*>(dst + 2 * lane) = (uint16_t)(c[0] | (c[EPL - 1] << 8));
      }
    }
  } else {  // 4-bit: element 2j in the low nibble of byte j
    if (EPL == 2) {
      if (has) dst[lane] = (uint8_t)(c[0] | (c[EPL - 1] << 4));
    } else {
      const uint32_t nb = (uint32_t)__shfl_down((int)c[0], 1, 64);
      if (has && (lane & 1) == 0) dst[lane >> 1] = (uint8_t)(c[0] | (nb << 4));
    }
  }
  if (lane == 0) {
    scales[drow * groups_per_row + gr] = f32_to_bf16(scale);
    biases[drow * groups_per_row + gr] = f32_to_bf16(bias);
  }
}

// One thread per 8 consecutive elements of one row (8 divides every group size).
template <int BITS>
__global__ __launch_bounds__(256) void dequantize_kernel(
    const uint8_t* __restrict__ codes, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, int64_t BH, int64_t cap, int64_t n, int D, int gs,
    uint16_t* __restrict__ out) {
  const int64_t per_row = D / 8;
  const int64_t total = BH * n * per_row;
  const int groups_per_row = D / gs;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row;  // output row in [BH * n)
    const int d0 = (int)(i - r * per_row) * 8;
    const int64_t bh = r / n;
    const int64_t t = r - bh * n;
    const int64_t crow = bh * cap + t;
    const int gr = d0 / gs;
    const float s = bf16_to_f32(scales[crow * groups_per_row + gr]);
    const float b = bf16_to_f32(biases[crow * groups_per_row + gr]);
    uint32_t cv[8];
    if (BITS == 8) {
      const uint2 w = *reinterpret_cast<const uint2*>(codes + crow * D + d0);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        cv[k] = (w.x >> (8 * k)) & 0xffu;
        cv[4 + k] = (w.y >> (8 * k)) & 0xffu;
      }
    } else {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(codes + crow * (D / 2) + d0 / 2);
#pragma unroll
      for (int k = 0; k < 8; ++k) cv[k] = (w >> (4 * k)) & 0xfu;
    }
    uint32_t o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint16_t a = f32_to_bf16(__fadd_rn(__fmul_rn(s, (float)cv[2 * k]), b));
      const uint16_t c = f32_to_bf16(__fadd_rn(__fmul_rn(s, (float)cv[2 * k + 1]), b));
      o[k] = (uint32_t)a | ((uint32_t)c << 16);
    }
    *reinterpret_cast<uint4*>(out + r * D + d0) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

template <int EPL, int BITS>
void launch_quantize(AppendTarget a, AppendTarget b, int two, int64_t ngroups, int gs, int gpr,
                     int64_t L, int64_t cap, int64_t offset, hipStream_t st) {
  const int64_t blocks = ((two ? 2 : 1) * ngroups + kWaves - 1) / kWaves;
  quantize_append_kernel<EPL, BITS><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
      a, b, two, ngroups, gs, gpr, L, cap, offset);
}

}  // namespace

int quantize_append(AppendTarget a, AppendTarget b, int two, int64_t B, int64_t H, int64_t L,
                    int64_t D, int64_t cap, int64_t offset, int bits, int group_size,
                    hipStream_t st) {
  LQ_CHECK_ARG(bits == 4 || bits == 8, "bits must be 4 or 8 (got %d)", bits);
  LQ_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
               "group_size must be 32, 64 or 128 (got %d)", group_size);
  LQ_CHECK_ARG(B >= 1 && H >= 1 && L >= 0 && D >= 1, "bad shape B=%lld H=%lld L=%lld D=%lld",
               (long long)B, (long long)H, (long long)L, (long long)D);
  LQ_CHECK_ARG(D % group_size == 0, "head_dim %lld is not a multiple of group_size %d",
               (long long)D, group_size);
  LQ_CHECK_ARG(offset >= 0 && offset + L <= cap, "rows [%lld, %lld) exceed capacity %lld",
               (long long)offset, (long long)(offset + L), (long long)cap);
  LQ_CHECK_ARG(a.src && a.codes && a.scales && a.biases, "null pointer");
  LQ_CHECK_ARG(!two || (b.src && b.codes && b.scales && b.biases), "null pointer");
  if (L == 0) return LQ_OK;
  const int gpr = (int)(D / group_size);
  const int64_t ngroups = B * H * L * gpr;
  if (group_size == 128) {
    if (bits == 8) launch_quantize<2, 8>(a, b, two, ngroups, group_size, gpr, L, cap, offset, st);
    else launch_quantize<2, 4>(a, b, two, ngroups, group_size, gpr, L, cap, offset, st);
  } else {
    if (bits == 8) launch_quantize<1, 8>(a, b, two, ngroups, group_size, gpr, L, cap, offset, st);
    else launch_quantize<1, 4>(a, b, two, ngroups, group_size, gpr, L, cap, offset, st);
  }
  LQ_CHECK_LAUNCH("quantize_append_kernel");
  return LQ_OK;
}

}  // namespace lq

extern "C" int lq_quantize_append(const uint16_t* src, int64_t B, int64_t H, int64_t L, int64_t D,
                                  uint8_t* codes, uint16_t* scales, uint16_t* biases, int64_t cap,
                                  int64_t offset, int bits, int group_size, void* stream) {
  using namespace lq;
  clear_error();
  const AppendTarget a{src, codes, scales, biases};
  return quantize_append(a, a, 0, B, H, L, D, cap, offset, bits, group_size, (hipStream_t)stream);
}

extern "C" int lq_quantize_append_kv(const uint16_t* k_src, const uint16_t* v_src, int64_t B,
                                     int64_t H, int64_t L, int64_t D, uint8_t* k_codes,
                                     uint16_t* k_scales, uint16_t* k_biases, uint8_t* v_codes,
                                     uint16_t* v_scales, uint16_t* v_biases, int64_t cap,
                                     int64_t offset, int bits, int group_size, void* stream) {
  using namespace lq;
  clear_error();
  const AppendTarget a{k_src, k_codes, k_scales, k_biases};
  const AppendTarget b{v_src, v_codes, v_scales, v_biases};
  return quantize_append(a, b, 1, B, H, L, D, cap, offset, bits, group_size, (hipStream_t)stream);
}

extern "C" int lq_dequantize(const uint8_t* codes, const uint16_t* scales, const uint16_t* biases,
                             int64_t B, int64_t H, int64_t cap, int64_t n, int64_t D, int bits,
                             int group_size, uint16_t* out, void* stream) {
  using namespace lq;
  clear_error();
  LQ_CHECK_ARG(bits == 4 || bits == 8, "bits must be 4 or 8 (got %d)", bits);
  LQ_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
               "group_size must be 32, 64 or 128 (got %d)", group_size);
  LQ_CHECK_ARG(B >= 1 && H >= 1 && D >= 1 && D % group_size == 0, "bad shape");
  LQ_CHECK_ARG(n >= 0 && n <= cap, "n=%lld outside [0, cap=%lld]", (long long)n, (long long)cap);
  LQ_CHECK_ARG(codes && scales && biases && out, "null pointer");
  if (n == 0) return LQ_OK;
  const int64_t total = B * H * n * (D / 8);
  const int64_t blocks = std::min<int64_t>((total + 255) / 256, 65536);
  hipStream_t st = (hipStream_t)stream;
  if (bits == 8)
    dequantize_kernel<8><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(codes, scales, biases, B * H, cap, n, (int)D, group_size, out);
  else
    dequantize_kernel<4><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(codes, scales, biases, B * H, cap, n, (int)D, group_size, out);
  LQ_CHECK_LAUNCH("dequantize_kernel");
  return LQ_OK;
}
