// Quantize-on-append and dequantize for the affine group-quantized KV cache.
//
// lq_quantize_append replaces mx.quantize as called by mlx-lm QuantizedKVCache.update_and_fetch
// from DequantKVCache.update_and_fetch (laguna_mlx/cache.py:89-90). A lane takes 8 consecutive
// values of a row (one 16-byte load) and the gs / 8 lanes of a group (32, 64 or 128 values, side
// by side in one wave) reduce its min and max with DPP; every lane then derives the group's
// scale/bias with IEEE fp32 arithmetic (correctly rounded division, round-half-away) and writes
// its 8 codes (8 or 4 bytes), and the group's first lane writes the bf16 scale and bias. The
// arithmetic is bit-for-bit the MLX affine quantizer restated in oracle/quantize.py.
//
// lq_dequantize replaces mx.dequantize on the unfused path (cache.py:99-100):
// bf16(fp32(scale) * code + fp32(bias)) with an unfused multiply then add.
#include "common.h"

namespace lq {
namespace {

// Unsigned division by a fixed divisor d >= 1 of values below 2^31: q = (mulhi(n, m) + n) >> l
// with 2^(l-1) < d <= 2^l and m = floor(2^32 (2^l - d) / d) + 1 (Granlund and Montgomery, 1994).
struct FastDiv {
  uint32_t m, l;
};
FastDiv make_fastdiv(uint32_t d) {
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint64_t m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return {(uint32_t)m, l};
}
__device__ __forceinline__ uint32_t fdiv_u(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.m) + n) >> f.l;
}

// Code of one value: round-half-away(fl(fl(x - bias) / scale)) clamped to 2^BITS - 1, as
// affine_code. Fast path: u = (x - bias) * (1 / scale) + 0.5 (v_rcp_f32, 1 ulp) is within
// 6.1e-5 of fl(fl(x - bias) / scale) + 0.5 for quotients below 512 (ours stay below 257), so
// floor(u) is the code unless u lies within 2e-4 of an integer; those lanes (and NaN/inf) take the
// correctly rounded division instead. Returns the code; sets `slow` for the lanes that need it.
template <int BITS>
__device__ __forceinline__ uint32_t fast_code(float x, const AffineParams& p, float rs, bool& slow) {
  constexpr float n_bins = (float)((1 << BITS) - 1);
  const float u = fmaf(x - p.bias, rs, 0.5f);
  const float f = u - floorf(u);
  slow = !(fabsf(f - 0.5f) < 0.4998f);
  return (uint32_t)fminf(floorf(u), n_bins);
}

// LPG = group_size / 8 lanes per group; UN chunks of 8 values per lane per pass (loads issued
// together). Chunks [0, chunks) go to target a, [chunks, 2 chunks) to target b when `two` (K and V
// of one update in one launch). Chunk c of a target: row c / cpr (row = bh L + l, cache row
// bh cap + offset + l), values 8 (c % cpr) .. + 7.
template <int BITS, int LPG, int UN>
__global__ __launch_bounds__(256) void quantize_append_kernel(
    AppendTarget a, AppendTarget b, int64_t chunks, int64_t total, FastDiv fd_cpr, FastDiv fd_L,
    int cpr, int L, int64_t cap, int64_t offset) {
  const int lane = threadIdx.x & 63;
  const int gpr = cpr / LPG;  // groups per row
  const int64_t stride = (int64_t)gridDim.x * 256 * UN;
  for (int64_t base = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64 * UN; base < total;
       base += stride) {  // wave-uniform
    uint4 raw[UN];
    int64_t cc[UN];
    bool sec[UN], in[UN];
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const int64_t i = base + 64 * u + lane;
      in[u] = i < total;
      sec[u] = i >= chunks;
      cc[u] = sec[u] ? i - chunks : i;
      const uint16_t* src = sec[u] ? b.src : a.src;
      raw[u] = in[u] ? *reinterpret_cast<const uint4*>(src + cc[u] * 8) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < UN; ++u) {
      const uint32_t w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
      float x[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[2 * j] = bf16_lo(w[j]);
        x[2 * j + 1] = bf16_hi(w[j]);
      }
      float lo = INFINITY, hi = -INFINITY;
      if (in[u]) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          lo = fminf(lo, x[j]);
          hi = fmaxf(hi, x[j]);
        }
      }
      // group min / max over its LPG lanes (quads, then half rows, then rows)
      lo = fminf(lo, dpp<DPP_QUAD_XOR1>(lo));
      hi = fmaxf(hi, dpp<DPP_QUAD_XOR1>(hi));
      lo = fminf(lo, dpp<DPP_QUAD_XOR2>(lo));
      hi = fmaxf(hi, dpp<DPP_QUAD_XOR2>(hi));
      if (LPG >= 8) {
        lo = fminf(lo, dpp<DPP_ROW_HALF_MIRROR>(lo));
        hi = fmaxf(hi, dpp<DPP_ROW_HALF_MIRROR>(hi));
      }
      if (LPG >= 16) {
        lo = fminf(lo, dpp<DPP_ROW_MIRROR>(lo));
        hi = fmaxf(hi, dpp<DPP_ROW_MIRROR>(hi));
      }
      const AffineParams p = affine_params<BITS>(lo, hi);
      const float rs = __builtin_amdgcn_rcpf(p.scale);
      uint32_t c[8];
      bool any_slow = false, slow[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        c[j] = fast_code<BITS>(x[j], p, rs, slow[j]);
        any_slow |= slow[j];
      }
      if (__builtin_amdgcn_ballot_w64(any_slow && in[u])) {  // rare: a value near a rounding edge
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (slow[j]) c[j] = affine_code<BITS>(x[j], p);
      }
      if (in[u]) {
        const uint32_t cu = (uint32_t)cc[u];
        const uint32_t row = fdiv_u(cu, fd_cpr);
        const int ch = (int)(cu - row * (uint32_t)cpr);
        const uint32_t bh = fdiv_u(row, fd_L);
        const int64_t drow = (int64_t)bh * cap + offset + (int64_t)(row - bh * (uint32_t)L);
        uint8_t* codes = sec[u] ? b.codes : a.codes;
        if (BITS == 8) {
          const uint32_t d0 = c[0] | (c[1] << 8) | (c[2] << 16) | (c[3] << 24);
          const uint32_t d1 = c[4] | (c[5] << 8) | (c[6] << 16) | (c[7] << 24);
          *reinterpret_cast<uint2*>(codes + drow * (8 * cpr) + 8 * ch) = make_uint2(d0, d1);
        } else {  // element 2j in the low nibble of byte j
          uint32_t d0 = 0u;
#pragma unroll
          for (int j = 0; j < 8; ++j) d0 |= c[j] << (4 * j);
          *reinterpret_cast<uint32_t*>(codes + drow * (4 * cpr) + 4 * ch) = d0;
        }
        if (ch % LPG == 0) {
          uint16_t* scales = sec[u] ? b.scales : a.scales;
          uint16_t* biases = sec[u] ? b.biases : a.biases;
          scales[drow * gpr + ch / LPG] = f32_to_bf16(p.scale);
          biases[drow * gpr + ch / LPG] = f32_to_bf16(p.bias);
        }
      }
    }
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

template <int BITS, int LPG>
void launch_quantize(AppendTarget a, AppendTarget b, int64_t chunks, int64_t total, int cpr, int L,
                     int64_t cap, int64_t offset, hipStream_t st) {
  constexpr int UN = 4;
  const int64_t waves = (total + 64 * UN - 1) / (64 * UN);
  const int64_t blocks = std::min<int64_t>((waves + 3) / 4, 8192);
  quantize_append_kernel<BITS, LPG, UN><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
      a, b, chunks, total, make_fastdiv((uint32_t)cpr), make_fastdiv((uint32_t)L), cpr, L, cap,
      offset);
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
  const int64_t chunks = B * H * L * (D / 8);  // 8 values each
  const int64_t total = (two ? 2 : 1) * chunks;
  LQ_CHECK_ARG(total < (int64_t)1 << 31 && L < (int64_t)1 << 31 && D / 8 < (int64_t)1 << 31,
               "append of %lld values is too large for one call", (long long)(total * 8));
  const int cpr = (int)(D / 8);
  if (group_size == 32) {
    if (bits == 8) launch_quantize<8, 4>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
    else launch_quantize<4, 4>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
  } else if (group_size == 64) {
    if (bits == 8) launch_quantize<8, 8>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
    else launch_quantize<4, 8>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
  } else {
    if (bits == 8) launch_quantize<8, 16>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
    else launch_quantize<4, 16>(a, b, chunks, total, cpr, (int)L, cap, offset, st);
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
