// Quantize-on-append and dequantize for the affine group-quantized KV cache.
//
// lq_quantize_append replaces mx.quantize as called by mlx-lm QuantizedKVCache.update_and_fetch
// from DequantKVCache.update_and_fetch (laguna_mlx/cache.py:89-90). One lane quantizes one whole
// group (32, 64 or 128 values): a wave's 64 groups are contiguous in the source, so they go to LDS
// with plain coalesced DMA copies (each copy fills 1 KB; a group's 16-byte chunks land at swizzled
// positions, chunk c of group g at c ^ s(g)), and each lane reads its own group back with
// conflict-free 16-byte LDS reads. The lane then takes the group's min and max in registers (no
// cross-lane reduction), derives scale and bias once with IEEE fp32 arithmetic (correctly rounded
// division, round-half-away), and writes the group's codes and its bf16 scale and bias. The
// arithmetic is bit-for-bit the MLX affine quantizer restated in oracle/quantize.py.
//
// lq_dequantize replaces mx.dequantize on the unfused path (cache.py:99-100):
// bf16(fp32(scale) * code + fp32(bias)) with an unfused multiply then add.
#include "attn_dev.h"

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
// correctly rounded division instead. u >= 0 up to rounding (the bias is the group's edge on the
// side the scale's sign points away from), so truncation is the floor and a slightly negative u
// converts to 0, as its floor clamps there. Returns the code; sets `slow` for the lanes that need
// the division.
template <int BITS>
__device__ __forceinline__ uint32_t fast_code(float x, const AffineParams& p, float rs, bool& slow) {
  const float u = fmaf(x - p.bias, rs, 0.5f);
  const float f = __builtin_amdgcn_fractf(u);
  slow = !(fabsf(f - 0.5f) < 0.4998f);
  return min((uint32_t)u, (uint32_t)((1 << BITS) - 1));
}

// One lane per group of GS values (CH = GS / 8 chunks of 16 bytes); a wave takes 64 consecutive
// groups (every group of the update lies in one row: GS divides the head dim). Groups [0, groups_a)
// belong to target a, [groups_a, groups) to target b (K and V of one update in one launch). Group
// q of a target: row q / gpr (row = bh L + l, cache row bh cap + offset + l), group q % gpr of it,
// source values GS q .. GS q + GS - 1.
//
// LDS layout per wave: group g's CH chunks at 16-byte slots CH g + (c ^ s(g)), s(g) = (g / (16 /
// CH)) % CH, so that the 16 lanes of one ds_read_b128 pass hit 16 different bank groups. Copy i of
// lane l fills slot 64 i + l.
template <int BITS, int GS>
__global__ __launch_bounds__(256) void quantize_group_kernel(
    AppendTarget a, AppendTarget b, int64_t groups_a, int64_t groups, FastDiv fd_gpr, FastDiv fd_L,
    int gpr, int L, int64_t cap, int64_t offset) {
  constexpr int CH = GS / 8;
  constexpr int CB = 2 * GS;          // source bytes per group
  constexpr int CPB = BITS * GS / 8;  // code bytes per group
  __shared__ __attribute__((aligned(16))) uint8_t stage[4][64 * CB];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));  // wave-uniform
  const uint32_t st_lds = attn::lds_addr(&stage[wv][0]);
  auto swz = [](int g) { return (g / (16 / CH)) % CH; };
  // per-lane byte offset of copy i within the wave's 64 CB source bytes (same for every wave)
  uint32_t voff[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int slot = 64 * i + lane, g = slot / CH, pos = slot % CH;
    voff[i] = (uint32_t)(g * CB + 16 * (pos ^ swz(g)));
  }
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t wbase = ((int64_t)blockIdx.x * 4 + wv) * 64; wbase < groups; wbase += stride) {
    // copies: one target and no tail (the common case) with a scalar base, else per-lane addresses
    if (wbase + 64 <= groups && (wbase + 64 <= groups_a || wbase >= groups_a)) {
      const bool in_a = wbase < groups_a;
      const uint8_t* base = reinterpret_cast<const uint8_t*>(in_a ? a.src : b.src) +
                            (in_a ? wbase : wbase - groups_a) * CB;
#pragma unroll
      for (int i = 0; i < CH; ++i)
        asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                     :: "v"(voff[i]), "s"(base), "s"(st_lds + 1024u * i) : "memory");
    } else {
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        const int slot = 64 * i + lane;
        const int64_t g = min(wbase + slot / CH, groups - 1);  // past the end: a valid group
        const bool in_a = g < groups_a;
        const uint8_t* src = reinterpret_cast<const uint8_t*>(in_a ? a.src : b.src) +
                             (in_a ? g : g - groups_a) * CB + (voff[i] % CB);
        asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                     :: "v"(src), "s"(st_lds + 1024u * i) : "memory");
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // this lane's group, in registers
    float x[GS];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint4 u = *reinterpret_cast<const uint4*>(&stage[wv][16 * (CH * lane + (c ^ swz(lane)))]);
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x[8 * c + 2 * j] = bf16_lo(w[j]);
        x[8 * c + 2 * j + 1] = bf16_hi(w[j]);
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // reads done before the next copies
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // min and max with v_min3/v_max3 as written: fminf/fmaxf would first quiet every decoded
    // value (a possible signalling NaN) with one more instruction each
    float lo = x[0], hi = x[0];
#pragma unroll
    for (int k = 1; k + 1 < GS; k += 2) {
      asm("v_min3_f32 %0, %1, %2, %3" : "=v"(lo) : "v"(lo), "v"(x[k]), "v"(x[k + 1]));
      asm("v_max3_f32 %0, %1, %2, %3" : "=v"(hi) : "v"(hi), "v"(x[k]), "v"(x[k + 1]));
    }
    asm("v_min_f32 %0, %1, %2" : "=v"(lo) : "v"(lo), "v"(x[GS - 1]));
    asm("v_max_f32 %0, %1, %2" : "=v"(hi) : "v"(hi), "v"(x[GS - 1]));
    const AffineParams p = affine_params<BITS>(lo, hi);
    const float rs = __builtin_amdgcn_rcpf(p.scale);
    // codes, one output dword (4 or 8 codes) at a time; the rare slow lanes redo their values
    constexpr int PER = 32 / BITS;  // codes per dword
    uint32_t out[GS / PER];
#pragma unroll
    for (int d = 0; d < GS / PER; ++d) {
      uint32_t c[PER];
      bool any = false;
#pragma unroll
      for (int r = 0; r < PER; ++r) {
        bool sl;
        c[r] = fast_code<BITS>(x[PER * d + r], p, rs, sl);
        any |= sl;
      }
      if (__builtin_amdgcn_ballot_w64(any)) {
#pragma unroll
        for (int r = 0; r < PER; ++r) {
          bool sl;
          (void)fast_code<BITS>(x[PER * d + r], p, rs, sl);
          if (sl) c[r] = affine_code<BITS>(x[PER * d + r], p);
        }
      }
      uint32_t wd = c[0];
#pragma unroll
      for (int r = 1; r < PER; ++r) wd |= c[r] << (BITS * r);
      out[d] = wd;
    }
    const int64_t gi = wbase + lane;
    if (gi < groups) {
      const bool in_a = gi < groups_a;
      const uint32_t q = (uint32_t)(in_a ? gi : gi - groups_a);
      const uint32_t row = fdiv_u(q, fd_gpr);
      const int gq = (int)(q - row * (uint32_t)gpr);
      const uint32_t bh = fdiv_u(row, fd_L);
      const int64_t drow = (int64_t)bh * cap + offset + (int64_t)(row - bh * (uint32_t)L);
      uint8_t* codes = (in_a ? a.codes : b.codes) + drow * ((int64_t)gpr * CPB) + (int64_t)gq * CPB;
#pragma unroll
      for (int d = 0; d < GS / PER; d += 4)
        *reinterpret_cast<uint4*>(codes + 4 * d) = make_uint4(out[d], out[d + 1], out[d + 2], out[d + 3]);
      (in_a ? a.scales : b.scales)[drow * gpr + gq] = f32_to_bf16(p.scale);
      (in_a ? a.biases : b.biases)[drow * gpr + gq] = f32_to_bf16(p.bias);
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

template <int BITS, int GS>
void launch_quantize(AppendTarget a, AppendTarget b, int64_t groups_a, int64_t groups, int gpr,
                     int L, int64_t cap, int64_t offset, hipStream_t st) {
  const int64_t blocks = std::min<int64_t>((groups + 255) / 256, 1 << 20);
  quantize_group_kernel<BITS, GS><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
      a, b, groups_a, groups, make_fastdiv((uint32_t)gpr), make_fastdiv((uint32_t)L), gpr, L, cap,
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
  const int64_t groups_a = B * H * L * (D / group_size);
  const int64_t groups = (two ? 2 : 1) * groups_a;
  LQ_CHECK_ARG(groups < (int64_t)1 << 31 && L < (int64_t)1 << 31,
               "append of %lld values is too large for one call",
               (long long)(groups * group_size));
  const int gpr = (int)(D / group_size);
  if (group_size == 32) {
    if (bits == 8) launch_quantize<8, 32>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
    else launch_quantize<4, 32>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
  } else if (group_size == 64) {
    if (bits == 8) launch_quantize<8, 64>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
    else launch_quantize<4, 64>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
  } else {
    if (bits == 8) launch_quantize<8, 128>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
    else launch_quantize<4, 128>(a, b, groups_a, groups, gpr, (int)L, cap, offset, st);
  }
  LQ_CHECK_LAUNCH("quantize_group_kernel");
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
