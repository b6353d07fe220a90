// Shared helpers for the gfx950 kernels of liblaguna_hip.so: status/error reporting, bf16 and
// fp16 bit tricks, wave64 cross-lane reductions, device properties.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/laguna_hip.h"

namespace lq {

// ---------------------------------------------------------------------------------------------
// host: error reporting
// ---------------------------------------------------------------------------------------------

void set_error(const char* fmt, ...);
void clear_error();

#define LQ_CHECK_ARG(cond, ...)          \
  do {                                   \
    if (!(cond)) {                       \
      ::lq::set_error(__VA_ARGS__);      \
      return LQ_EINVAL;                  \
    }                                    \
  } while (0)

#define LQ_CHECK_HIP(expr)                                                          \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess) {                                                         \
      ::lq::set_error("%s failed: %s", #expr, hipGetErrorString(e_));               \
      return LQ_EHIP;                                                               \
    }                                                                               \
  } while (0)

// Launch-error check right after a <<<>>> launch.
#define LQ_CHECK_LAUNCH(name)                                                       \
  do {                                                                              \
    hipError_t e_ = hipGetLastError();                                              \
    if (e_ != hipSuccess) {                                                         \
      ::lq::set_error("launch of %s failed: %s", name, hipGetErrorString(e_));      \
      return LQ_EHIP;                                                               \
    }                                                                               \
  } while (0)

// Compute units of the current device (cached per device id).
int device_cu_count();

// One tensor to append to a cache: source rows (bf16 [B, H, L, D]) and the cache buffers.
struct AppendTarget {
  const uint16_t* src;
  uint8_t* codes;
  uint16_t* scales;
  uint16_t* biases;
};
// Quantize-on-append of a (and b when `two`) into rows [offset, offset + L), one launch.
// Validates its arguments (LQ_EINVAL with the error set).
int quantize_append(AppendTarget a, AppendTarget b, int two, int64_t B, int64_t H, int64_t L,
                    int64_t D, int64_t cap, int64_t offset, int bits, int group_size,
                    hipStream_t st);

// ---------------------------------------------------------------------------------------------
// device: number formats
// ---------------------------------------------------------------------------------------------

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (NaN -> quiet NaN).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Affine group quantizer (MLX affine_quantize, restated in oracle/quantize.py): parameters from
// the group's min and max, then one code per value. IEEE fp32, correctly rounded division, Metal
// round (halves away from zero). Shared by every kernel that quantizes so that the codes agree
// bit for bit.
struct AffineParams {
  float scale, bias;
};
template <int BITS>
__device__ __forceinline__ AffineParams affine_params(float w_min, float w_max) {
  constexpr float n_bins = (float)((1 << BITS) - 1);
  float scale = fmaxf(__fdiv_rn(w_max - w_min, n_bins), 1e-7f);
  const bool side = fabsf(w_min) > fabsf(w_max);
  scale = side ? scale : -scale;
  const float edge = side ? w_min : w_max;
  const float q0 = roundf(__fdiv_rn(edge, scale));
  const bool at_zero = q0 == 0.0f;
  return {at_zero ? scale : __fdiv_rn(edge, q0), at_zero ? 0.0f : edge};
}
template <int BITS>
__device__ __forceinline__ uint32_t affine_code(float x, AffineParams p) {
  constexpr float n_bins = (float)((1 << BITS) - 1);
  return (uint32_t)fminf(roundf(__fdiv_rn(x - p.bias, p.scale)), n_bins);
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Two codes of w as fp16 subnormals (bit pattern 0x00cc = c * 2^-24, exact): bytes (0,1) or (2,3).
__device__ __forceinline__ uint32_t codes_sub_w(uint32_t w, uint32_t sel) {
  return __builtin_amdgcn_perm(0u, w, sel);
}
constexpr uint32_t SUB_B01 = 0x0c010c00u;
constexpr uint32_t SUB_B23 = 0x0c030c02u;

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }


// ---------------------------------------------------------------------------------------------
// device: wave64 cross-lane helpers
// ---------------------------------------------------------------------------------------------

// DPP control codes (GCN/CDNA): quad permutes and row (16-lane) rotations.
constexpr int DPP_QUAD_XOR1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR4 = 0x124;   // row_ror:4
constexpr int DPP_ROW_ROR8 = 0x128;   // row_ror:8
constexpr int DPP_ROW_MIRROR = 0x140;       // lane i of a row <- lane 15 - i
constexpr int DPP_ROW_HALF_MIRROR = 0x141;  // lane i of a half row <- lane 7 - i

// x of another lane of the same row of 16. Only controls under which every lane reads a valid
// source lane (quad_perm, row_ror, the mirrors), so the DPP "old" value is never used: it is left
// undefined, which lets the compiler fold the move into the VALU op that consumes it
// (v_add_f32_dpp, v_max_f32_dpp, ...). With an explicit old value each use was three instructions
// (v_mov of the old value, v_mov_b32_dpp, the op), a latency chain in the reductions.
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  static_assert(CTRL <= 0xFF || (CTRL >= 0x121 && CTRL <= 0x12F) || CTRL == 0x140 || CTRL == 0x141,
                "dpp: only full permutations within a row (no shifts or broadcasts)");
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xF, 0xF, true));
}

// IEEE 754-2019 maximum (NaN if either operand is NaN; equal to fmaxf on everything else): one
// v_maximum3_f32. fmaxf of a value the compiler cannot prove canonical -- the result of a DPP move
// or a lane swap -- costs a canonicalizing v_max_f32 per such operand first, three or four
// instructions per reduction step instead of one; the attention reductions (scores, the
// merges' maxima, |q| and |scale_v|) use this one. The quantizers keep fmaxf.
__device__ __forceinline__ float max_ieee(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max / sum with the lane 16 (32) apart, on the VALU: v_permlane16_swap (v_permlane32_swap)
// exchanges whole rows of 16 (halves of 32) lanes between two registers, so combining the two
// results gives every lane the op over itself and its partner. All 64 lanes must be active.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_ieee(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over each aligned group of 4 lanes, result in all 4 lanes.
__device__ __forceinline__ float quad_sum(float x) {
  x += dpp<DPP_QUAD_XOR1>(x);
  x += dpp<DPP_QUAD_XOR2>(x);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp<DPP_QUAD_XOR1>(x));
  x = fmaxf(x, dpp<DPP_QUAD_XOR2>(x));
  x = fmaxf(x, dpp<DPP_ROW_ROR4>(x));
  x = fmaxf(x, dpp<DPP_ROW_ROR8>(x));
  x = fmaxf(x, __shfl_xor(x, 16, 64));
  x = fmaxf(x, __shfl_xor(x, 32, 64));
  return x;
}

__device__ __forceinline__ float wave_min(float x) {
  x = fminf(x, dpp<DPP_QUAD_XOR1>(x));
  x = fminf(x, dpp<DPP_QUAD_XOR2>(x));
  x = fminf(x, dpp<DPP_ROW_ROR4>(x));
  x = fminf(x, dpp<DPP_ROW_ROR8>(x));
  x = fminf(x, __shfl_xor(x, 16, 64));
  x = fminf(x, __shfl_xor(x, 32, 64));
  return x;
}

// Sum over all 64 lanes, in every lane, on the VALU (DPP row steps, then the row and half
// swaps): no LDS round trips, unlike a butterfly of cross-lane reads. All lanes active.
__device__ __forceinline__ float wave_sum(float x) {
  x += dpp<DPP_QUAD_XOR1>(x);
  x += dpp<DPP_QUAD_XOR2>(x);
  x += dpp<DPP_ROW_ROR4>(x);
  x += dpp<DPP_ROW_ROR8>(x);
  return sum_xor32(sum_xor16(x));
}

// RMSNorm (times w, rounded to bf16) and RoPE at position `pos` of one 128-dim head row held by
// one wave (the reference's q_norm / k_norm, then rope, laguna_mlx/laguna.py:97-101): lane l
// holds dims 2l and 2l + 1 as the bf16 pair x2 (norm weights w2); returns the lane's output pair.
// The normalized row is rounded to bf16 before the rotation, as the reference's two separate ops
// round between them; the rotation is the non-interleaved form on the first rot_dims dims (dim i
// pairs with dim i + rot_dims / 2, the partner value rot_dims / 4 lanes away), angle pos *
// inv_freq[i], rotated dims scaled by mscale.
// sin and cos of the fp32 angle a (|a| up to ~2^24): the reduction by 2 pi is done in fp64 (exact
// to ~1e-11 for these magnitudes), so sincosf runs on |r| <= pi, its short path.
__device__ __forceinline__ void sincos_reduced(float a, float* s, float* c) {
  const double ad = (double)a;
  const double k = rint(ad * 0.15915494309189535);      // 1 / (2 pi)
  sincosf((float)fma(-k, 6.283185307179586, ad), s, c);  // 2 pi
}

// The value of lane (lane +- off) for rotation partners: whole-row swaps on the VALU for off 16
// and 32 (the half- and full-rotary cases of head_dim 128), a cross-lane read otherwise. All 64
// lanes must be active; lanes without a partner get an unspecified value.
__device__ __forceinline__ float rope_partner(float y, int lane, int off, int partner) {
  if (off == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float((lane & 16) ? r[0] : r[1]);
  }
  if (off == 32) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(y), __float_as_uint(y), false, false);
    return __uint_as_float((lane & 32) ? r[0] : r[1]);
  }
  return __shfl(y, partner, 64);
}

// The rotation of lane `lane` at position pos: sin and cos of its two angles (the same for every
// row at that position), whether its dims rotate and whether they are the first half's.
struct RopeLane {
  float s0, c0, s1, c1;
  bool rot, first;
};
__device__ __forceinline__ RopeLane rope_lane(int lane, const float* __restrict__ inv_freq,
                                              int rot_dims, float pos) {
  RopeLane r{0.f, 1.f, 0.f, 1.f, 2 * lane < rot_dims, 4 * lane < rot_dims};
  if (r.rot) {
    const int i0 = r.first ? 2 * lane : 2 * lane - (rot_dims >> 1);
    sincos_reduced(pos * inv_freq[i0], &r.s0, &r.c0);
    sincos_reduced(pos * inv_freq[i0 + 1], &r.s1, &r.c1);
  }
  return r;
}

// RMSNorm of N rows held two values per lane (row j: pair x2[j], norm weights w2[j]), then the
// rotation rl (from rope_lane), in place. The rows go through each phase together (reductions,
// then the partner exchanges under one branch on the partner distance, then the rotations), so
// that their dependency chains interleave; each row's arithmetic is that of the one-row case.
template <int N>
__device__ __forceinline__ void norm_rope_rows(uint32_t (&x2)[N], const uint32_t (&w2)[N], int lane,
                                               float eps, const RopeLane& rl, int rot_dims,
                                               float mscale) {
  float y0[N], y1[N];
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float x0 = bf16_lo(x2[j]), x1 = bf16_hi(x2[j]);
    float ss = x0 * x0 + x1 * x1;  // sum over the wave: rows of 16 by DPP, then row swaps
    ss += dpp<DPP_QUAD_XOR1>(ss);
    ss += dpp<DPP_QUAD_XOR2>(ss);
    ss += dpp<DPP_ROW_ROR4>(ss);
    ss += dpp<DPP_ROW_ROR8>(ss);
    ss = sum_xor32(sum_xor16(ss));
    const float inv = rsqrtf(ss * (1.0f / 128) + eps);
    // RMSNorm output, rounded to bf16 (the reference's norm returns bf16)
    y0[j] = bf16_to_f32(f32_to_bf16(x0 * inv * bf16_lo(w2[j])));
    y1[j] = bf16_to_f32(f32_to_bf16(x1 * inv * bf16_hi(w2[j])));
  }
  const int half = rot_dims >> 1;      // rotated pairs
  const int lane_off = rot_dims >> 2;  // partner lane distance
  const int partner = rl.rot ? (2 * lane < half ? lane + lane_off : lane - lane_off) : lane;
  float p0[N], p1[N];
  if (lane_off == 16) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      p0[j] = rope_partner(y0[j], lane, 16, partner);
      p1[j] = rope_partner(y1[j], lane, 16, partner);
    }
  } else if (lane_off == 32) {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      p0[j] = rope_partner(y0[j], lane, 32, partner);
      p1[j] = rope_partner(y1[j], lane, 32, partner);
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) {
      p0[j] = rope_partner(y0[j], lane, lane_off, partner);
      p1[j] = rope_partner(y1[j], lane, lane_off, partner);
    }
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    float r0 = y0[j], r1 = y1[j];
    if (rl.rot) {
      const float a0 = r0 * mscale, a1 = r1 * mscale, b0 = p0[j] * mscale, b1 = p1[j] * mscale;
      if (rl.first) {  // dims i < half: out = x_i cos - x_{i+half} sin
        r0 = a0 * rl.c0 - b0 * rl.s0;
        r1 = a1 * rl.c1 - b1 * rl.s1;
      } else {  // this lane holds x_{i+half}; the partner holds x_i
        r0 = b0 * rl.s0 + a0 * rl.c0;
        r1 = b1 * rl.s1 + a1 * rl.c1;
      }
    }
    x2[j] = (uint32_t)f32_to_bf16(r0) | ((uint32_t)f32_to_bf16(r1) << 16);
  }
}

// One row: returns the lane's output pair.
__device__ __forceinline__ uint32_t norm_rope_apply(uint32_t x2, uint32_t w2, int lane, float eps,
                                                    const RopeLane& rl, int rot_dims, float mscale) {
  uint32_t x[1] = {x2};
  const uint32_t w[1] = {w2};
  norm_rope_rows<1>(x, w, lane, eps, rl, rot_dims, mscale);
  return x[0];
}

__device__ __forceinline__ uint32_t norm_rope_lane(uint32_t x2, uint32_t w2, int lane, float eps,
                                                   const float* __restrict__ inv_freq,
                                                   int rot_dims, float mscale, float pos) {
  return norm_rope_apply(x2, w2, lane, eps, rope_lane(lane, inv_freq, rot_dims, pos), rot_dims,
                         mscale);
}

}  // namespace lq
