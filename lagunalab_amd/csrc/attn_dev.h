// Device-side building blocks shared by the attention kernels (qattn.hip, attn_bf16.hip,
// attn_q4.hip): MFMA operand types and conversions, the global -> LDS copy helpers, agent-scope
// partial accesses, the row quantizer of the fused append, and the packed kernels' epilogue with
// the in-kernel split merge.
#pragma once

#include <type_traits>

#include "common.h"
#include "qattn.h"

namespace lq {
namespace attn {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef int v2i_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i_t lds_v2i_t;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr float RESCALE_LOG2 = 8.0f;  // lazy softmax rescale threshold (log2 units)

// 2^x for x <= 0 (softmax weights against a running or merged maximum): the hardware exp2
// without the library's denormal-range fix-up; results below 2^-126 are negligible next to the
// maximum's weight 1.
__device__ __forceinline__ float exp2_nonpos(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 codes (two words) as fp16 subnormals c * 2^-24 for an MFMA operand.
__device__ __forceinline__ half8_t codes8_sub(uint32_t w0, uint32_t w1) {
  typedef uint32_t u4v_t __attribute__((ext_vector_type(4)));
  const u4v_t u = {codes_sub_w(w0, SUB_B01), codes_sub_w(w0, SUB_B23), codes_sub_w(w1, SUB_B01),
                   codes_sub_w(w1, SUB_B23)};
  return __builtin_bit_cast(half8_t, u);
}
__device__ __forceinline__ half8_t words_as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  typedef uint32_t u4v_t __attribute__((ext_vector_type(4)));
  const u4v_t u = {a, b, c, d};
  return __builtin_bit_cast(half8_t, u);
}
// Two floats as one dword of fp16 (round to nearest even), x in the low half.
__device__ __forceinline__ uint32_t pack_h2(float x, float y) {
  const half2_t h = {(_Float16)x, (_Float16)y};
  return __builtin_bit_cast(uint32_t, h);
}


// One bf16 half of a word as fp32 with one v_perm_b32, the half chosen by a per-lane selector
// (SEL_LO: bits 0-15, SEL_HI: bits 16-31, moved to the top, zeros below).
constexpr uint32_t SEL_LO = 0x01000c0cu;
constexpr uint32_t SEL_HI = 0x03020c0cu;
__device__ __forceinline__ float bf16_pick(uint32_t w, uint32_t sel) {
  return __uint_as_float(__builtin_amdgcn_perm(0u, w, sel));
}

// ---- fp16 operand range. The MFMA operands are fp16 (normal from 2^-14 to 65504, subnormal
// steps of 2^-24), while the reference computes in fp32 (q8_attn.py:117). Two power-of-two
// factors keep the operands where fp16 holds them to 11 bits, and come back out exactly:
//  * q: every query row of a wave is multiplied by one 2^kq that puts the largest |q| element in
//    [2^14, 2^15) before the fp16 conversion (exact for bf16 values in the normal range); 2^-kq
//    goes into the per-key K factor. Supported: finite q with max |q| in about [1e-25, 1e34];
//    elements more than 2^28 below a wave's largest lose bits, at a relative weight < 2^-28.
//  * P.V: B = p * scale_v * 2^kv per quant group and wave, 2^kv chosen so that the largest
//    |scale_v| of the valid keys of a super-tile lies in [16, 32); it is kept while that largest
//    value stays within [0.25, 128] (p <= 2^8 under the lazy softmax rescale, so B <= 2^15), and
//    otherwise re-chosen and the group's accumulators rescaled by the exact ratio. 2^-kv is taken
//    out before the epilogue. Supported: |scale_v| in about [3e-11, 1.7e13] (kv in [-40, 40]).

// 2^k as a float, k in [-126, 127].
__device__ __forceinline__ float pow2f(int k) { return __uint_as_float((uint32_t)(k + 127) << 23); }

// k with amax * 2^k in [2^(e - 1), 2^e), clamped to [lo, hi]; amax > 0 and finite.
__device__ __forceinline__ int pow2_exp_into(float amax, int e, int lo, int hi) {
  return min(max(e - __builtin_amdgcn_frexp_expf(amax), lo), hi);
}

// Max over all 64 lanes on the VALU (DPP row steps, then row and half swaps); all lanes active.
__device__ __forceinline__ float wave_max_valu(float x) {
  x = max_ieee(x, dpp<DPP_QUAD_XOR1>(x));
  x = max_ieee(x, dpp<DPP_QUAD_XOR2>(x));
  x = max_ieee(x, dpp<DPP_ROW_ROR4>(x));
  x = max_ieee(x, dpp<DPP_ROW_ROR8>(x));
  return max_xor32(max_xor16(x));
}

// Largest magnitude of the two bf16 values of a dword, as bf16 bits (an unsigned 16-bit max of
// the magnitudes orders them like the values; NaN payloads compare above infinity).
__device__ __forceinline__ uint32_t bf16x2_absmax_bits(uint32_t acc, uint32_t w) {
  typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
  const u16x2_t a = __builtin_bit_cast(u16x2_t, acc), b = __builtin_bit_cast(u16x2_t, w & 0x7fff7fffu);
  return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}
__device__ __forceinline__ float bf16x2_max_value(uint32_t m) {
  return fmaxf(bf16_lo(m), bf16_hi(m));
}

// Workgroup barrier over LDS data only: the wave's LDS operations complete, then s_barrier.
// Vector memory operations in flight (copies into LDS counted by vmcnt) are not waited for.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// The q exponent kq of a wave from the largest |q| element any lane of it holds (0 when q is 0).
__device__ __forceinline__ int q_pow2_exp(float amax_lane) {
  const float m = wave_max_valu(amax_lane);
  return m > 0.0f ? pow2_exp_into(m, 15, -100, 100) : 0;
}

constexpr float VF_HI = 128.0f;  // re-choose the P.V factor when a scaled |scale_v| exceeds this
constexpr float VF_LO = 0.25f;   // ... or when all of a super-tile's are below this
constexpr int VK_NONE = -1000;   // P.V exponent before the first key with a nonzero V scale

// The P.V exponents kv of a wave, one per quant group, and their factors 2^kv (0 before set).
struct VScale {
  int k0 = VK_NONE, k1 = VK_NONE;
  float f0 = 0.0f, f1 = 0.0f;
};

// Whether the P.V factors of a wave must be re-chosen for the super-tile whose keys the lanes
// hold: a0 / a1 are |scale_v| of this lane's key (0 for keys past the sequence). All 64 lanes
// active; every lane passes its key's values; the result is wave-uniform. Kernels test it in the
// same branch as the lazy softmax rescale, so the hot path gets no branch of its own.
__device__ __forceinline__ bool vscale_check(float a0, float a1, const VScale& v) {
  const bool over = fmaxf(a0 * v.f0, a1 * v.f1) > VF_HI;
  const uint64_t big0 = __builtin_amdgcn_ballot_w64(a0 * v.f0 >= VF_LO);
  const uint64_t big1 = __builtin_amdgcn_ballot_w64(a1 * v.f1 >= VF_LO);
  return (__builtin_amdgcn_ballot_w64(over) | (big0 == 0) | (big1 == 0)) != 0;
}

// Re-chooses the P.V factors (after vscale_check returned true) and rescales the accumulators by
// the exact ratio. oacc: NACC sets of 8 accumulators, in each of which [0..3] hold group 0 dims
// and [4..7] group 1 (in every kernel that calls this). The caller then rewrites the scaled V
// terms of the tile.
template <int NACC = 1>
__device__ __forceinline__ void vscale_apply(float a0, float a1, VScale& v, f4_t* oacc) {
  const float m0 = wave_max_valu(a0), m1 = wave_max_valu(a1);
  const int n0 = m0 > 0.0f ? pow2_exp_into(m0, 5, -40, 40) : v.k0;
  const int n1 = m1 > 0.0f ? pow2_exp_into(m1, 5, -40, 40) : v.k1;
  // exact power-of-two ratios; an unset factor (0) had produced zero accumulators, so with both
  // unset (the first super-tile) nothing is scaled (wave-uniform)
  const float r0 = v.k0 == VK_NONE ? 0.0f : pow2f(n0 - v.k0);
  const float r1 = v.k1 == VK_NONE ? 0.0f : pow2f(n1 - v.k1);
  if (v.k0 != VK_NONE || v.k1 != VK_NONE) {
#pragma unroll
    for (int i = 0; i < NACC; ++i)
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) oacc[8 * i + dt] *= dt < 4 ? r0 : r1;
  }
  v.k0 = n0;
  v.k1 = n1;
  v.f0 = n0 == VK_NONE ? 0.0f : pow2f(n0);
  v.f1 = n1 == VK_NONE ? 0.0f : pow2f(n1);
}

// The packed finish's per-wave output factors: base * 2^-kv of the dim's quant group, times `odd`
// for odd dims in the 4-bit layout (class 2 g + (dim & 1)); applied to the summed accumulators
// instead of rescaling each accumulator before the finish (exact: powers of two).
__device__ __forceinline__ void vscale_out(const VScale& v, float base, float odd, float (&osc)[4]) {
  const float i0 = v.k0 == VK_NONE ? base : base * pow2f(-v.k0);
  const float i1 = v.k1 == VK_NONE ? base : base * pow2f(-v.k1);
  osc[0] = i0;
  osc[1] = i0 * odd;
  osc[2] = i1;
  osc[3] = i1 * odd;
}

// Takes the P.V factors back out of the accumulators (before the epilogue).
template <int NACC = 1>
__device__ __forceinline__ void vscale_remove(const VScale& v, f4_t* oacc) {
  const float i0 = v.k0 == VK_NONE ? 1.0f : pow2f(-v.k0);
  const float i1 = v.k1 == VK_NONE ? 1.0f : pow2f(-v.k1);
#pragma unroll
  for (int i = 0; i < NACC; ++i)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) oacc[8 * i + dt] *= dt < 4 ? i0 : i1;
}

// Global -> LDS copies (LDS destination = lds_base + size * lane; lds_base wave-uniform). They are
// issued as inline asm on purpose: the compiler then has no pending LDS write to guard and adds no
// blanket vmcnt(0) in front of every LDS read, which would wait for the prefetched tile too.
// Every wait on these copies is explicit (s_waitcnt vmcnt(N) with the count of copies issued
// after the ones needed).
// The copies carry the non-temporal hint (nt): the cache streams through once per call, and
// marking it streaming keeps it from displacing other lines (measured on the 8-bit decode at
// 82,671 keys over 10 rotating layer caches: 42.8 -> 40.8 us per launch).
__device__ __forceinline__ uint32_t lds_u32(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ void g2l_b32(const void* g, void* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off nt"
               :: "v"(g), "s"(lds_u32(lds_base)) : "memory");
}
__device__ __forceinline__ void g2l_b128(const void* g, void* lds_base) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :: "v"(g), "s"(lds_u32(lds_base)) : "memory");
}
// Same copies with a wave-uniform global base (SGPR pair) plus a 32-bit per-lane offset, into
// LDS at lds + LOFF (lds wave-uniform): no 64-bit address arithmetic per lane and no
// readfirstlane per copy. The instruction's immediate offset stays 0 (it would move the LDS
// destination too). The asm only moves into M0 (no SCC-writing instruction: the compiler may
// keep a carry live across the statement).
template <int LOFF>
__device__ __forceinline__ void dma_b128(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
               :: "v"(voff), "s"(sbase), "s"(lds + LOFF) : "memory");
}
template <int LOFF>
__device__ __forceinline__ void dma_b32(const void* sbase, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1 nt"
               :: "v"(voff), "s"(sbase), "s"(lds + LOFF) : "memory");
}
// Copy groups of a full super-tile under one M0: four 16-byte copies from rows RS bytes apart in
// global memory to LDS destinations RS bytes apart (the immediate offset moves both), or the four
// word arrays of a super-tile (bases pre-shifted by -OFS_j so that offset OFS_j lands each in its
// LDS array, the arrays OFS bytes apart). One M0 write and its wait state per group instead of
// per copy.
template <int LOFF, int RS>
__device__ __forceinline__ void dma4_b128(const void* sbase, uint32_t voff, uint32_t lds) {
  static_assert(3 * RS < 4096, "immediate offsets are 12-bit");
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\t"
               "global_load_lds_dwordx4 %0, %1 nt\n\t"
               "global_load_lds_dwordx4 %0, %1 offset:%3 nt\n\t"
               "global_load_lds_dwordx4 %0, %1 offset:%4 nt\n\t"
               "global_load_lds_dwordx4 %0, %1 offset:%5 nt"
               :: "v"(voff), "s"(sbase), "s"(lds + LOFF), "i"(RS), "i"(2 * RS), "i"(3 * RS)
               : "memory");
}
template <int LOFF, int OFS>
__device__ __forceinline__ void dma4_b32(const void* s0, const void* s1, const void* s2,
                                         const void* s3, uint32_t voff, uint32_t lds) {
  static_assert(3 * OFS < 4096, "immediate offsets are 12-bit");
  asm volatile("s_mov_b32 m0, %5\n\ts_nop 0\n\t"
               "global_load_lds_dword %0, %1 nt\n\t"
               "global_load_lds_dword %0, %2 offset:%6 nt\n\t"
               "global_load_lds_dword %0, %3 offset:%7 nt\n\t"
               "global_load_lds_dword %0, %4 offset:%8 nt"
               :: "v"(voff), "s"(s0), "s"(s1), "s"(s2), "s"(s3), "s"(lds + LOFF), "i"(OFS),
                  "i"(2 * OFS), "i"(3 * OFS)
               : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One 128-element bf16 row quantized to 8 bits in groups of 64 by one wave, lane l holding
// elements 2l and 2l+1 (group l / 32): the two codes of the lane (low 16 bits) and the bf16 scale
// and bias of its group. Same arithmetic as quantize_group_kernel (affine_params/affine_code on
// the group min and max), so the codes agree bit for bit. All 64 lanes must be active.
struct QPair {
  uint32_t codes;
  uint16_t scale, bias;
};
__device__ __forceinline__ QPair quantize_pair_q8(uint32_t x2) {
  const float x0 = bf16_lo(x2), x1 = bf16_hi(x2);
  float lo = fminf(x0, x1), hi = fmaxf(x0, x1);
  lo = fminf(lo, dpp<DPP_QUAD_XOR1>(lo));
  hi = fmaxf(hi, dpp<DPP_QUAD_XOR1>(hi));
  lo = fminf(lo, dpp<DPP_QUAD_XOR2>(lo));
  hi = fmaxf(hi, dpp<DPP_QUAD_XOR2>(hi));
  lo = fminf(lo, dpp<DPP_ROW_ROR4>(lo));
  hi = fmaxf(hi, dpp<DPP_ROW_ROR4>(hi));
  lo = fminf(lo, dpp<DPP_ROW_ROR8>(lo));
  hi = fmaxf(hi, dpp<DPP_ROW_ROR8>(hi));
  const auto rl = __builtin_amdgcn_permlane16_swap(__float_as_uint(lo), __float_as_uint(lo), false, false);
  const auto rh = __builtin_amdgcn_permlane16_swap(__float_as_uint(hi), __float_as_uint(hi), false, false);
  lo = fminf(__uint_as_float(rl[0]), __uint_as_float(rl[1]));
  hi = fmaxf(__uint_as_float(rh[0]), __uint_as_float(rh[1]));
  const AffineParams p = affine_params<8>(lo, hi);
  return {affine_code<8>(x0, p) | (affine_code<8>(x1, p) << 8), f32_to_bf16(p.scale),
          f32_to_bf16(p.bias)};
}

// Agent-scope relaxed atomic accesses: written through to / read from the device-coherent level,
// so partials published by one workgroup are visible to a workgroup on another XCD without a
// release fence (which writes back a whole L2) in every workgroup.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// Two consecutive floats (8-byte aligned) as one 8-byte agent-scope store.
__device__ __forceinline__ void st_agent2(float* p, float lo, float hi) {
  const uint64_t u = (uint64_t)__float_as_uint(lo) | ((uint64_t)__float_as_uint(hi) << 32);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Four consecutive floats (16-byte aligned) read at the device-coherent level with one 16-byte
// load (buffer_load_dwordx4 sc1, the cache policy of an agent-scope load): `rsrc` covers the
// buffer, `off` is the byte offset in it.
__device__ __forceinline__ f4_t ld_agent4(__amdgpu_buffer_rsrc_t rsrc, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(rsrc, off, 0, 16);
}
// Two consecutive floats (8-byte aligned) read at the device-coherent level: one 8-byte
// agent-scope load (global_load_dwordx2 sc1), which no stale line of this XCD's L2 can serve, so
// a reader needs no cache invalidation before it. Loads of a batch go out together.
__device__ __forceinline__ float2 ld_agent2(const float* p) {
  const uint64_t u = __hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<float*>(p)),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)u), __uint_as_float((uint32_t)(u >> 32)));
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// Log-sum-exp merge of the split partials of sequence b, KV head hk (R <= RW query rows, RW = 4
// or 8) by one workgroup of NW waves, into the output rows (b * Hkv + hk) * R + row of
// out [B, Hq, L, D] (bf16). Partial (m, l, acc) of split s, row r: part_ml / part_acc at
// (s * Hkv + hk) * R + r.
// Thread t takes 4 dims (t % 32) of row (t % 32 RW) / 32 over the splits of parity t / 32 RW (one
// to four parities: NW * 64 / (32 RW)): it loads the acc of up to MCH splits at once (one memory
// round trip for up to MCH splits per parity: 16 with one or two parities, 8 with four), merges
// them with its own running max, and the parities meet in LDS. The (m, l) of each (split, row)
// are loaded once, by one thread, and shared through LDS: the 32 threads of a row all need them,
// and as one load per thread they cost the texture path half as many bytes again as the acc
// partials (its bytes per lane, not the unique bytes, set the merge's load time). The merging
// kernels have at most 32 splits per sequence (the plan caps them), so one load per thread
// covers them. red: LDS scratch of at least 6 * 32 RW * max(1, parities - 1) + 2 * 32 RW floats.
template <int NW, int RW = 4>
__device__ void merge_rows4(int b, int hk, int Hkv, int R, const DecodePlan& plan,
                            const float* __restrict__ part_acc,
                            const float2* __restrict__ part_ml, uint16_t* __restrict__ out,
                            float* red) {
  constexpr int TPR = 32 * RW;         // threads per parity
  constexpr int NPAR = 64 * NW / TPR;  // split parities
  static_assert(RW == 4 || RW == 8, "4 or 8 rows per parity");
  static_assert(NPAR == 1 || NPAR == 2 || NPAR == 4, "one, two or four split parities");
  static_assert(32 * RW <= 64 * NW, "one (m, l) load per thread covers 32 splits");
  constexpr int MCH = NPAR == 4 ? 8 : 16;
  const int tid = threadIdx.x;
  const int s0 = plan.split_begin[b];
  const int ns = plan.split_begin[b + 1] - s0;
  const int64_t rs = (int64_t)Hkv * R;
  const int64_t r0 = (int64_t)hk * R;
  const int o = tid % TPR;
  const int row = o >> 5;
  const int d0 = 4 * (o & 31);
  const int par = tid / TPR;
  const int rowc = min(row, R - 1);  // threads past the rows load and weigh row R - 1, unused
  float2* const mls = reinterpret_cast<float2*>(red + 6 * TPR * (NPAR > 2 ? NPAR - 1 : 1));
  // (m, l) of (split mi / R, row mi % R) first, then the first batch of this thread's acc
  // partials (through one buffer resource with the sequence's first split as its wave-uniform
  // base, 16 bytes at a 32-bit byte offset per split), all in flight before the LDS exchange
  const int nml = ns * R;
  const int mi = min(tid, nml - 1);
  const int msp = mi / R;
  const float2 mlt = ld_agent2(reinterpret_cast<const float*>(
      part_ml + (int64_t)(s0 + msp) * rs + r0 + (mi - msp * R)));
  const __amdgpu_buffer_rsrc_t rsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float*>(part_acc + (int64_t)s0 * rs * D), 0, 0x7fffffff, 0x00020000);
  const uint32_t abase = (uint32_t)(((r0 + rowc) * D + d0) * 4);
  const int step = (int)rs;
  auto load_acc = [&](int base, f4_t (&av)[MCH]) {
#pragma unroll
    for (int k = 0; k < MCH; ++k)
      av[k] = ld_agent4(rsrc, abase + (uint32_t)(min(base + NPAR * k, ns - 1) * step) * (D * 4));
  };
  f4_t av0[MCH];
  load_acc(par, av0);
  if (tid < nml) mls[tid] = mlt;
  __syncthreads();
  float M = -INFINITY, den = 0.0f;
  float a[4] = {0.f, 0.f, 0.f, 0.f};
  // Branch-free: every loaded value is used on every path (with the weighting under a branch on
  // the maxima the compiler had waited for the m values before issuing the acc loads: a second
  // memory round trip). Splits whose rows saw no key (m = -inf) weigh 0.
  auto weigh = [&](int base, const f4_t (&av)[MCH]) {
    float mv[MCH], lv[MCH];
#pragma unroll
    for (int k = 0; k < MCH; ++k) {
      const float2 ml = mls[min(base + NPAR * k, ns - 1) * R + rowc];
      mv[k] = ml.x;
      lv[k] = ml.y;
    }
    float cm = -INFINITY;
#pragma unroll
    for (int k = 0; k < MCH; ++k) cm = max_ieee(cm, base + NPAR * k < ns ? mv[k] : -INFINITY);
    const float Mn = max_ieee(M, cm);
    const float Mr = Mn == -INFINITY ? 0.0f : Mn;
    const float sc = M == -INFINITY ? 0.0f : exp2_nonpos(M - Mr);
    den *= sc;
#pragma unroll
    for (int j = 0; j < 4; ++j) a[j] *= sc;
#pragma unroll
    for (int k = 0; k < MCH; ++k) {
      const bool use = base + NPAR * k < ns && mv[k] != -INFINITY;
      const float w = use ? exp2_nonpos(mv[k] - Mr) : 0.0f;
      den = fmaf(w, lv[k], den);
#pragma unroll
      for (int j = 0; j < 4; ++j) a[j] = fmaf(w, av[k][j], a[j]);
    }
    M = Mn;
  };
  weigh(par, av0);
  // a parity's later batches (one parity over more than MCH splits: the bf16 kernel's two waves)
  for (int base = par + NPAR * MCH; base < ns; base += NPAR * MCH) {
    f4_t av[MCH];
    load_acc(base, av);
    weigh(base, av);
  }
  if constexpr (NPAR == 4) {
    // parities 1-3 hand (M, den, a) to parity 0 through LDS; one log-sum-exp over the four
    if (par > 0) {
      float* r = red + 6 * TPR * (par - 1);
      r[o] = M;
      r[TPR + o] = den;
      *reinterpret_cast<float4*>(r + 2 * TPR + 4 * o) = make_float4(a[0], a[1], a[2], a[3]);
    }
    __syncthreads();
    if (par == 0 && row < R) {
      float Mp[4] = {M, red[o], red[6 * TPR + o], red[12 * TPR + o]};
      const float Mx = max_ieee(max_ieee(Mp[0], Mp[1]), max_ieee(Mp[2], Mp[3]));
      float num[4] = {0.f, 0.f, 0.f, 0.f}, dsum = 0.0f;
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float e = Mp[p] == -INFINITY ? 0.0f : exp2_nonpos(Mp[p] - Mx);
        const float dp = p == 0 ? den : red[6 * TPR * (p - 1) + TPR + o];
        const float4 ap = p == 0 ? make_float4(a[0], a[1], a[2], a[3])
                                 : *reinterpret_cast<const float4*>(red + 6 * TPR * (p - 1) + 2 * TPR + 4 * o);
        dsum = fmaf(e, dp, dsum);
        num[0] = fmaf(e, ap.x, num[0]);
        num[1] = fmaf(e, ap.y, num[1]);
        num[2] = fmaf(e, ap.z, num[2]);
        num[3] = fmaf(e, ap.w, num[3]);
      }
      const float inv = 1.0f / dsum;
      const uint32_t lo = (uint32_t)f32_to_bf16(num[0] * inv) | ((uint32_t)f32_to_bf16(num[1] * inv) << 16);
      const uint32_t hi = (uint32_t)f32_to_bf16(num[2] * inv) | ((uint32_t)f32_to_bf16(num[3] * inv) << 16);
      *reinterpret_cast<uint2*>(out + (((int64_t)b * Hkv + hk) * R + row) * D + d0) = make_uint2(lo, hi);
    }
    return;
  }
  // parity 1 hands (M, den, a) to parity 0 through LDS
  float M1 = -INFINITY, den1 = 0.0f;
  float4 a1 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (NPAR == 2) {
    if (par == 1) {
      red[o] = M;
      red[TPR + o] = den;
      *reinterpret_cast<float4*>(red + 2 * TPR + 4 * o) = make_float4(a[0], a[1], a[2], a[3]);
    }
    __syncthreads();
    if (par == 0) {
      M1 = red[o];
      den1 = red[TPR + o];
      a1 = *reinterpret_cast<const float4*>(red + 2 * TPR + 4 * o);
    }
  }
  if (par == 0 && row < R) {
    const float Mx = max_ieee(M, M1);
    const float e0 = M == -INFINITY ? 0.0f : exp2_nonpos(M - Mx);
    const float e1 = M1 == -INFINITY ? 0.0f : exp2_nonpos(M1 - Mx);
    const float inv = 1.0f / (e0 * den + e1 * den1);
    const float r0v = (e0 * a[0] + e1 * a1.x) * inv, r1v = (e0 * a[1] + e1 * a1.y) * inv;
    const float r2v = (e0 * a[2] + e1 * a1.z) * inv, r3v = (e0 * a[3] + e1 * a1.w) * inv;
    const uint32_t lo = (uint32_t)f32_to_bf16(r0v) | ((uint32_t)f32_to_bf16(r1v) << 16);
    const uint32_t hi = (uint32_t)f32_to_bf16(r2v) | ((uint32_t)f32_to_bf16(r3v) << 16);
    *reinterpret_cast<uint2*>(out + (((int64_t)b * Hkv + hk) * R + row) * D + d0) = make_uint2(lo, hi);
  }
}

// Epilogue of the packed kernels. Per wave: the accumulator columns of the 4 key tiles of each
// query row are summed (lanes 4 and 8 apart in a row), the softmax sum and the two bias sums over
// all lanes; then the NW waves meet in LDS and their log-sum-exp merge is the workgroup's split
// partial: acc * (the wave's output factor of the dim's class, osc) + bias sum of the quant
// group, written with agent-scope stores. LDS layout: wave w's 4 rows at acc_lds + w acc_ws, rows
// FIN_ROW floats apart (a row of D floats, padded by 16 bytes so that the four rows' 16-byte
// writes of one instruction fall in different banks: each lane holding a row writes its dims with
// 8 ds_write_b128) -- in the wave's own tile buffers, free once its loop has ended, so the caller
// needs no barrier before this and waves that end early write while the others finish; st_lds
// [4][4][NW] (outside every wave's buffers): m, l, bias sum 0, bias sum 1 of each wave side by
// side, then [4][NW]: the output factors. Each output pair of dims then takes NW 8-byte reads and
// three NW-wide reads. Then the arrival count, and the last workgroup of the (sequence, KV head)
// merges all splits (merge_rows4, with acc_lds as its scratch). acc_lds and st_lds 16-byte
// aligned; each wave's area at least 4 FIN_ROW floats, wave 0's at least 6 * 128 + 256 (merge
// scratch), st_lds 20 NW floats.
// EVEN_ODD: accumulator tile 2j + p holds dims 32 j + 2 (4 lane group + r) + p (the 4-bit
// kernel's P.V operands); otherwise tile j holds dims 16 j + 4 lane group + r. osc: output factor
// of dim class 2 (dim / 64) + (EVEN_ODD ? dim & 1 : 0).
constexpr int FIN_ROW = D + 4;
template <int NW>
struct WaveVec;
template <>
struct WaveVec<4> {
  typedef float4 T;
  static __device__ __forceinline__ float get(const float4& v, int w) {
    return w == 0 ? v.x : w == 1 ? v.y : w == 2 ? v.z : v.w;
  }
};
template <>
struct WaveVec<2> {
  typedef float2 T;
  static __device__ __forceinline__ float get(const float2& v, int w) { return w == 0 ? v.x : v.y; }
};

template <int NW, bool EVEN_ODD = false>
__device__ void packed_finish(f4_t (&oacc)[8], float m_run, float lsum, float bsum0, float bsum1,
                              const float (&osc)[4], float* acc_lds, int acc_ws, float* st_lds,
                              int* sh_last, const AttnArgs& args, const DecodePlan& plan, int x,
                              int b, int hk, int R) {
  typedef typename WaveVec<NW>::T wvec;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int lc = lane & 15;
  const int lq4 = lane >> 4;
  const int Hkv = args.Hkv;
  // The sums are pinned in every lane before the branch below (the empty asm): left to itself
  // the compiler moved the adds into the branch, away from their DPP moves, and each step became
  // three instructions (zero, DPP move, add) instead of one v_add_f32_dpp -- at one wave per SIMD
  // that is ~1 us of issue time after the last tile.
#pragma unroll
  for (int dt = 0; dt < 8; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = oacc[dt][r];
      v += dpp<DPP_ROW_ROR4>(v);
      v += dpp<DPP_ROW_ROR8>(v);
      asm("" : "+v"(v));
      oacc[dt][r] = v;
    }
  float tot[3] = {lsum, bsum0, bsum1};
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    float v = tot[k];
    v += dpp<DPP_ROW_ROR4>(v);
    v += dpp<DPP_ROW_ROR8>(v);
    v = sum_xor16(v);
    v = sum_xor32(v);
    tot[k] = v;
  }
  if (lc < 4) {  // lane (lane group, row lc) holds the row's sums for dims of its lane group
    float* dst = acc_lds + wv * acc_ws + lc * FIN_ROW;
    if constexpr (EVEN_ODD) {
      // tiles 2 t and 2 t + 1: dims 32 t + 8 lq4 + 2 r + (0, 1)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f4_t e = oacc[2 * t], o = oacc[2 * t + 1];
        *reinterpret_cast<float4*>(dst + 32 * t + 8 * lq4) = make_float4(e[0], o[0], e[1], o[1]);
        *reinterpret_cast<float4*>(dst + 32 * t + 8 * lq4 + 4) = make_float4(e[2], o[2], e[3], o[3]);
      }
    } else {
#pragma unroll
      for (int dt = 0; dt < 8; ++dt)
        *reinterpret_cast<float4*>(dst + 16 * dt + 4 * lq4) =
            make_float4(oacc[dt][0], oacc[dt][1], oacc[dt][2], oacc[dt][3]);
    }
    if (lq4 == 0) {
      st_lds[(lc * 4 + 0) * NW + wv] = m_run;
      st_lds[(lc * 4 + 1) * NW + wv] = tot[0];
      st_lds[(lc * 4 + 2) * NW + wv] = tot[1];
      st_lds[(lc * 4 + 3) * NW + wv] = tot[2];
    }
    if (lane == 0) {
#pragma unroll
      for (int c = 0; c < 4; ++c) st_lds[(16 + c) * NW + wv] = osc[c];
    }
  }
  __syncthreads();
  // two dims (d, d + 1) of row col per item
  for (int o = tid; o < R * (D / 2); o += 64 * NW) {
    const int col = o / (D / 2);
    const int d = 2 * (o - col * (D / 2));
    const int g = d >> 6;
    const wvec m = *reinterpret_cast<const wvec*>(st_lds + (col * 4 + 0) * NW);
    const wvec bs = *reinterpret_cast<const wvec*>(st_lds + (col * 4 + 2 + g) * NW);
    const wvec os0 = *reinterpret_cast<const wvec*>(st_lds + (16 + 2 * g) * NW);
    const wvec os1 = *reinterpret_cast<const wvec*>(st_lds + (16 + 2 * g + (EVEN_ODD ? 1 : 0)) * NW);
    float2 ac[NW];
#pragma unroll
    for (int w = 0; w < NW; ++w)
      ac[w] = *reinterpret_cast<const float2*>(acc_lds + w * acc_ws + col * FIN_ROW + d);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = max_ieee(M, WaveVec<NW>::get(m, w));
    // the items of a row fill one wave, whose first lane also stores the row's (M, l)
    const wvec l = *reinterpret_cast<const wvec*>(st_lds + (col * 4 + 1) * NW);
    float a0 = 0.0f, a1 = 0.0f, lt = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float mw = WaveVec<NW>::get(m, w);
      const float e = mw == -INFINITY ? 0.0f : exp2_nonpos(mw - M);
      a0 += e * fmaf(ac[w].x, WaveVec<NW>::get(os0, w), WaveVec<NW>::get(bs, w));
      a1 += e * fmaf(ac[w].y, WaveVec<NW>::get(os1, w), WaveVec<NW>::get(bs, w));
      lt += mw == -INFINITY ? 0.0f : e * WaveVec<NW>::get(l, w);
    }
    const int64_t prow = (int64_t)x * Hkv * R + (int64_t)hk * R + col;
    st_agent2(args.part_acc + prow * D + d, a0, a1);
    if (d == 0) st_agent2(reinterpret_cast<float*>(args.part_ml + prow), M, lt);
  }

  // ---- split merge, fused: the last workgroup of (sequence, KV head) to store its partials
  // merges those of all the sequence's splits and writes the output rows. The partials are
  // written with agent-scope stores; every thread's stores (and its wave's last tile-counter
  // grab) have completed (vmcnt 0) before the barrier that precedes the arrival count, and the
  // last workgroup reads only after its count returned. The last arrival also resets the
  // arrival and tile counters to zero for the next call.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (tid == 0) {
    uint32_t* c = arrival_counter(args.counters, b * Hkv + hk);
    const uint32_t ns = (uint32_t)(plan.split_begin[b + 1] - plan.split_begin[b]);
    const uint32_t prev = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int last = prev + 1 == ns;
    if (last) {  // every workgroup of (b, hk) is past its loop: reset both counters
      __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(c + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    *sh_last = last;
  }
  __syncthreads();
  if (!*sh_last) return;
  // The loads of merge_rows4 are agent-scope (device-coherent level) and issued after the count
  // returned: they see every split's partials without an acquire fence (an invalidation of the
  // CU's and the XCD's caches, ~0.4 us on this path).
  merge_rows4<NW>(b, hk, Hkv, R, plan, args.part_acc, args.part_ml, args.out, acc_lds);
}

}  // namespace attn
}  // namespace lq
