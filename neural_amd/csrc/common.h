// Shared device helpers for the gfx950 kernels of the GPT-OSS MoE hot path.
//
// Numerics conventions (the reference's rounding points, restated):
//   * bf16 values travel as uint16 bit patterns; rb() is IEEE round-to-nearest-even fp32 -> bf16 -> fp32, the
//     rounding torch applies after every bf16 op and Triton's _rb applies explicitly (fused_core.py:67-69).
//   * E2M1 codes are dequantised by the gfx950 conversion instruction v_cvt_scalef32_pk_bf16_fp4 with scale 1.0
//     (exact: every E2M1 value is a bf16), the E8M0 scale 2^(s-127) is applied to a 32-element group partial with
//     v_ldexp_f32 (exact), as the algebra of reference mxfp4_kernels.py:116-123 allows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define NA_DEVICE __device__ __forceinline__

namespace na {

// ---- status codes returned by every extern "C" entry point (0 = launched)
enum Status : int {
  kOk = 0,
  kErrArgs = -1,        // null pointer, bad size or unsupported geometry
  kErrLaunch = -2,      // hipGetLastError after the launch
  kErrTooLarge = -3,    // a size beyond what the kernel's fixed buffers hold
  kErrResident = -4,    // the device cannot hold every workgroup of a launch at once (a launch that needs it)
};

// ---- GPT-OSS-120B expert geometry (reference neural/moe/layout.py:143-157)
constexpr int kH = 2880;          // hidden
constexpr int kGU = 5760;         // gate_up rows ([gate | up])
constexpr int kI = 2880;          // intermediate
constexpr int kGK = 90;           // groups of 32 per row (K = 2880)
constexpr int kRowBytes = kGK * 16;   // 1440 code bytes per row
constexpr int kPs4Row = 1 + kGK / 2;  // 46 B per PS4 scale row
constexpr long long kOffDownCodes = (long long)kGU * kRowBytes;                      // 8,294,400
constexpr long long kOffGateScales = kOffDownCodes + (long long)kH * kRowBytes;     // 12,441,600
constexpr long long kSlotRaw = kOffGateScales + (long long)(kGU + kH) * kGK;        // 13,219,200
constexpr long long kSlotPs4 = kOffGateScales + (long long)(kGU + kH) * kPs4Row;    // 12,839,040

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2_t;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16_t;
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// 128-bit weight load.  STREAM = true marks it non-temporal (weights are read once per step).
template <bool STREAM = false>
NA_DEVICE uint4 load16(const void* p) {
  u32x4_t v;
  if constexpr (STREAM) v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  else v = *reinterpret_cast<const u32x4_t*>(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Kernel arguments read at entry: an empty asm that takes each argument in scalar registers makes the compiler load
// them in one batch before the first instruction that depends on memory, instead of with one dependent scalar load
// (a round trip to the L2) at each first use further down the kernel.
NA_DEVICE void sgpr_use(const void* v) { asm volatile("" ::"s"(v)); }
NA_DEVICE void sgpr_use(long long v) { asm volatile("" ::"s"(v)); }
NA_DEVICE void sgpr_use(int v) { asm volatile("" ::"s"(v)); }
NA_DEVICE void sgpr_use(float v) { asm volatile("" ::"s"(v)); }
template <typename... T>
NA_DEVICE void args_at_entry(T... v) {
  (sgpr_use(v), ...);
}

NA_DEVICE float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even, in integer arithmetic (NaN -> quiet NaN).  The reference rounding of the
// device self-check; the kernels use the hardware conversion below.
NA_DEVICE uint16_t f32_to_bf16_int(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);   // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
typedef float f32x2v_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16 round to nearest even with gfx950's v_cvt_pk_bf16_f32 (one instruction for two values).  Checked
// against the integer rounding above over every bf16 boundary case by the device self-check na_selftest_bf16.
NA_DEVICE uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2v_t v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2v_t));
}

NA_DEVICE uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

NA_DEVICE float rb(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Two E2M1 codes of byte `sel` of `word` -> packed bf16 pair (low nibble -> element 0 in the low half).
template <int SEL>
NA_DEVICE uint32_t fp4x2_to_bf16x2(uint32_t word) {
  auto v = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, 1.0f, SEL);
  return __builtin_bit_cast(uint32_t, v);
}

// acc + w.x (two bf16 products, exact in fp32, accumulated in fp32)
NA_DEVICE float dot2_bf16(uint32_t w, uint32_t x, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), __builtin_bit_cast(bf16x2_t, x), acc,
                                          false);
}

// 32-element group dot: 16 code bytes (4 dwords) against 16 dwords of bf16 pairs of x.
NA_DEVICE float group_dot(const uint4 c, const uint32_t* x) {
  float a0 = 0.f, a1 = 0.f;
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    a0 = dot2_bf16(fp4x2_to_bf16x2<0>(w[d]), x[4 * d + 0], a0);
    a1 = dot2_bf16(fp4x2_to_bf16x2<1>(w[d]), x[4 * d + 1], a1);
    a0 = dot2_bf16(fp4x2_to_bf16x2<2>(w[d]), x[4 * d + 2], a0);
    a1 = dot2_bf16(fp4x2_to_bf16x2<3>(w[d]), x[4 * d + 3], a1);
  }
  return a0 + a1;
}

// Pairs are (token b, rank k) flattened as p = 4b + k, one bit each in a 64-bit mask.  Of each token's pairs in
// mask x, keep the lowest (the first of its ranks routed to the same expert): a token that lists one expert twice
// is computed once and its result written to every duplicate pair.
NA_DEVICE uint64_t first_per_token(uint64_t x) {
  const uint64_t b1 = (x << 1) & 0xEEEEEEEEEEEEEEEEull, b2 = (x << 2) & 0xCCCCCCCCCCCCCCCCull,
                 b3 = (x << 3) & 0x8888888888888888ull;
  return x & ~(b1 | b2 | b3);
}

// E8M0 exponent applied exactly: v * 2^(s-127)  (s = 255 -> inf for v != 0, as exp2(128) in fp32).
NA_DEVICE float e8m0_scale(float v, int s) {
  return s == 255 ? v * __builtin_inff() : __builtin_amdgcn_ldexpf(v, s - 127);
}

template <int CTRL>
NA_DEVICE float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// The value of lane i ^ 16 (v_permlane16_swap with v as both operands: odd rows <-> even rows) and of lane i ^ 32
// (v_permlane32_swap: upper half <-> lower half).  VALU permutations, no LDS round trip.  Must run with all lanes
// active.
NA_DEVICE float lane_xor16(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto p = __builtin_amdgcn_permlane16_swap(b, b, false, false);
  return __builtin_bit_cast(float, ((threadIdx.x >> 4) & 1) ? p[0] : p[1]);
}
NA_DEVICE float lane_xor32(float v) {
  const uint32_t b = __builtin_bit_cast(uint32_t, v);
  const auto p = __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __builtin_bit_cast(float, ((threadIdx.x >> 5) & 1) ? p[0] : p[1]);
}

// Sums by DPP and lane permutations.  Each returns, in the lanes stated, exactly the value of the xor butterfly
// v += v(lane ^ o) over the offsets in the order named (the same pairs, the same association), so the result does not
// depend on which of these implementations computed it; the other lanes hold partial or differently associated sums.
// row_shl:N (lane i reads lane i + N of its row) equals the xor partner for the lanes that the following levels read.
// Must run with all lanes active.

// Offsets 1, 2, 4, 8: exact in lane 0 of each row of 16.
NA_DEVICE float row16_sum(float v) {
  v += dpp<0xB1>(v);      // quad_perm [1,0,3,2]: lane i ^ 1
  v += dpp<0x4E>(v);      // quad_perm [2,3,0,1]: lane i ^ 2
  v += dpp<0x104>(v);     // row_shl:4: lane i + 4 (= i ^ 4 for lanes 0..3 of the row)
  return v + dpp<0x108>(v);   // row_shl:8: lane i + 8 (= i ^ 8 for lanes 0..7)
}

// Offsets 32, 16, 8, 4, 2, 1 (a whole wavefront): exact in lane 0.
NA_DEVICE float wave_sum_lane0(float v) {
  v += lane_xor32(v);
  v += lane_xor16(v);
  v += dpp<0x108>(v);     // row_shl:8: exact for lanes 0..7
  v += dpp<0x104>(v);     // row_shl:4: exact for lanes 0..3
  v += dpp<0x4E>(v);      // quad xor 2
  return v + dpp<0xB1>(v);    // quad xor 1
}

// Largest value over the 16 lanes of each row of the wavefront (lanes 16 r .. 16 r + 15), returned to all 16: DPP
// quad_perm [1,0,3,2], [2,3,0,1], then row_ror 4 and 8.  Must run with all lanes active.
NA_DEVICE float row16_max(float v) {
  v = fmaxf(v, dpp<0xB1>(v));
  v = fmaxf(v, dpp<0x4E>(v));
  v = fmaxf(v, dpp<0x124>(v));
  return fmaxf(v, dpp<0x128>(v));
}

// Sum over the 64 lanes of a wavefront, returned (wave-uniform) to every lane.  Must run with all lanes active.
// Fixed order: lane pairs, quads (DPP quad_perm), rows of 16 (DPP row_ror 4, 8), then the four row sums.
NA_DEVICE float wave_total(float v) {
  v += dpp<0xB1>(v);      // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);      // quad_perm [2,3,0,1]
  v += dpp<0x124>(v);     // row_ror:4
  v += dpp<0x128>(v);     // row_ror:8
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
  return (r0 + r1) + (r2 + r3);
}

// Clamped SwiGLU of one (gate, up) element pair with torch's bf16 op-by-op rounding
// (reference neural/q80/expert_runtime.py:63-72, server.py:2014-2021): inputs are bf16 values.
NA_DEVICE float swiglu_clamp_bf16(float g, float u, float alpha, float limit) {
  const float gate = fminf(g, limit);
  const float up = fminf(fmaxf(u, -limit), limit);
  const float t = rb(gate * alpha);
  const float s = rb(1.0f / (1.0f + expf(-t)));
  const float glu = rb(gate * s);
  return rb(rb(up + 1.0f) * glu);
}

}  // namespace na
