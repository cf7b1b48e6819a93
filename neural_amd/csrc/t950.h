// gfx950 tile layout ("t950") of one GPT-OSS-120B expert slot, shared by the repack, decode and prefill kernels.
//
// 13,271,040 B per slot: 540 row blocks of 16 rows (gate_up rows 0..5759 = blocks 0..359, the up half from block 180;
// down rows 0..2879 = blocks 360..539), each 24,576 B:
//   codes  [0, 23040):  90 groups of 256 B, group-major: byte 256 g + 16 n + b = code byte b of (row n, group g).
//          k-tile t (groups 4t..4t+3; the last, t = 22, only groups 88 and 89 in 512 B) is the 1024 B at 1024 t, and
//          lane l = 16 kb + n owns its bytes [16 l, 16 l + 16) = E2M1 elements 32 (4t + kb) .. + 31 of row n: one
//          128-bit load per lane is the FP4 B operand of v_mfma_scale_f32_16x16x128_f8f6f4 as it stands.
//   scales [23040, 24576): 16 rows x 96 B, byte n * 96 + g = E8M0 of (row n, group g), bytes 90..95 of a row = 0.
#pragma once
#include "common.h"

namespace na {

constexpr int kTRows = 16;
constexpr int kTFull = 22;
constexpr int kTTiles = 23;                         // 22 full + 1 half
constexpr int kTCodes = kTFull * 1024 + 512;        // 23,040
constexpr int kTScalePitch = 96;
constexpr int kTBlock = kTCodes + kTRows * kTScalePitch;   // 24,576
constexpr int kTGateBlocks = kGU / kTRows;          // 360
constexpr int kTDownBlocks = kH / kTRows;           // 180
constexpr long long kTSlot = (long long)(kTGateBlocks + kTDownBlocks) * kTBlock;   // 13,271,040
constexpr long long kTDownOff = (long long)kTGateBlocks * kTBlock;
constexpr int kTUpBlock0 = kI / kTRows;             // first row block of the up half of gate_up (180)

NA_DEVICE float e8m0_f32(uint32_t s) { return __uint_as_float(s << 23); }

typedef int mfma_i32x8_t __attribute__((ext_vector_type(8)));
typedef short fp8x2_t __attribute__((ext_vector_type(2)));

// ---- activations as E4M3 for the block-scaled MFMA.  A bf16 row x becomes two E4M3 rows, hi = RNE(x / s_hi) and
// lo = RNE((x - hi s_hi) / s_lo), each with one E8M0 scale per 32-element block: s = 2^(e - 7) for the block's largest
// magnitude m (2^e <= m < 2^(e+1)), so every scaled value is below 256 and the conversion never saturates.  hi s_hi
// carries the top 4 significant bits of an element and lo s_lo the remaining 4 bits of a bf16, exactly for every
// element within 2^13 of its block's largest magnitude and to within 2^-21 of that magnitude below it, so the MFMA's
// products hi w + lo w are the reference's exact bf16 x E2M1 products to that precision.  The conversions are gfx950's
// v_cvt_scalef32_pk_fp8_bf16 / _fp8_f32 (x / scale, round to nearest even, OCP E4M3) and v_cvt_scalef32_pk_f32_fp8,
// which decodes hi exactly for the remainder (checked on the device by na_selftest_x8).
constexpr int kX8Pitch = kH + 16;   // LDS bytes per E4M3 row: 16 rows at one offset hit 16 disjoint bank quads
constexpr int kX8ScPitch = 96;      // E8M0 bytes per row (90 blocks)
constexpr int kChunks = kH / 8;     // 360 chunks of 8 elements per row, 4 chunks per 32-element block

// Biased E8M0 exponent of the scale of a block whose largest magnitude is m: 2^(e - 7), kept in [2^-126, 2^127].
NA_DEVICE uint32_t x8_scale_byte(float m) {
  const int e = (int)((__float_as_uint(m) >> 23) & 0xff);   // biased exponent of m (0 for zero and subnormals)
  return (uint32_t)min(max(e - 7, 1), 254);
}

// E4M3 codes of the 8 bf16 elements of one chunk: hi and lo (4 codes per dword, element order), sh / sl = the E8M0
// bytes of the chunk's 32-element block.  The 4 chunks of a block sit in 4 consecutive lanes (lane % 4 = chunk % 4):
// every lane of the wave must call it (the block maxima are exchanged between lanes).
NA_DEVICE void x8_quant_chunk(uint4 v, uint2& hi, uint2& lo, uint32_t& sh, uint32_t& sl) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float f[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_to_f32((uint16_t)(w[i] & 0xffff));
    f[2 * i + 1] = bf16_to_f32((uint16_t)(w[i] >> 16));
  }
  float m = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(f[i]));
  m = fmaxf(m, __shfl_xor(m, 1));
  m = fmaxf(m, __shfl_xor(m, 2));
  sh = x8_scale_byte(m);
  const float s_hi = e8m0_f32(sh);
  uint32_t hc[2];
  float r[8];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    fp8x2_t o = {0, 0};
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2_t, w[2 * d]), s_hi, false);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(o, __builtin_bit_cast(bf16x2_t, w[2 * d + 1]), s_hi, true);
    hc[d] = __builtin_bit_cast(uint32_t, o);
    const auto b0 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hc[d], s_hi, false);
    const auto b1 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hc[d], s_hi, true);
    r[4 * d + 0] = f[4 * d + 0] - b0[0];
    r[4 * d + 1] = f[4 * d + 1] - b0[1];
    r[4 * d + 2] = f[4 * d + 2] - b1[0];
    r[4 * d + 3] = f[4 * d + 3] - b1[1];
  }
  float mr = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) mr = fmaxf(mr, fabsf(r[i]));
  mr = fmaxf(mr, __shfl_xor(mr, 1));
  mr = fmaxf(mr, __shfl_xor(mr, 2));
  sl = x8_scale_byte(mr);
  const float s_lo = e8m0_f32(sl);
  uint32_t lc[2];
#pragma unroll
  for (int d = 0; d < 2; ++d) {
    fp8x2_t o = {0, 0};
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, r[4 * d], r[4 * d + 1], s_lo, false);
    o = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o, r[4 * d + 2], r[4 * d + 3], s_lo, true);
    lc[d] = __builtin_bit_cast(uint32_t, o);
  }
  hi = make_uint2(hc[0], hc[1]);
  lo = make_uint2(lc[0], lc[1]);
}

}  // namespace na
