// gfx950 tile layout ("t950") of one GPT-OSS-120B expert slot, shared by the repack, decode and prefill kernels.
//
// 13,271,040 B per slot: 540 row blocks of 16 rows (gate_up rows 0..5759 = blocks 0..359, the up half from block 180;
// down rows 0..2879 = blocks 360..539), each 24,576 B:
//   codes  [0, 23040):  22 full k-tiles of 1024 B (groups 4t..4t+3) and one half k-tile of 512 B (groups 88, 89).
//          In a full tile, lane l = 16 q + n owns bytes [16 l, 16 l + 16) = for j = 0..3 the 4 code bytes 4q..4q+3 of
//          (row n, group 4t + j), i.e. E2M1 elements 32 (4t + j) + 8q .. + 7 of row n.  In the half tile lane l owns
//          8 bytes at 8 l: the same for j = 0, 1 (groups 88, 89).
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

// 8 bf16 B values (one MFMA operand) from one code dword and its scale: v_cvt_scalef32_pk_bf16_fp4 per byte (low
// nibble first), exact for the E8M0 range of the store (E2M1 x 2^(s-127) is a bf16).
NA_DEVICE bf16x8_t dequant8(uint32_t w, float scale) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4v;
  u32x4v r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
  return __builtin_bit_cast(bf16x8_t, r);
}

}  // namespace na
