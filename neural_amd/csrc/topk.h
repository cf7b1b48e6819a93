// Top 4 of a layer's 128 router logits and their softmax, shared by the router (core.hip: the decode router, the
// attention block's router phase, the prompt rows) and the single-launch expert body that selects its experts from
// the logits itself (tiles.hip).  One wave holds the 128 logits (lane l: logits l and l + 64).
#pragma once
#include "common.h"

namespace na {

// Top 4 of 128 logits held by one wave (lane l: logits l and l + 64) by repeated argmax, lowest index on ties; lanes
// 0..3 write ids[k] and the weights bf16(exp(v_k - v_0) / sum_k exp(v_k - v_0)) (the reference's softmax over the
// four, fused_core.py:486-502).  The logits are bf16 values (the router rounds them), so (value, index) fits one
// 32-bit key that orders exactly as the comparison "larger value, then smaller index" (-0 as +0): each round is one
// wavefront maximum of keys by DPP and four lane reads, with no LDS round trip.
NA_DEVICE uint32_t top_key(float v, int idx) {
  uint32_t b = __float_as_uint(v) >> 16;
  if (b == 0x8000u) b = 0;
  const uint32_t ord = (b & 0x8000u) ? (~b & 0xFFFFu) : (b | 0x8000u);
  return (ord << 16) | (uint32_t)(0xFFFF - idx);
}
NA_DEVICE float top_key_value(uint32_t key) {
  const uint32_t ord = key >> 16;
  return bf16_to_f32((uint16_t)((ord & 0x8000u) ? (ord & 0x7FFFu) : (~ord & 0xFFFFu)));
}
template <int CTRL>
NA_DEVICE uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
// The largest key of the wavefront, in every lane: DPP maxima within each row of 16, then the four rows'.
NA_DEVICE uint32_t wave_max_key(uint32_t k) {
  k = max(k, dpp_u32<0xB1>(k));
  k = max(k, dpp_u32<0x4E>(k));
  k = max(k, dpp_u32<0x124>(k));
  k = max(k, dpp_u32<0x128>(k));
  const uint32_t r0 = (uint32_t)__builtin_amdgcn_readlane((int)k, 0), r1 = (uint32_t)__builtin_amdgcn_readlane((int)k, 16);
  const uint32_t r2 = (uint32_t)__builtin_amdgcn_readlane((int)k, 32), r3 = (uint32_t)__builtin_amdgcn_readlane((int)k, 48);
  return max(max(r0, r1), max(r2, r3));
}
// The 4 largest (value, index) of the wave's logits, in every lane, in rank order (repeated argmax, lowest index on
// ties, -0 as +0).
NA_DEVICE void top4_select(float v0, float v1, int lane, float (&tv)[4], int (&ti)[4]) {
  uint32_t k0 = top_key(v0, lane), k1 = top_key(v1, lane + 64);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t best = wave_max_key(max(k0, k1));
    tv[k] = top_key_value(best);
    ti[k] = 0xFFFF - (int)(best & 0xFFFFu);
    if (k0 == best) k0 = 0;                          // every real key is above 0
    if (k1 == best) k1 = 0;
  }
}
// Rank r's routing weight: bf16(exp(v_r - v_0) / sum_k exp(v_k - v_0)) (the reference's softmax over the four,
// fused_core.py:486-502); r is per lane.
NA_DEVICE uint16_t top4_weight(const float (&tv)[4], int r) {
  float ex[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) ex[k] = expf(tv[k] - tv[0]);
  const float sum = ((ex[0] + ex[1]) + ex[2]) + ex[3];
  const float mine = r == 0 ? ex[0] : r == 1 ? ex[1] : r == 2 ? ex[2] : ex[3];
  return f32_to_bf16(mine / sum);
}
// Rank r's expert id (r per lane, 0..3).
NA_DEVICE int top4_id(const int (&ti)[4], int r) { return r == 0 ? ti[0] : r == 1 ? ti[1] : r == 2 ? ti[2] : ti[3]; }
// Lanes 0..3 write ids[lane] and wts[lane].
NA_DEVICE void top4_softmax(float v0, float v1, int lane, int64_t* __restrict__ ids, uint16_t* __restrict__ wts) {
  float tv[4];
  int ti[4];
  top4_select(v0, v1, lane, tv, ti);
  if (lane < 4) {
    ids[lane] = top4_id(ti, lane);
    wts[lane] = top4_weight(tv, lane);
  }
}

}  // namespace na
