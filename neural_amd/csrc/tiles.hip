// gfx950 tile layout ("t950") of GPT-OSS-120B expert slots, its lossless repack from/to the store layouts, and the
// MFMA decode kernels that stream it.
//
// Layout of one slot (13,271,040 B): 540 row blocks of 16 rows (gate_up rows 0..5759 = blocks 0..359, down rows
// 0..2879 = blocks 360..539), each 24,576 B:
//   codes  [0, 23040):  22 full k-tiles of 1024 B (groups 4t..4t+3) and one half k-tile of 512 B (groups 88, 89).
//          In a full tile, lane l = 16 q + n owns bytes [16 l, 16 l + 16) = for j = 0..3 the 4 code bytes 4q..4q+3 of
//          (row n, group 4t + j), i.e. E2M1 elements 32 (4t + j) + 8q .. + 7 of row n.  In the half tile lane l owns
//          8 bytes at 8 l: the same for j = 0, 1 (groups 88, 89).
//   scales [23040, 24576): 16 rows x 96 B, byte n * 96 + g = E8M0 of (row n, group g), bytes 90..95 of a row = 0.
// One 128-bit load per lane of a full tile is exactly the B operands of four v_mfma_f32_16x16x32_bf16 (one per group:
// lane l supplies B[k = 8 (l / 16) + 0..7][n = l % 16]) for the 16 rows of the block.  The codes are the store's
// E2M1 nibbles unchanged and the scales the store's E8M0 bytes unchanged (PS4 rows are expanded), so the repack is a
// byte permutation plus padding and round-trips exactly (na_repack_from_t950).
#include "common.h"

#include <hip/hip_ext.h>

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

// ------------------------------------------------------------------------------------------------- repack
// Source row r of a slot in the store layout: code row bytes and its E8M0 scale of group g.
NA_DEVICE const uint8_t* store_code_row(const uint8_t* slot, int mat, int row) {
  return slot + (mat == 0 ? 0 : kOffDownCodes) + (long long)row * kRowBytes;
}

NA_DEVICE int store_scale(const uint8_t* slot, int ps4, int mat, int row, int g) {
  const int srow = ps4 ? kPs4Row : kGK;
  const uint8_t* s = slot + kOffGateScales + (long long)(mat == 0 ? row : kGU + row) * srow;
  if (!ps4) return s[g];
  const int b = s[1 + (g >> 1)];
  return s[0] + ((g & 1) ? (b >> 4) : (b & 15));
}

// One thread per 16 bytes of destination.  Per row block: 1440 code pieces (22 x 64 full-tile pieces, then 32 pieces
// of the half tile, two lanes' 8 bytes each) and 96 scale pieces (16 rows x 6).
constexpr int kTPiecesPerBlock = kTCodes / 16 + kTRows * kTScalePitch / 16;   // 1440 + 96 = 1536

__global__ __launch_bounds__(256) void k_repack_to_t950(const uint8_t* __restrict__ src, long long src_stride, int ps4,
                                                        uint8_t* __restrict__ dst, long long dst_stride, int n_slots) {
  const long long gidx = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long per_slot = (long long)(kTGateBlocks + kTDownBlocks) * kTPiecesPerBlock;
  if (gidx >= per_slot * n_slots) return;
  const int s = (int)(gidx / per_slot);
  const int rem = (int)(gidx - (long long)s * per_slot);
  const int blk = rem / kTPiecesPerBlock, pc = rem - blk * kTPiecesPerBlock;
  const int mat = blk < kTGateBlocks ? 0 : 1;
  const int row0 = (mat == 0 ? blk : blk - kTGateBlocks) * kTRows;
  const uint8_t* slot = src + (long long)s * src_stride;
  uint32_t out[4];
  if (pc < kTFull * 64) {                               // full tile t, lane l
    const int t = pc >> 6, l = pc & 63, n = l & 15, q = l >> 4;
    const uint8_t* row = store_code_row(slot, mat, row0 + n);
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = *reinterpret_cast<const uint32_t*>(row + (4 * t + j) * 16 + 4 * q);
  } else if (pc < kTCodes / 16) {                       // half tile: two lanes (2 x 8 bytes)
    const int lp = 2 * (pc - kTFull * 64);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int l = lp + h, n = l & 15, q = l >> 4;
      const uint8_t* row = store_code_row(slot, mat, row0 + n);
#pragma unroll
      for (int j = 0; j < 2; ++j) out[2 * h + j] = *reinterpret_cast<const uint32_t*>(row + (88 + j) * 16 + 4 * q);
    }
  } else {                                              // scales: row n, bytes 16c .. 16c + 15
    const int sp = pc - kTCodes / 16, n = sp / 6, c = sp - 6 * (sp / 6);
    uint8_t b[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int g = 16 * c + i;
      b[i] = g < kGK ? (uint8_t)store_scale(slot, ps4, mat, row0 + n, g) : 0;
    }
#pragma unroll
    for (int w = 0; w < 4; ++w)
      out[w] = (uint32_t)b[4 * w] | ((uint32_t)b[4 * w + 1] << 8) | ((uint32_t)b[4 * w + 2] << 16) |
               ((uint32_t)b[4 * w + 3] << 24);
  }
  uint8_t* d = dst + (long long)s * dst_stride + (long long)blk * kTBlock + 16LL * pc;
  *reinterpret_cast<uint4*>(d) = make_uint4(out[0], out[1], out[2], out[3]);
}

// Inverse: one thread per 16 bytes of t950 source code pieces (scatter), plus one thread per scale row.
__global__ __launch_bounds__(256) void k_repack_from_t950(const uint8_t* __restrict__ src, long long src_stride,
                                                          uint8_t* __restrict__ dst, long long dst_stride, int ps4,
                                                          int n_slots) {
  const long long gidx = (long long)blockIdx.x * 256 + threadIdx.x;
  constexpr int kPer = kTCodes / 16 + kTRows;          // code pieces + scale rows per block
  const long long per_slot = (long long)(kTGateBlocks + kTDownBlocks) * kPer;
  if (gidx >= per_slot * n_slots) return;
  const int s = (int)(gidx / per_slot);
  const int rem = (int)(gidx - (long long)s * per_slot);
  const int blk = rem / kPer, pc = rem - blk * kPer;
  const int mat = blk < kTGateBlocks ? 0 : 1;
  const int row0 = (mat == 0 ? blk : blk - kTGateBlocks) * kTRows;
  const uint8_t* b = src + (long long)s * src_stride + (long long)blk * kTBlock;
  uint8_t* slot = dst + (long long)s * dst_stride;
  if (pc < kTFull * 64) {
    const int t = pc >> 6, l = pc & 63, n = l & 15, q = l >> 4;
    const uint4 v = *reinterpret_cast<const uint4*>(b + 16 * pc);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint8_t* row = slot + (mat == 0 ? 0 : kOffDownCodes) + (long long)(row0 + n) * kRowBytes;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(row + (4 * t + j) * 16 + 4 * q) = w[j];
  } else if (pc < kTCodes / 16) {
    const int lp = 2 * (pc - kTFull * 64);
    const uint4 v = *reinterpret_cast<const uint4*>(b + 16 * pc);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int l = lp + h, n = l & 15, q = l >> 4;
      uint8_t* row = slot + (mat == 0 ? 0 : kOffDownCodes) + (long long)(row0 + n) * kRowBytes;
#pragma unroll
      for (int j = 0; j < 2; ++j) *reinterpret_cast<uint32_t*>(row + (88 + j) * 16 + 4 * q) = w[2 * h + j];
    }
  } else {
    const int n = pc - kTCodes / 16;
    const uint8_t* sr = b + kTCodes + n * kTScalePitch;
    const int srow = ps4 ? kPs4Row : kGK;
    uint8_t* d = slot + kOffGateScales + (long long)(mat == 0 ? row0 + n : kGU + row0 + n) * srow;
    if (!ps4) {
      for (int g = 0; g < kGK; ++g) d[g] = sr[g];
    } else {                                            // canonical PS4: base = row minimum
      int mn = 255;
      for (int g = 0; g < kGK; ++g) mn = min(mn, (int)sr[g]);
      d[0] = (uint8_t)mn;
      for (int k = 0; k < kGK / 2; ++k) d[1 + k] = (uint8_t)((sr[2 * k] - mn) | ((sr[2 * k + 1] - mn) << 4));
    }
  }
}

// ------------------------------------------------------------------------------------ MFMA decode kernels
// Work item = (distinct expert of the batch, 16-row output block); the KS waves of a workgroup split the 23 k-tiles,
// each accumulates D[token m][row n] with v_mfma_f32_16x16x32_bf16 (A = x of the expert's tokens, m < nt, else 0;
// B = codes dequantised in registers by v_cvt_scalef32_pk_bf16_fp4 with the group's E8M0 scale), and the partial D
// tiles are summed in a fixed order through LDS.  No cross-lane reduction and no per-group scaling pass: the MFMA
// accumulates over all of K.  Exact dequant: E2M1 x 2^(s-127) is a bf16 for the configured exponent range.
constexpr int kMaxTokT = 16;                 // tokens per expert the MFMA M dimension holds
constexpr int kXPitch = kH * 2 + 16;         // LDS bytes per staged token row (padded against bank conflicts)

NA_DEVICE float e8m0_f32(uint32_t s) { return __uint_as_float(s << 23); }

// 8 bf16 B values (one MFMA operand) from one code dword and its scale.
NA_DEVICE bf16x8_t dequant8(uint32_t w, float scale) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4v;
  u32x4v r;
  r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 0));
  r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 1));
  r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 2));
  r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, scale, 3));
  return __builtin_bit_cast(bf16x8_t, r);
}

// k-tile range of wave w of KS
template <int KS>
NA_DEVICE void ktile_range(int w, int& t0, int& t1) {
  t0 = (kTTiles * w) / KS;
  t1 = (kTTiles * (w + 1)) / KS;
}

constexpr int kMaxTilesPerWave = 23;

// Accumulate one row block over k-tiles [t0, t1) of this wave.  Code and scale loads of every tile are issued first.
// Code and scale registers of one row block over this wave's k-tiles [t0, t1).
template <int MT>
struct BlockRegs {
  uint4 c[MT];
  uint32_t sc[MT];
};

template <int MT>
NA_DEVICE void block_load(const uint8_t* blk, int lane, int t0, int t1, BlockRegs<MT>& r) {
  const int n = lane & 15;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = t0 + i;
    if (t < t1) {
      if (t < kTFull) {
        r.c[i] = load16(blk + t * 1024 + 16 * lane);
      } else {
        const uint2 h = *reinterpret_cast<const uint2*>(blk + kTFull * 1024 + 8 * lane);
        r.c[i] = make_uint4(h.x, h.y, 0, 0);
      }
      r.sc[i] = *reinterpret_cast<const uint32_t*>(blk + kTCodes + n * kTScalePitch + 4 * t);
    }
  }
}

// xs_lds points at this lane's staged x row (token m = lane % 16, clamped to a staged row: rows m >= nt only feed
// D rows that are never read).
template <int MT>
NA_DEVICE void block_compute(const BlockRegs<MT>& r, const uint8_t* xs_lds, int lane, int t0, int t1, f32x4_t& acc) {
  const int q = lane >> 4;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = t0 + i;
    if (t < t1) {
      const uint32_t w[4] = {r.c[i].x, r.c[i].y, r.c[i].z, r.c[i].w};
      const int ng = t < kTFull ? 4 : 2;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < ng) {
          const int g = 4 * t + j;
          const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(xs_lds + (32 * g + 8 * q) * 2);
          const bf16x8_t b = dequant8(w[j], e8m0_f32((r.sc[i] >> (8 * j)) & 0xff));
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
        }
      }
    }
  }
}

// x rows of up to XT tokens, staged through registers: piece p = tid + NTH * k (k < XP) of 360 * XT 16-byte pieces.
template <int XT, int NTH>
struct XRegs {
  static constexpr int XP = (XT * (kH / 8) + NTH - 1) / NTH;
  uint4 v[XP];
};

template <int XT, int NTH>
NA_DEVICE void x_load(const uint16_t* base, long long row_stride, const int* rows, int nt, XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = threadIdx.x + NTH * k;
    const int t = p / (kH / 8), pp = p - t * (kH / 8);
    if (t < XT && t < nt)
      xr.v[k] = load16(reinterpret_cast<const uint8_t*>(base + (long long)rows[t] * row_stride) + 16 * pp);
  }
}

template <int XT, int NTH>
NA_DEVICE void x_store(uint8_t* lds, int nt, const XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = threadIdx.x + NTH * k;
    const int t = p / (kH / 8), pp = p - t * (kH / 8);
    if (t < XT && t < nt) *reinterpret_cast<uint4*>(lds + t * kXPitch + 16 * pp) = xr.v[k];
  }
}

// Route of a decode batch (same rule as the store-layout kernels): the `item`-th distinct expert in first-appearance
// order; returns its id (or -1: no such item; 128: an invalid id) and the ascending pair list of its tokens.
NA_DEVICE int route_t950(const int64_t* ids, int npairs, int item, int& nt, int* pair, int& distinct) {
  const int lane = threadIdx.x & 63;
  int my = 129;
  if (lane < npairs) {
    const long long v = ids[lane];
    my = (v >= 0 && v < 128) ? (int)v : 128;
  }
  bool dup = false;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int o = __builtin_amdgcn_readlane(my, j);
    dup |= (j < lane) && (o == my);
  }
  uint64_t fm = __ballot(lane < npairs && !dup);
  distinct = __popcll(fm);
  if (item >= distinct) return -1;
  for (int i = 0; i < item; ++i) fm &= fm - 1;
  const int e = __builtin_amdgcn_readlane(my, __ffsll((long long)fm) - 1);
  uint64_t users = __ballot(lane < npairs && my == e);
  nt = 0;
#pragma unroll
  for (int t = 0; t < kMaxTokT; ++t) {
    pair[t] = 0;
    if (users) {
      pair[t] = __ffsll((long long)users) - 1;
      users &= users - 1;
      nt = t + 1;
    }
  }
  return e;
}

// Kernel templates: KS waves per workgroup split the k-tiles; XT token rows staged (at least the batch size B).
// Order: route -> x loads -> code and scale loads -> x to LDS, barrier -> MFMA tile by tile (each waits only for
// its own loads) -> fixed-order sum of the KS partial tiles through LDS -> epilogue in wave 0.

// gate_up: output block b (rows j = 16b .. 16b + 15 of gate and of up) -> h[pair, j]
template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_gate_up_t950(
    const uint16_t* __restrict__ x, const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool,
    long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
    const uint16_t* __restrict__ bias_gu, uint16_t* __restrict__ h, float alpha, float limit) {
  constexpr int MT = (kTTiles + KS - 1) / KS;
  __shared__ __align__(16) uint8_t xs[XT * kXPitch];
  __shared__ f32x4_t red[KS > 1 ? KS : 1][2][64];
  __shared__ int pairs_s[kMaxTokT];
  int pair[kMaxTokT], nt, distinct;
  const int e = route_t950(ids, 4 * B, blockIdx.x, nt, pair, distinct);
  if (e < 0 || e == 128) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const long long gid = expert_base + e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sbase = pool + slot * slot_bytes;
  const int b = blockIdx.y;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  int tok[XT];
#pragma unroll
  for (int t = 0; t < XT; ++t) tok[t] = pair[t] >> 2;
  XRegs<XT, 64 * KS> xr;
  x_load<XT, 64 * KS>(x, kH, tok, nt, xr);
  BlockRegs<MT> rg, ru;
  block_load<MT>(sbase + (long long)b * kTBlock, lane, t0, t1, rg);
  block_load<MT>(sbase + (long long)(kTUpBlock0 + b) * kTBlock, lane, t0, t1, ru);
  if (threadIdx.x == 0) {
#pragma unroll
    for (int t = 0; t < kMaxTokT; ++t) pairs_s[t] = pair[t];
  }
  x_store<XT, 64 * KS>(xs, nt, xr);
  __syncthreads();
  const uint8_t* xrow = xs + min(lane & 15, XT - 1) * kXPitch;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rg, xrow, lane, t0, t1, ag);
  block_compute<MT>(ru, xrow, lane, t0, t1, au);
  if constexpr (KS > 1) {
    red[wave][0][lane] = ag;
    red[wave][1][lane] = au;
    __syncthreads();
    if (wave != 0) return;
    ag = red[0][0][lane];
    au = red[0][1][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      ag += red[w][0][lane];
      au += red[w][1][lane];
    }
  }
  const int n = lane & 15, j = 16 * b + n;
  const uint16_t* bg = bias_gu ? bias_gu + gid * kGU : nullptr;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    if (m < nt) {
      float gb = rb(ag[r]), ub = rb(au[r]);
      if (bg) {
        gb = rb(gb + bf16_to_f32(bg[j]));
        ub = rb(ub + bf16_to_f32(bg[kI + j]));
      }
      h[(long long)pairs_s[m] * kI + j] = f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit));
    }
  }
}

// down: output block b (rows n = 16b .. 16b + 15) from each routed token's own h, + bias, x routing weight -> yw
template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_down_t950(
    const uint16_t* __restrict__ h, const int64_t* __restrict__ ids, const uint16_t* __restrict__ wts, int B,
    const uint8_t* __restrict__ pool, long long slot_bytes, const int64_t* __restrict__ slot_tab,
    long long expert_base, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  constexpr int MT = (kTTiles + KS - 1) / KS;
  __shared__ __align__(16) uint8_t xs[XT * kXPitch];
  __shared__ f32x4_t red[KS > 1 ? KS : 1][64];
  __shared__ int pairs_s[kMaxTokT];
  int pair[kMaxTokT], nt, distinct;
  const int e = route_t950(ids, 4 * B, blockIdx.x, nt, pair, distinct);
  if (e < 0) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.y;
  if (threadIdx.x == 0) {
#pragma unroll
    for (int t = 0; t < kMaxTokT; ++t) pairs_s[t] = pair[t];
  }
  if (e == 128) {                                      // invalid id: its pairs contribute +0
    __syncthreads();
    for (int i = threadIdx.x; i < nt * kTRows; i += 64 * KS)
      yw[(long long)pairs_s[i / kTRows] * kH + 16 * b + (i % kTRows)] = 0;
    return;
  }
  const long long gid = expert_base + e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sbase = pool + slot * slot_bytes;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  XRegs<XT, 64 * KS> xr;
  x_load<XT, 64 * KS>(h, kI, pair, nt, xr);
  BlockRegs<MT> rd;
  block_load<MT>(sbase + kTDownOff + (long long)b * kTBlock, lane, t0, t1, rd);
  x_store<XT, 64 * KS>(xs, nt, xr);
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rd, xs + min(lane & 15, XT - 1) * kXPitch, lane, t0, t1, acc);
  if constexpr (KS > 1) {
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    acc = red[0][lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) acc += red[w][lane];
  }
  const int n = 16 * b + (lane & 15);
  const uint16_t* bd = bias_dn ? bias_dn + gid * kH : nullptr;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    if (m < nt) {
      float y = rb(acc[r]);
      if (bd) y = rb(y + bf16_to_f32(bd[n]));
      const int p = pairs_s[m];
      yw[(long long)p * kH + n] = f32_to_bf16(y * bf16_to_f32(wts[p]));
    }
  }
}

__global__ __launch_bounds__(256) void k_combine_t950(const uint32_t* __restrict__ yw, int B, uint32_t* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= B * (kH / 2)) return;
  const int b = i / (kH / 2), n2 = i - b * (kH / 2);
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t v = yw[(long long)(4 * b + k) * (kH / 2) + n2];
    a0 += bf16_to_f32((uint16_t)(v & 0xffff));
    a1 += bf16_to_f32((uint16_t)(v >> 16));
  }
  out[i] = (uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16);
}

template <typename... KArgs, typename... Args>
static void launch_t(void (*kern)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                     Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, e0, e1, 0, static_cast<KArgs>(args)...);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, stream, static_cast<KArgs>(args)...);
}

typedef void (*GateUpT)(const uint16_t*, const int64_t*, int, const uint8_t*, long long, const int64_t*, long long,
                        const uint16_t*, uint16_t*, float, float);
typedef void (*DownT)(const uint16_t*, const int64_t*, const uint16_t*, int, const uint8_t*, long long, const int64_t*,
                      long long, const uint16_t*, uint16_t*);

template <int KS>
static GateUpT gate_up_t950_xt(int xt) {
  return xt == 1 ? k_moe_gate_up_t950<KS, 1> : xt == 2 ? k_moe_gate_up_t950<KS, 2>
       : xt == 4 ? k_moe_gate_up_t950<KS, 4> : k_moe_gate_up_t950<KS, 8>;
}
static GateUpT pick_gate_up_t950(int ks, int xt) {
  return ks == 1 ? gate_up_t950_xt<1>(xt) : ks == 2 ? gate_up_t950_xt<2>(xt) : gate_up_t950_xt<4>(xt);
}
template <int KS>
static DownT down_t950_xt(int xt) {
  return xt == 1 ? k_moe_down_t950<KS, 1> : xt == 2 ? k_moe_down_t950<KS, 2>
       : xt == 4 ? k_moe_down_t950<KS, 4> : k_moe_down_t950<KS, 8>;
}
static DownT pick_down_t950(int ks, int xt) {
  return ks == 1 ? down_t950_xt<1>(xt) : ks == 2 ? down_t950_xt<2>(xt) : down_t950_xt<4>(xt);
}

}  // namespace na

using namespace na;

extern "C" {

long long na_t950_slot_bytes(void) { return kTSlot; }

int na_repack_to_t950(const void* src, long long src_stride, int src_ps4, void* dst, long long dst_stride,
                      int n_slots, hipStream_t stream) {
  if (!src || !dst || n_slots <= 0 || (src_ps4 != 0 && src_ps4 != 1)) return kErrArgs;
  if (src_stride < (src_ps4 ? kSlotPs4 : kSlotRaw) || dst_stride < kTSlot) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(dst) & 15) || (dst_stride & 15) || (reinterpret_cast<uintptr_t>(src) & 3) ||
      (src_stride & 3))
    return kErrArgs;
  const long long n = (long long)(kTGateBlocks + kTDownBlocks) * kTPiecesPerBlock * n_slots;
  launch_t(k_repack_to_t950, dim3((unsigned)((n + 255) / 256)), dim3(256), stream, nullptr, nullptr,
           (const uint8_t*)src, src_stride, src_ps4, (uint8_t*)dst, dst_stride, n_slots);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_repack_from_t950(const void* src, long long src_stride, void* dst, long long dst_stride, int dst_ps4,
                        int n_slots, hipStream_t stream) {
  if (!src || !dst || n_slots <= 0 || (dst_ps4 != 0 && dst_ps4 != 1)) return kErrArgs;
  if (src_stride < kTSlot || dst_stride < (dst_ps4 ? kSlotPs4 : kSlotRaw)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(src) & 15) || (src_stride & 15) || (reinterpret_cast<uintptr_t>(dst) & 3) ||
      (dst_stride & 3))
    return kErrArgs;
  const long long n = (long long)(kTGateBlocks + kTDownBlocks) * (kTCodes / 16 + kTRows) * n_slots;
  launch_t(k_repack_from_t950, dim3((unsigned)((n + 255) / 256)), dim3(256), stream, nullptr, nullptr,
           (const uint8_t*)src, src_stride, (uint8_t*)dst, dst_stride, dst_ps4, n_slots);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_moe_decode_t950(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                       long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                       const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha, float limit,
                       int k_split, void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !h_scratch || !yw_scratch || B <= 0) return kErrArgs;
  if (B > 8) return kErrTooLarge;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if (k_split <= 0) k_split = 4;
  if (k_split != 1 && k_split != 2 && k_split != 4) return kErrArgs;
  hipEvent_t ev[6] = {};
  if (events)
    for (int i = 0; i < 6; ++i) ev[i] = (hipEvent_t)events[i];
  const int items = 4 * B;
  const dim3 g1(items, kTDownBlocks), g2(items, kTDownBlocks);
  const dim3 blk(64 * k_split);
  const int xt = B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;
  auto gu = pick_gate_up_t950(k_split, xt);
  auto dn = pick_down_t950(k_split, xt);
  launch_t(gu, g1, blk, stream, ev[0], ev[1], (const uint16_t*)x, topk_ids, B, (const uint8_t*)pool, slot_bytes,
           slot_tab, expert_base, (const uint16_t*)bias_gu, (uint16_t*)h_scratch, alpha, limit);
  launch_t(dn, g2, blk, stream, ev[2], ev[3], (const uint16_t*)h_scratch, topk_ids, (const uint16_t*)topk_w, B,
           (const uint8_t*)pool, slot_bytes, slot_tab, expert_base, (const uint16_t*)bias_dn, (uint16_t*)yw_scratch);
  if (out)
    launch_t(k_combine_t950, dim3((B * kH / 2 + 255) / 256), dim3(256), stream, ev[4], ev[5],
             (const uint32_t*)yw_scratch, B, (uint32_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
