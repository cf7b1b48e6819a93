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
#include "t950.h"

#include <hip/hip_ext.h>

namespace na {

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
// Code tiles are read with non-temporal 128-bit loads (each weight byte is used once per step); a row block's 1,536
// scale bytes are read by the workgroup with coalesced 16-byte loads and staged in LDS, so that each wave reads its
// scales from LDS instead of issuing one scattered 64-lane load per tile.
constexpr int kMaxTokT = 16;                 // tokens per expert the MFMA M dimension holds
constexpr int kXPitch = kH * 2 + 16;         // LDS bytes per staged token row (padded against bank conflicts)
constexpr int kScPitch = 112;                // LDS bytes per staged scale row: 28 dwords, so 16 rows hit 16 banks
constexpr int kScLds = kTRows * kScPitch;    // 1,792 LDS bytes per staged row block
constexpr int kScPieces = kTRows * kTScalePitch / 16;   // 96 16-byte pieces of scales per row block

// k-tile range of wave w of KS
template <int KS>
NA_DEVICE void ktile_range(int w, int& t0, int& t1) {
  t0 = (kTTiles * w) / KS;
  t1 = (kTTiles * (w + 1)) / KS;
}

// Code registers of one row block over this wave's k-tiles [t0, t1).
template <int MT>
struct CodeRegs {
  uint4 c[MT];
};

// Branch-free: every wave issues exactly MT loads, all before any wait.  Slot i holds tile t0 + i when that is below
// t1, else a copy of tile t0 whose codes block_compute replaces by zeros (E2M1 code 0 is +0, so the slot adds
// nothing).  The half tile is read as 16 bytes per lane at 8-byte stride (the last lane's excess bytes fall in the
// block's scale rows) and block_compute zeroes its groups 90 and 91.  The zeroing happens at the use, so that no
// wait for the codes is placed before the first barrier.
NA_DEVICE int slot_tile(int t0, int t1, int i) { return t0 + i < t1 ? t0 + i : t0; }

template <int MT>
NA_DEVICE void code_load(const uint8_t* blk, int lane, int t0, int t1, CodeRegs<MT>& r) {
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = slot_tile(t0, t1, i);
    const int off = t < kTFull ? t * 1024 + 16 * lane : kTFull * 1024 + 8 * lane;
    r.c[i] = load16<true>(blk + off);
  }
}

// Scale rows of NB row blocks (NB = 1 or 2) through registers to LDS: piece p = tid + NTH k of NB x 96 pieces;
// piece p of block p / 96 is bytes 16 c .. 16 c + 15 of scale row n (p % 96 = 6 n + c).
template <int NB, int NTH>
struct ScaleRegs {
  static constexpr int SP = (NB * kScPieces + NTH - 1) / NTH;
  uint4 v[SP];
};

// Branch-free: thread tid handles piece min(tid + NTH k, NB x 96 - 1); the clamped duplicates store the same bytes.
template <int NB, int NTH>
NA_DEVICE void scale_load(int tid, const uint8_t* blk0, const uint8_t* blk1, ScaleRegs<NB, NTH>& r) {
#pragma unroll
  for (int k = 0; k < ScaleRegs<NB, NTH>::SP; ++k) {
    const int p = min(tid + NTH * k, NB * kScPieces - 1);
    const int bi = p >= kScPieces ? 1 : 0, q = p - bi * kScPieces;
    r.v[k] = load16((bi ? blk1 : blk0) + kTCodes + 16 * q);
  }
}

template <int NB, int NTH>
NA_DEVICE void scale_store(int tid, uint8_t* lds, const ScaleRegs<NB, NTH>& r) {
#pragma unroll
  for (int k = 0; k < ScaleRegs<NB, NTH>::SP; ++k) {
    const int p = min(tid + NTH * k, NB * kScPieces - 1);
    const int bi = p >= kScPieces ? 1 : 0, q = p - bi * kScPieces, n = q / 6, c = q - 6 * n;
    *reinterpret_cast<uint4*>(lds + bi * kScLds + n * kScPitch + 16 * c) = r.v[k];
  }
}

// xs_lds points at this lane's A row (token m = lane % 16; rows m >= nt only feed D rows that are never read),
// sc_row at this lane's staged scale row (row n = lane % 16 of the block).
template <int MT>
NA_DEVICE void block_compute(const CodeRegs<MT>& r, const uint8_t* sc_row, const uint8_t* xs_lds, int lane, int t0,
                             int t1, f32x4_t& acc) {
  const int q = lane >> 4;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = slot_tile(t0, t1, i);
    const bool live = t0 + i < t1, full = live && t < kTFull;
    const uint32_t w[4] = {live ? r.c[i].x : 0u, live ? r.c[i].y : 0u, full ? r.c[i].z : 0u, full ? r.c[i].w : 0u};
    const uint32_t sc = *reinterpret_cast<const uint32_t*>(sc_row + 4 * t);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int g = min(4 * t + j, kGK - 1);             // zeroed groups 90, 91 read a finite A row
      const bf16x8_t a = *reinterpret_cast<const bf16x8_t*>(xs_lds + (32 * g + 8 * q) * 2);
      const bf16x8_t b = dequant8(w[j], e8m0_f32((sc >> (8 * j)) & 0xff));
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
    }
  }
}

// Activation rows (x, or h) of up to XT tokens, staged through registers: piece p = tid + NTH * k (k < XP) of
// 360 * XT 16-byte pieces.
template <int XT, int NTH>
struct XRegs {
  static constexpr int XP = (XT * (kH / 8) + NTH - 1) / NTH;
  uint4 v[XP];
};

// Thread tid stages pieces p = tid + NTH k < nt x 360 (a per-lane predicate, no branch), i.e. rows t < nt
// (1 <= nt <= XT) of the staged block, row t = source row row_of(t).  Staged rows t >= nt are not written: they only
// feed D rows m >= nt, which are never read (each MFMA output row depends on its own A row only).
template <int XT, int NTH, typename RowOf>
NA_DEVICE void x_load(int tid, const uint16_t* base, long long row_stride, RowOf row_of, int nt, XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = tid + NTH * k;
    const int t = p / (kH / 8), pp = p - t * (kH / 8);
    if (p < nt * (kH / 8))
      xr.v[k] = load16(reinterpret_cast<const uint8_t*>(base + (long long)row_of(t) * row_stride) + 16 * pp);
  }
}

template <int XT, int NTH>
NA_DEVICE void x_store(int tid, uint8_t* lds, int nt, const XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = tid + NTH * k;
    const int t = p / (kH / 8), pp = p - t * (kH / 8);
    if (p < nt * (kH / 8)) *reinterpret_cast<uint4*>(lds + t * kXPitch + 16 * pp) = xr.v[k];
  }
}

// Store the bf16 values v held as D columns n = lane % 16 (16 lanes per D row) as 32-bit pairs: even lanes write
// (v[n], v[n + 1]) to row_ptr + n.  All lanes must call it (it exchanges values between neighbouring lanes).
NA_DEVICE void store_row_pairs(uint16_t* row_ptr, uint16_t v, bool ok) {
  const int lane = threadIdx.x & 63;
  const uint32_t hi = (uint32_t)__shfl_xor((int)v, 1) & 0xffff;
  if (ok && !(lane & 1)) *reinterpret_cast<uint32_t*>(row_ptr + (lane & 15)) = (uint32_t)v | (hi << 16);
}

// The id of this lane's pair (lanes past the pairs re-read the last one): the first read of a decode kernel, issued
// by its first instructions (the id pointer arrives preloaded in scalar registers) so that its round trip overlaps
// the loads of the remaining kernel arguments.
NA_DEVICE long long route_ids_load(const int64_t* ids, int npairs) {
  return ids[min((int)(threadIdx.x & 63), npairs - 1)];
}

// Route of a decode batch (same rule as the store-layout kernels): the `item`-th distinct expert in first-appearance
// order; returns its id (or -1: no such item; 128: an invalid id), `all` = the mask of its pairs (bit p = pair
// p = 4 token + k), `users` = the first of them per token (first_per_token) and nt = their number (the tokens routed
// to the expert, <= B); pair_at(users, m) is the m-th user in ascending order.  The MFMA rows are the users; each
// result is written to every pair of its token in `all`.  `valid` = distinct experts with a valid id (the invalid
// marker 128 excluded).  Pair lists stay masks in scalar registers: an indexed register array would be placed in
// scratch memory.
// v = the id of this lane's pair, from route_ids_load.  MAXP bounds the pair count (npairs <= MAXP <= 32): the dedupe
// compares each pair with the MAXP - 1 before it.
template <int MAXP>
NA_DEVICE int route_t950(long long v, int npairs, int item, int& nt, uint64_t& users, uint64_t& all, int& distinct,
                         int& valid) {
  static_assert(MAXP >= 1 && MAXP <= 32, "at most 8 tokens x top-4 pairs");
  const int lane = threadIdx.x & 63;
  const int my = lane < npairs ? ((v >= 0 && v < 128) ? (int)v : 128) : 129;
  bool dup = false;
#pragma unroll
  for (int j = 0; j < MAXP - 1; ++j) {
    const int o = __builtin_amdgcn_readlane(my, j);
    dup |= (j < lane) && (o == my);
  }
  uint64_t fm = __ballot(lane < npairs && !dup);
  distinct = __popcll(fm);
  valid = __popcll(__ballot(lane < npairs && !dup && my != 128));
  users = 0;
  all = 0;
  nt = 0;
  if (item >= distinct) return -1;
  for (int i = 0; i < item; ++i) fm &= fm - 1;
  const int e = __builtin_amdgcn_readlane(my, __ffsll((long long)fm) - 1);
  all = __ballot(lane < npairs && my == e);
  users = first_per_token(all);
  const int nu = __popcll(users);
  nt = nu < kMaxTokT ? nu : kMaxTokT;
  return e;
}

// The pairs of user pair p's token that `all` routes to the same expert, as a 4-bit mask over the ranks k.
NA_DEVICE uint32_t token_dups(uint64_t all, int p) { return (uint32_t)(all >> (p & ~3)) & 0xFu; }

// The m-th pair (ascending) of a route's mask, 0 <= m < kMaxTokT; the mask is uniform, the walk is scalar.
NA_DEVICE int pair_at(uint64_t users, int m) {
  int p = __ffsll((long long)users) - 1;
  uint64_t u = users;
#pragma unroll
  for (int t = 1; t < kMaxTokT; ++t) {
    u &= u - 1;
    const int pt = __ffsll((long long)u) - 1;
    p = (t == m) ? pt : p;
  }
  return p;
}

// The duplicate pairs' rows: for D row m < nt (user pair p), the same values v[r] also go to every other pair of
// p's token that `all` routes to the expert (row stride `stride` elements, columns 16b .. 16b + 15).  All lanes call
// it.  Kept out of line of the common path, which stores only the users' rows.
__device__ __noinline__ void dup_rows_store(uint16_t* base, int stride, uint64_t users, uint64_t all, int nt, int b,
                                            uint16_t v0, uint16_t v1, uint16_t v2, uint16_t v3) {
  const int lane = threadIdx.x & 63;
  const uint16_t v[4] = {v0, v1, v2, v3};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    const int p = pair_at(users, min(m, nt - 1));
    const uint32_t dm = token_dups(all, p) & ~(1u << (p & 3));
    for (int k = 0; k < 4; ++k)
      store_row_pairs(base + (long long)((p & ~3) + k) * stride + 16 * b, v[r], m < nt && ((dm >> k) & 1));
  }
}

// As dup_rows_store for the down outputs: pair q gets bf16(y[r] x w[q]) with its own routing weight.
__device__ __noinline__ void dup_rows_store_w(uint16_t* yw, uint64_t users, uint64_t all, int nt, int b, float y0,
                                              float y1, float y2, float y3, const uint16_t* wts) {
  const int lane = threadIdx.x & 63;
  const float y[4] = {y0, y1, y2, y3};
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    const int p = pair_at(users, min(m, nt - 1));
    const uint32_t dm = token_dups(all, p) & ~(1u << (p & 3));
    for (int k = 0; k < 4; ++k) {
      const int q = (p & ~3) + k;
      store_row_pairs(yw + (long long)q * kH + 16 * b, f32_to_bf16(y[r] * bf16_to_f32(wts[q])),
                      m < nt && ((dm >> k) & 1));
    }
  }
}

// LDS of one expert-major decode workgroup: staged x (or h) rows, scale rows, the KS partial D tiles [KS][2][64].
// With 4 or more staged rows the partial tiles reuse the rows' space (after a barrier that ends every wave's reads
// of them), which keeps three workgroups per CU at 8 rows instead of two.
template <int KS, int XT>
struct DecodeLds {
  static constexpr bool kAliasRed = XT >= 4;
  static constexpr int kRedBytes = (KS > 1 ? KS : 1) * 2 * 64 * 16;
  static_assert(!kAliasRed || kRedBytes <= XT * kXPitch, "partial tiles must fit in the staged rows");
  __align__(16) uint8_t xs[XT * kXPitch];
  __align__(16) uint8_t sc[2 * kScLds];
  __align__(16) uint8_t red_own[kAliasRed ? 16 : kRedBytes];
  NA_DEVICE f32x4_t* red() { return reinterpret_cast<f32x4_t*>(kAliasRed ? xs : red_own); }
};

// gate_up: output block b (rows j = 16b .. 16b + 15 of gate and of up) of the item-th distinct expert -> h[pair, j].
// Order: route and slot -> every global load (codes, scales, x, bias) -> x and scales to LDS, barrier -> MFMA tile by
// tile (each waits only for its own codes) -> fixed-order sum of the KS partial tiles through LDS -> epilogue in wave
// 0, which reads nothing from global memory.
template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_gate_up_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ bias_gu, uint16_t* __restrict__ h, float alpha, float limit) {
  constexpr int MT = (kTTiles + KS - 1) / KS;
  constexpr int NTH = 64 * KS;
  __shared__ DecodeLds<KS, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(x, bias_gu, h, alpha, limit);          // past the preloaded arguments: fetched while the ids fly
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, 4 * B, blockIdx.x, nt, users, all, distinct, valid);
  if (e < 0 || e == 128) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.y;
  const long long gid = expert_base + e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* gblk = pool + slot * slot_bytes + (long long)b * kTBlock;
  const uint8_t* ublk = gblk + (long long)kTUpBlock0 * kTBlock;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  ScaleRegs<2, NTH> sr;
  scale_load<2, NTH>(tid, gblk, ublk, sr);
  XRegs<XT, NTH> xr;
  x_load<XT, NTH>(tid, x, kH, [users](int t) { return pair_at(users, t) >> 2; }, nt, xr);
  const int j = 16 * b + (lane & 15);
  const uint16_t* bg = bias_gu ? bias_gu + gid * kGU : nullptr;
  // epilogue operands are loaded now and converted at their use, so no wait is placed before the barrier
  // (unconditional loads: without a bias they read x, in bounds, and the value is not used)
  const uint16_t* bgs = bg ? bg : x;
  const uint16_t* bus = bg ? bg + kI : x;
  const uint16_t bgj = bgs[j], buj = bus[j];
  CodeRegs<MT> rg, ru;
  code_load<MT>(gblk, lane, t0, t1, rg);
  code_load<MT>(ublk, lane, t0, t1, ru);
  // every load is issued above; the first wait (for x and the scales, issued first) comes below
  __builtin_amdgcn_sched_barrier(0);
  x_store<XT, NTH>(tid, L.xs, nt, xr);
  scale_store<2, NTH>(tid, L.sc, sr);
  __syncthreads();
  const uint8_t* xrow = L.xs + min(lane & 15, XT - 1) * kXPitch;
  const uint8_t* srow = L.sc + (lane & 15) * kScPitch;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rg, srow, xrow, lane, t0, t1, ag);
  block_compute<MT>(ru, srow + kScLds, xrow, lane, t0, t1, au);
  if constexpr (XT == 1) {
    // one token: only D row 0 (element 0 of lanes 0..15) is used; the same sums in the same order as below
    if constexpr (KS > 1) {
      float* red = reinterpret_cast<float*>(L.red());           // [KS][2][16]
      if (lane < 16) {
        red[(2 * wave) * 16 + lane] = ag[0];
        red[(2 * wave + 1) * 16 + lane] = au[0];
      }
      __syncthreads();
      if (wave != 0) return;
      const int l = lane & 15;
      float g = red[l], u = red[16 + l];
#pragma unroll
      for (int w = 1; w < KS; ++w) {
        g += red[(2 * w) * 16 + l];
        u += red[(2 * w + 1) * 16 + l];
      }
      ag[0] = g;
      au[0] = u;
    }
    float gb = rb(ag[0]), ub = rb(au[0]);
    if (bg) {
      gb = rb(gb + bf16_to_f32(bgj));
      ub = rb(ub + bf16_to_f32(buj));
    }
    const uint16_t hv0 = f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit));
    store_row_pairs(h + (long long)pair_at(users, 0) * kI + 16 * b, hv0, lane < 16);
    if (all != users) dup_rows_store(h, kI, users, all, nt, b, hv0, hv0, hv0, hv0);   // uniform, rare
    return;
  }
  if constexpr (KS > 1) {
    f32x4_t* red = L.red();
    if constexpr (DecodeLds<KS, XT>::kAliasRed) __syncthreads();   // every wave is done with the staged rows
    red[(2 * wave) * 64 + lane] = ag;
    red[(2 * wave + 1) * 64 + lane] = au;
    __syncthreads();
    if (wave != 0) return;
    ag = red[lane];
    au = red[64 + lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      ag += red[(2 * w) * 64 + lane];
      au += red[(2 * w + 1) * 64 + lane];
    }
  }
  uint16_t hv[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    float gb = rb(ag[r]), ub = rb(au[r]);
    if (bg) {
      gb = rb(gb + bf16_to_f32(bgj));
      ub = rb(ub + bf16_to_f32(buj));
    }
    hv[r] = f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit));
    store_row_pairs(h + (long long)pair_at(users, min(m, nt - 1)) * kI + 16 * b, hv[r], m < nt);
  }
  if (all != users) dup_rows_store(h, kI, users, all, nt, b, hv[0], hv[1], hv[2], hv[3]);   // uniform, rare
}

// down, expert-major: output block b (rows n = 16b .. 16b + 15) of the item-th distinct expert from each routed
// token's own h row, + bias, x routing weight -> yw[pair, n].  An invalid id (128) writes +0 for its pairs and reads
// no weights.  The top-k sum is left to k_combine_t950.  Load order as in the gate_up kernel.
template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_down_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ h,
    const uint16_t* __restrict__ wts, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  constexpr int MT = (kTTiles + KS - 1) / KS;
  constexpr int NTH = 64 * KS;
  __shared__ DecodeLds<KS, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(h, wts, bias_dn, yw);                  // past the preloaded arguments: fetched while the ids fly
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, 4 * B, blockIdx.x, nt, users, all, distinct, valid);
  if (e < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int b = blockIdx.y;
  if (e == 128) {                                      // invalid ids: each of their pairs contributes +0
    for (int i = tid; i < 4 * B * (kTRows / 2); i += NTH) {
      const int q = i / (kTRows / 2), c = i - q * (kTRows / 2);
      if ((all >> q) & 1) *reinterpret_cast<uint32_t*>(yw + (long long)q * kH + 16 * b + 2 * c) = 0u;
    }
    return;
  }
  const long long gid = expert_base + e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* blk = pool + slot * slot_bytes + kTDownOff + (long long)b * kTBlock;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  ScaleRegs<1, NTH> sr;
  scale_load<1, NTH>(tid, blk, blk, sr);
  XRegs<XT, NTH> xr;
  x_load<XT, NTH>(tid, h, kI, [users](int t) { return pair_at(users, t); }, nt, xr);
  const int n = 16 * b + (lane & 15);
  // epilogue operands are loaded now and converted at their use, so no wait is placed before the barrier
  const uint16_t bdn = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  uint16_t wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) wr[r] = wts[pair_at(users, min(4 * (lane >> 4) + r, nt - 1))];
  CodeRegs<MT> rd;
  code_load<MT>(blk, lane, t0, t1, rd);
  __builtin_amdgcn_sched_barrier(0);
  x_store<XT, NTH>(tid, L.xs, nt, xr);
  scale_store<1, NTH>(tid, L.sc, sr);
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rd, L.sc + (lane & 15) * kScPitch, L.xs + min(lane & 15, XT - 1) * kXPitch, lane, t0, t1, acc);
  if constexpr (KS > 1) {
    f32x4_t* red = L.red();
    if constexpr (DecodeLds<KS, XT>::kAliasRed) __syncthreads();   // every wave is done with the staged rows
    red[(2 * wave) * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    acc = red[lane];
#pragma unroll
    for (int w = 1; w < KS; ++w) acc += red[(2 * w) * 64 + lane];
  }
  float yb[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * (lane >> 4) + r;
    float y = rb(acc[r]);
    if (bias_dn) y = rb(y + bf16_to_f32(bdn));
    yb[r] = y;
    store_row_pairs(yw + (long long)pair_at(users, min(m, nt - 1)) * kH + 16 * b,
                    f32_to_bf16(y * bf16_to_f32(wr[r])), m < nt);
  }
  if (all != users) dup_rows_store_w(yw, users, all, nt, b, yb[0], yb[1], yb[2], yb[3], wts);   // uniform, rare
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

// down + combine, row-block-major, for B <= 2 (at most G = 16 / KSD distinct experts): one workgroup of 16 waves per
// output block b holds every distinct expert of the batch (G groups of KSD waves; group g serves the g-th distinct
// expert), so the top-k sum needs no third kernel and no cross-workgroup exchange.  All 4B h rows are staged in
// LDS once; each group runs the expert-major down arithmetic on its pairs' rows; the group leaders leave each pair's
// bf16 yw row slice in LDS; after a barrier, out[t, 16b + n] = bf16(sum_k yw[4t + k, n]) in top-k order.
constexpr int kDcWaves = 16;

template <int KSD, int XT>
struct DownCombLds {
  static constexpr int G = kDcWaves / KSD;
  __align__(16) uint8_t hs[4 * XT * kXPitch];           // h rows of all pairs, row p = pair p
  __align__(16) uint8_t sc[G * kScLds];
  f32x4_t red[kDcWaves][64];
  float yw[4 * XT][kTRows];
};

template <int KSD, int XT>
__global__ __launch_bounds__(64 * kDcWaves) void k_moe_down_comb_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ h,
    const uint16_t* __restrict__ wts, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ out) {
  constexpr int MT = (kTTiles + KSD - 1) / KSD;
  constexpr int NTH = 64 * kDcWaves;
  constexpr int GTH = 64 * KSD;
  __shared__ DownCombLds<KSD, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(h, wts, bias_dn, out);                 // past the preloaded arguments: fetched while the ids fly
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = wave / KSD, kw = wave - g * KSD, gtid = tid - g * GTH;
  const int b = blockIdx.x;
  const int npairs = 4 * B;
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, npairs, g, nt, users, all, distinct, valid);
  const bool live = e >= 0 && e != 128;
  const long long gid = expert_base + (live ? e : 0);
  // groups without a live expert load slot 0's block (valid memory) with every tile slot zeroed, so that the loads
  // stay unconditional and are all issued before the first wait
  const long long slot = live ? (slot_tab ? slot_tab[gid] : gid) : 0;
  const uint8_t* blk = pool + slot * slot_bytes + kTDownOff + (long long)b * kTBlock;
  int t0, t1;
  ktile_range<KSD>(kw, t0, t1);
  ScaleRegs<1, GTH> sr;
  scale_load<1, GTH>(gtid, blk, blk, sr);
  XRegs<4 * XT, NTH> xr;                                 // all pairs' h rows: staged row p = pair p
  x_load<4 * XT, NTH>(tid, h, kI, [](int t) { return t; }, npairs, xr);
  const int n = 16 * b + (lane & 15);
  const uint16_t bdn = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  uint16_t wr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) wr[r] = wts[live ? pair_at(users, min(4 * (lane >> 4) + r, nt - 1)) : 0];
  CodeRegs<MT> rd;
  code_load<MT>(blk, lane, t0, live ? t1 : t0, rd);
  __builtin_amdgcn_sched_barrier(0);
  x_store<4 * XT, NTH>(tid, L.hs, npairs, xr);
  scale_store<1, GTH>(gtid, L.sc + g * kScLds, sr);
  if (e == 128 && kw == 0) {                             // invalid ids: each of their pairs contributes +0
    for (int i = lane; i < npairs * kTRows; i += 64)
      if ((all >> (i / kTRows)) & 1) L.yw[i / kTRows][i % kTRows] = 0.f;
  }
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int pm = live ? pair_at(users, min(lane & 15, nt - 1)) : 0;   // A row of token slot m = lane % 16
  if (live)
    block_compute<MT>(rd, L.sc + g * kScLds + (lane & 15) * kScPitch, L.hs + pm * kXPitch, lane, t0, t1, acc);
  if constexpr (XT == 1) {
    // one token: nt <= 1, only D row 0 (element 0 of lanes 0..15) is used; the same sums in the same order
    float* red = reinterpret_cast<float*>(&L.red[0][0]);   // [kDcWaves][16]
    if (lane < 16) red[wave * 16 + lane] = acc[0];
    __syncthreads();
    if (live && kw == 0 && lane < 16) {
#pragma unroll
      for (int w = 1; w < KSD; ++w) acc[0] += red[(wave + w) * 16 + lane];
      float y = rb(acc[0]);
      if (bias_dn) y = rb(y + bf16_to_f32(bdn));
      const int p = pair_at(users, 0);
      if (all == users) {                                // uniform: no token lists this expert twice
        L.yw[p][lane] = rb(y * bf16_to_f32(wr[0]));
      } else {
        const uint32_t dm = token_dups(all, p);
        for (int k = 0; k < 4; ++k)
          if ((dm >> k) & 1) L.yw[(p & ~3) + k][lane] = rb(y * bf16_to_f32(wts[(p & ~3) + k]));
      }
    }
  } else {
    L.red[wave][lane] = acc;
    __syncthreads();
    if (live && kw == 0) {
#pragma unroll
      for (int w = 1; w < KSD; ++w) acc += L.red[wave + w][lane];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 4 * (lane >> 4) + r;
        if (m < nt) {
          float y = rb(acc[r]);
          if (bias_dn) y = rb(y + bf16_to_f32(bdn));
          const int p = pair_at(users, m);
          if (all == users) {                              // uniform: no token lists this expert twice
            L.yw[p][lane & 15] = rb(y * bf16_to_f32(wr[r]));
          } else {
            const uint32_t dm = token_dups(all, p);
            for (int k = 0; k < 4; ++k)
              if ((dm >> k) & 1) L.yw[(p & ~3) + k][lane & 15] = rb(y * bf16_to_f32(wts[(p & ~3) + k]));
          }
        }
      }
    }
  }
  __syncthreads();
  if (tid < B * kTRows) {
    const int t = tid / kTRows, c = tid - t * kTRows;
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a += L.yw[4 * t + k][c];
    out[(long long)t * kH + 16 * b + c] = f32_to_bf16(a);
  }
}

// ------------------------------------------------------------------------- one launch per layer (one token)
// gate_up and down + combine of one token's top-4 experts in a single launch: 180 workgroups, one per 16-row output
// block b, of 16 waves = 4 subgroups of 4 waves; subgroup s serves pair s (the token's s-th routed expert) and its
// waves split K as in the expert-major kernels.  Phase 1: gate_up rows j = 16b .. 16b + 15 (gate block b, up block
// b + 180) -> h[s][j] with device-coherent stores.  The workgroup then arrives at a grid-wide barrier, and before
// waiting it issues the loads of its down block's codes and scales, so that the down weights stream while the last
// workgroups finish phase 1.  Phase 2: down rows n = 16b .. 16b + 15 of each pair from its h row (device-coherent
// loads), + bias, x routing weight, and the top-4 sum in pair order -> out[n].  The arithmetic is the two-launch
// path's (k_moe_gate_up_t950 + k_moe_down_comb_t950) step for step, so the results are identical.
// The barrier needs all 180 workgroups resident at once (the host checks the occupancy before launching).  Its wait
// is bounded: past spin_limit polls a workgroup sets sync[2] and goes on (the outputs are then undefined; the kernel
// still ends).  The last workgroup to leave resets sync[0] and sync[1], so a completed launch leaves them zero.
constexpr int kLwWaves = 16, kLwKS = 4;
constexpr int kLwHWords = 4 * kI / 2;                  // h of the 4 pairs as bf16 pairs

union LayerLds {
  struct {
    __align__(16) uint8_t xs[kXPitch];
    __align__(16) uint8_t sc[4][2 * kScLds];
    f32x4_t red[kLwWaves][2][64];
  } p1;
  struct {
    __align__(16) uint8_t hs[4 * kXPitch];
    __align__(16) uint8_t sc[4][kScLds];
    f32x4_t red[kLwWaves][64];
    float yw[4][kTRows];
  } p2;
};

__global__ __launch_bounds__(64 * kLwWaves) void k_moe_layer_t950(
    const uint16_t* __restrict__ x, const int64_t* __restrict__ ids, const uint16_t* __restrict__ wts,
    const uint8_t* __restrict__ pool, long long slot_bytes, const int64_t* __restrict__ slot_tab,
    long long expert_base, const uint16_t* __restrict__ bias_gu, const uint16_t* __restrict__ bias_dn,
    uint32_t* __restrict__ hbuf, uint32_t* __restrict__ sync, int spin_limit, uint16_t* __restrict__ out,
    float alpha, float limit) {
  constexpr int MT = (kTTiles + kLwKS - 1) / kLwKS;
  constexpr int NTH = 64 * kLwWaves, STH = 64 * kLwKS;
  constexpr int HP = (kLwHWords + NTH - 1) / NTH;
  __shared__ LayerLds L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int s = wave / kLwKS, kw = wave - s * kLwKS, stid = tid - s * STH;
  const int b = blockIdx.x;
  const long long v = ids[s];
  const bool live = v >= 0 && v < 128;
  const long long gid = expert_base + (live ? v : 0);
  // a dead pair (invalid id) loads slot 0's blocks (valid memory) with every tile slot zeroed and computes nothing
  const long long slot = live ? (slot_tab ? slot_tab[gid] : gid) : 0;
  const uint8_t* sbase = pool + slot * slot_bytes;
  const uint8_t* gblk = sbase + (long long)b * kTBlock;
  const uint8_t* ublk = gblk + (long long)kTUpBlock0 * kTBlock;
  const uint8_t* dblk = sbase + kTDownOff + (long long)b * kTBlock;
  int t0, t1;
  ktile_range<kLwKS>(kw, t0, t1);
  const int t1l = live ? t1 : t0;

  // ---- phase 1: gate_up + bias + clamped SwiGLU of pair s, rows 16b .. 16b + 15
  ScaleRegs<2, STH> sr;
  scale_load<2, STH>(stid, gblk, ublk, sr);
  XRegs<1, NTH> xr;
  x_load<1, NTH>(tid, x, kH, [](int) { return 0; }, 1, xr);
  const int j = 16 * b + (lane & 15);
  const uint16_t* bgs = bias_gu ? bias_gu + gid * kGU : x;         // unconditional loads (x when there is no bias)
  const uint16_t bgj = bgs[bias_gu ? j : 0], buj = bgs[bias_gu ? kI + j : 0];
  CodeRegs<MT> rg, ru;
  code_load<MT>(gblk, lane, t0, t1l, rg);
  code_load<MT>(ublk, lane, t0, t1l, ru);
  __builtin_amdgcn_sched_barrier(0);
  x_store<1, NTH>(tid, L.p1.xs, 1, xr);
  scale_store<2, STH>(stid, L.p1.sc[s], sr);
  __syncthreads();
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  if (live) {
    const uint8_t* srow = L.p1.sc[s] + (lane & 15) * kScPitch;
    block_compute<MT>(rg, srow, L.p1.xs, lane, t0, t1, ag);
    block_compute<MT>(ru, srow + kScLds, L.p1.xs, lane, t0, t1, au);
  }
  L.p1.red[wave][0][lane] = ag;
  L.p1.red[wave][1][lane] = au;
  __syncthreads();
  if (kw == 0) {                                         // wave-uniform: the subgroup's first wave
    ag = L.p1.red[wave][0][lane];
    au = L.p1.red[wave][1][lane];
#pragma unroll
    for (int w = 1; w < kLwKS; ++w) {
      ag += L.p1.red[wave + w][0][lane];
      au += L.p1.red[wave + w][1][lane];
    }
    float gb = rb(ag[0]), ub = rb(au[0]);                // lanes 0..15: D row 0 (the token), column lane
    if (bias_gu) {
      gb = rb(gb + bf16_to_f32(bgj));
      ub = rb(ub + bf16_to_f32(buj));
    }
    const uint16_t hv = live ? f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit)) : (uint16_t)0;
    const uint32_t hi = (uint32_t)__shfl_xor((int)hv, 1) & 0xffff;
    if (lane < 16 && !(lane & 1))
      __hip_atomic_store(hbuf + s * (kI / 2) + (16 * b + lane) / 2, (uint32_t)hv | (hi << 16), __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
  }
  __builtin_amdgcn_s_waitcnt(0);                         // this wave's h stores are complete
  __syncthreads();                                       // (and phase 1's LDS is free for phase 2)
  if (tid == 0) __hip_atomic_fetch_add(sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // ---- the down block's weights, issued before the wait
  ScaleRegs<1, STH> sd;
  scale_load<1, STH>(stid, dblk, dblk, sd);
  const int n = 16 * b + (lane & 15);
  const uint16_t bdn = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  const uint16_t wv = wts[s];
  CodeRegs<MT> rd;
  code_load<MT>(dblk, lane, t0, t1l, rd);
  __builtin_amdgcn_sched_barrier(0);
  if (tid == 0) {
    int it = 0;
    while (__hip_atomic_load(sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gridDim.x) {
      __builtin_amdgcn_s_sleep(1);
      if (++it > spin_limit) {
        __hip_atomic_store(sync + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
    }
  }
  __syncthreads();

  // ---- phase 2: every pair's h row (device-coherent loads, all issued before the LDS stores), down, combine
  uint32_t hw[HP];
#pragma unroll
  for (int k = 0; k < HP; ++k)
    hw[k] = __hip_atomic_load(hbuf + min(tid + NTH * k, kLwHWords - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
  for (int k = 0; k < HP; ++k) {
    const int i = tid + NTH * k;
    if (i < kLwHWords) {
      const int p = i / (kI / 2), c = i - p * (kI / 2);
      *reinterpret_cast<uint32_t*>(L.p2.hs + p * kXPitch + 4 * c) = hw[k];
    }
  }
  scale_store<1, STH>(stid, L.p2.sc[s], sd);
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  if (live) block_compute<MT>(rd, L.p2.sc[s] + (lane & 15) * kScPitch, L.p2.hs + s * kXPitch, lane, t0, t1, acc);
  L.p2.red[wave][lane] = acc;
  __syncthreads();
  if (kw == 0 && lane < 16) {
#pragma unroll
    for (int w = 1; w < kLwKS; ++w) acc += L.p2.red[wave + w][lane];
    float y = rb(acc[0]);
    if (bias_dn) y = rb(y + bf16_to_f32(bdn));
    L.p2.yw[s][lane] = live ? rb(y * bf16_to_f32(wv)) : 0.f;
  }
  __syncthreads();
  if (tid < kTRows) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a += L.p2.yw[k][tid];
    out[16 * b + tid] = f32_to_bf16(a);
  }
  if (tid == 0) {
    const uint32_t done = __hip_atomic_fetch_add(sync + 1, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (done == gridDim.x - 1) {
      __hip_atomic_store(sync, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(sync + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

template <typename... KArgs, typename... Args>
static void launch_t(void (*kern)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                     Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, e0, e1, 0, static_cast<KArgs>(args)...);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, stream, static_cast<KArgs>(args)...);
}

typedef void (*GateUpT)(const int64_t*, int, const uint8_t*, long long, const int64_t*, long long, const uint16_t*,
                        const uint16_t*, uint16_t*, float, float);
typedef void (*DownT)(const int64_t*, int, const uint8_t*, long long, const int64_t*, long long, const uint16_t*,
                      const uint16_t*, const uint16_t*, uint16_t*);

template <int KS>
static GateUpT gate_up_t950_xt(int xt) {
  return xt == 1 ? k_moe_gate_up_t950<KS, 1> : xt == 2 ? k_moe_gate_up_t950<KS, 2>
       : xt == 4 ? k_moe_gate_up_t950<KS, 4> : k_moe_gate_up_t950<KS, 8>;
}
static GateUpT pick_gate_up_t950(int ks, int xt) {
  return ks == 1 ? gate_up_t950_xt<1>(xt) : ks == 2 ? gate_up_t950_xt<2>(xt)
       : ks == 4 ? gate_up_t950_xt<4>(xt) : gate_up_t950_xt<8>(xt);
}
template <int KS>
static DownT down_t950_xt(int xt) {
  return xt == 1 ? k_moe_down_t950<KS, 1> : xt == 2 ? k_moe_down_t950<KS, 2>
       : xt == 4 ? k_moe_down_t950<KS, 4> : k_moe_down_t950<KS, 8>;
}
static DownT pick_down_t950(int ks, int xt) {
  return ks == 1 ? down_t950_xt<1>(xt) : ks == 2 ? down_t950_xt<2>(xt)
       : ks == 4 ? down_t950_xt<4>(xt) : down_t950_xt<8>(xt);
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
                       int k_split, int down_mode, void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !h_scratch || !yw_scratch || B <= 0) return kErrArgs;
  if (down_mode != 0 && down_mode != 1) return kErrArgs;
  if (B > 8) return kErrTooLarge;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if (k_split <= 0) k_split = B == 1 ? 8 : 4;       // automatic: the fastest measured on MI355X per batch size
  if (k_split != 1 && k_split != 2 && k_split != 4 && k_split != 8) return kErrArgs;
  // down_mode 0, B = 1, with an output: gate_up, then down + combine (two launches); else gate_up, down, combine
  // (at B = 2 the row-block kernel's 16-wave workgroups with two waves per expert measured slower than three launches)
  const bool two = down_mode == 0 && out != nullptr && B == 1;
  hipEvent_t ev[6] = {};
  if (events)
    for (int i = 0; i < (two ? 4 : 6); ++i) ev[i] = (hipEvent_t)events[i];
  const int items = 4 * B;
  const dim3 g1(items, kTDownBlocks);
  const dim3 blk(64 * k_split);
  const int xt = B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;
  launch_t(pick_gate_up_t950(k_split, xt), g1, blk, stream, ev[0], ev[1], topk_ids, B, (const uint8_t*)pool,
           slot_bytes, slot_tab, expert_base, (const uint16_t*)x, (const uint16_t*)bias_gu, (uint16_t*)h_scratch,
           alpha, limit);
  if (two) {
    launch_t(k_moe_down_comb_t950<4, 1>, dim3(kTDownBlocks), dim3(64 * kDcWaves), stream, ev[2], ev[3], topk_ids, B,
             (const uint8_t*)pool, slot_bytes, slot_tab, expert_base, (const uint16_t*)h_scratch,
             (const uint16_t*)topk_w, (const uint16_t*)bias_dn, (uint16_t*)out);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
  }
  launch_t(pick_down_t950(k_split, xt), g1, blk, stream, ev[2], ev[3], topk_ids, B, (const uint8_t*)pool, slot_bytes,
           slot_tab, expert_base, (const uint16_t*)h_scratch, (const uint16_t*)topk_w, (const uint16_t*)bias_dn,
           (uint16_t*)yw_scratch);
  if (out)
    launch_t(k_combine_t950, dim3((B * kH / 2 + 255) / 256), dim3(256), stream, ev[4], ev[5],
             (const uint32_t*)yw_scratch, B, (uint32_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Single-launch decode layer for one token (k_moe_layer_t950).  Needs every one of its 180 workgroups resident at
// once: the occupancy is checked once per device; a device that cannot hold them gets kErrTooLarge.
int na_moe_layer_t950(const void* x, const int64_t* topk_ids, const void* topk_w, const void* pool,
                      long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                      const void* bias_dn, void* h_scratch, unsigned int* sync, void* out, float alpha, float limit,
                      void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !h_scratch || !sync || !out) return kErrArgs;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if (reinterpret_cast<uintptr_t>(h_scratch) & 15) return kErrArgs;
  static int fits[64];                                   // per device: 0 unknown, 1 fits, -1 does not
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kErrArgs;
  if (fits[dev] == 0) {
    int per_cu = 0, cus = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_layer_t950, 64 * kLwWaves, 0) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return kErrLaunch;
    fits[dev] = (long long)per_cu * cus >= kTDownBlocks ? 1 : -1;
  }
  if (fits[dev] < 0) return kErrTooLarge;
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  launch_t(k_moe_layer_t950, dim3(kTDownBlocks), dim3(64 * kLwWaves), stream, e0, e1, (const uint16_t*)x,
           topk_ids, (const uint16_t*)topk_w, (const uint8_t*)pool, slot_bytes, slot_tab, expert_base,
           (const uint16_t*)bias_gu, (const uint16_t*)bias_dn, (uint32_t*)h_scratch, (uint32_t*)sync, 1 << 22,
           (uint16_t*)out, alpha, limit);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
