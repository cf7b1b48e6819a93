// gfx950 tile layout ("t950") of GPT-OSS-120B expert slots, its lossless repack from/to the store layouts, and the
// MFMA decode kernels that stream it.
//
// Layout of one slot (13,271,040 B): 540 row blocks of 16 rows (gate_up rows 0..5759 = blocks 0..359, down rows
// 0..2879 = blocks 360..539), each 24,576 B:
//   codes  [0, 23040):  90 groups of 256 B, group-major: byte 256 g + 16 n + b = code byte b of (row n, group g).
//          k-tile t (groups 4t..4t+3; the last, t = 22, only groups 88 and 89) is the 1024 B at 1024 t, and lane
//          l = 16 kb + n owns its bytes [16 l, 16 l + 16) = E2M1 elements 32 (4t + kb) .. + 31 of row n.
//   scales [23040, 24576): 16 rows x 96 B, byte n * 96 + g = E8M0 of (row n, group g), bytes 90..95 of a row = 0.
// One 128-bit load per lane of a k-tile is exactly the FP4 B operand of one v_mfma_scale_f32_16x16x128_f8f6f4 (lane
// l supplies B[k = 32 (l / 16) + 0..31][n = l % 16]) for the 16 rows of the block.  The codes are the store's
// E2M1 nibbles unchanged and the scales the store's E8M0 bytes unchanged (PS4 rows are expanded), so the repack is a
// byte permutation plus padding and round-trips exactly (na_repack_from_t950).
#include "common.h"
#include "handoff.h"
#include "t950.h"
#include "topk.h"

#include <hip/hip_ext.h>

#include <cmath>
#include <mutex>

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

// One thread per 16 bytes of destination.  Per row block: 1440 code pieces (piece 16 g + n = the 16 code bytes of row
// n, group g) and 96 scale pieces (16 rows x 6).
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
  if (pc < kTCodes / 16) {                              // codes of (row n, group g)
    const int g = pc >> 4, n = pc & 15;
    const uint8_t* row = store_code_row(slot, mat, row0 + n) + 16 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) out[j] = *reinterpret_cast<const uint32_t*>(row + 4 * j);
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
  if (pc < kTCodes / 16) {                              // codes of (row n, group g)
    const int g = pc >> 4, n = pc & 15;
    const uint4 v = *reinterpret_cast<const uint4*>(b + 16 * pc);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint8_t* row = slot + (mat == 0 ? 0 : kOffDownCodes) + (long long)(row0 + n) * kRowBytes + 16 * g;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(row + 4 * j) = w[j];
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
// Work item = (distinct expert of the batch, 16-row output block); the KS waves of a workgroup split the 23 k-tiles.
// Each k-tile (16 rows x 128 K) is one v_mfma_scale_f32_16x16x128_f8f6f4: B = the block's E2M1 codes with their E8M0
// scales, consumed as stored (no dequantisation instruction); A = the activations of the expert's tokens as E4M3 with
// one E8M0 scale per 32-element block, two A rows per token (hi and lo, see x8_quant_chunk), so that one MFMA serves up
// to 8 tokens.  The KS partial tiles are summed in a fixed order through LDS.  Code tiles are read with non-temporal
// 128-bit loads (each weight byte is used once per step), one load per lane and k-tile being the MFMA's B operand as
// it stands; a row block's 1,536 scale bytes are read by the workgroup with coalesced 16-byte loads and staged in
// LDS, so that each wave reads its scales from LDS instead of issuing one scattered 64-lane load per tile.
constexpr int kMaxTokT = 8;                  // tokens per expert the MFMA M dimension holds (two A rows each)
constexpr int kScPitch = 112;                // LDS bytes per staged weight scale row: 28 dwords, 16 rows hit 16 banks
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
// nothing).  In the half tile (t = 22) lanes 32..63 (groups 90, 91, past K) read the first 512 bytes of the block's
// scale rows, which block_compute replaces by zeros.  The zeroing happens at the use, so that no wait for the codes
// is placed before the first barrier.
NA_DEVICE int slot_tile(int t0, int t1, int i) { return t0 + i < t1 ? t0 + i : t0; }

template <int MT>
NA_DEVICE void code_load(const uint8_t* blk, int lane, int t0, int t1, CodeRegs<MT>& r) {
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = slot_tile(t0, t1, i);
    r.c[i] = load16<true>(blk + t * 1024 + 16 * lane);
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

template <int NR>
struct X8Lds {
  __align__(16) uint8_t row[NR][kX8Pitch];   // row 2u = hi, 2u + 1 = lo of the u-th staged token
  __align__(16) uint8_t zero[128];           // the A operand of MFMA rows past the staged ones
  __align__(16) uint8_t sc[NR][kX8ScPitch];
};

// Activation rows (x, or h) of up to XT tokens, staged through registers: piece p = tid + NTH * k (k < XP) of
// 360 * XT 16-byte pieces (one chunk of 8 elements each).
template <int XT, int NTH>
struct XRegs {
  static constexpr int XP = (XT * kChunks + NTH - 1) / NTH;
  uint4 v[XP];
};

// Thread tid loads pieces p = tid + NTH k < nt x 360 (a per-lane predicate, no branch), i.e. rows t < nt
// (1 <= nt <= XT) of the staged block, row t = source row row_of(t); the other pieces are zero.
template <int XT, int NTH, typename RowOf>
NA_DEVICE void x_load(int tid, const uint16_t* base, long long row_stride, RowOf row_of, int nt, XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = tid + NTH * k;
    const int t = p / kChunks, pp = p - t * kChunks;
    xr.v[k] = make_uint4(0, 0, 0, 0);
    if (p < nt * kChunks)
      xr.v[k] = load16(reinterpret_cast<const uint8_t*>(base + (long long)row_of(t) * row_stride) + 16 * pp);
  }
}

// ---- h between the gate_up and down parts: the bf16 values of the reference's h, one 2880-element row per pair.  The
// down part quantises each row into E4M3 hi + lo rows with one E8M0 scale per 32-element block while it stages it
// (x8_store, as gate_up does with x), which holds every element within 2^13 of its block's largest magnitude exactly.
constexpr int kHRow = 2 * kI;               // bytes per pair
constexpr int kHPieces = kHRow / 16;        // 360 16-byte pieces per pair (= kChunks)

// ---- the single-launch expert body's handoffs as tagged words (handoff.h): h of pair p, row block b in the 8 words
// (p x 180 + b) x 8 + k (bf16 values 16b + 2k, 16b + 2k + 1), the weighted output yw of pair p, block b in the 8
// words (p x 180 + b) x 8 + k (outputs 16b + 2k, 16b + 2k + 1).  raw: the workgroup's launch count as thread 0 read it (other threads: 0), from which one_tag forms
// the launch's number (the kernel's comment below); err: the error word a wait that gives up raises.
constexpr int kOneWgs = 4 * kTDownBlocks;       // 720 workgroups
struct OneTags {
  uint64_t* h;
  uint64_t* y;
  uint32_t raw;
  uint32_t* err;
};
// What the single-launch body loads at entry, before its routing ids arrive (batch 1): the token's x (pieces of
// k_moe_gate_up_t950<4, 1>'s x_load) and the expert's pool slot, picked from the layer's 128 slot-table entries
// (-1: no slot table, slot = the global id).
struct OnePre {
  XRegs<1, 256> x;
  long long slot;
};

// The launch's number, in every lane of wave 0 (call it where lane 0 is active).  The empty asm keeps the division,
// and so the wait for the entry count, at the point of use.
NA_DEVICE uint32_t one_tag(const OneTags& tg) {
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)launch_tag(tg.raw));
}
NA_DEVICE uint64_t* one_h_words(const OneTags& tg, int pair, int b) { return tg.h + ((long long)pair * kTDownBlocks + b) * 8; }
NA_DEVICE uint64_t* one_y_words(const OneTags& tg, int pair, int b) { return tg.y + ((long long)pair * kTDownBlocks + b) * 8; }

// The pairs' h rows of up to XT staged tokens through registers: piece p = tid + NTH k < nt x 360; piece q = p % 360
// of token t = p / 360 is values 8q .. 8q + 7 of its row.
// 16 bytes at base + off with one device-coherent (sc1) load: what the same launch wrote on another XCD.  base is
// uniform across the wave (a buffer resource is scalar), off per lane and 16-byte aligned.
NA_DEVICE uint4 load16_sc1(const void* base, uint32_t off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
  const u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 16);
  return make_uint4(v.x, v.y, v.z, v.w);
}

template <int XT, int NTH, typename PairOf>
NA_DEVICE void h8_load(int tid, const uint8_t* h8, PairOf pair_of, int nt, XRegs<XT, NTH>& xr) {
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    const int p = tid + NTH * k;
    const int t = p / kHPieces, q = p - t * kHPieces;
    if (p < nt * kHPieces) xr.v[k] = load16(h8 + (long long)pair_of(t) * kHRow + 16 * q);
  }
}

// Quantise the loaded pieces into the E4M3 rows 2t (hi) / 2t + 1 (lo) of staged token t < nt and their scales, and
// clear the zero strip.  NTH is a multiple of 64 and 360 of 4, so the 4 chunks of a block are 4 lanes of one wave that
// are all inside or all outside p < nt x 360; rounds with no piece below nt x 360 are skipped (a uniform branch).
template <int XT, int NTH>
NA_DEVICE void x8_store(int tid, X8Lds<2 * XT>& L, int nt, const XRegs<XT, NTH>& xr) {
  static_assert(NTH % 64 == 0, "whole waves");
#pragma unroll
  for (int k = 0; k < XRegs<XT, NTH>::XP; ++k) {
    if (NTH * k >= nt * kChunks) break;
    const int p = tid + NTH * k;
    const int t = p / kChunks, c = p - t * kChunks;
    uint2 hi, lo;
    uint32_t sh, sl;
    x8_quant_chunk(xr.v[k], hi, lo, sh, sl);
    if (p < nt * kChunks) {
      *reinterpret_cast<uint2*>(L.row[2 * t] + 8 * c) = hi;
      *reinterpret_cast<uint2*>(L.row[2 * t + 1] + 8 * c) = lo;
      if ((c & 3) == 0) {
        L.sc[2 * t][c >> 2] = (uint8_t)sh;
        L.sc[2 * t + 1][c >> 2] = (uint8_t)sl;
      }
    }
  }
  if (tid < 8) reinterpret_cast<uint4*>(L.zero)[tid] = make_uint4(0, 0, 0, 0);
}

// One row block over this wave's k-tiles: D[m][n] += sum_k A[m][k] B[k][n], B = the codes (row n = lane % 16), A row
// m = lane % 16: `arow` is this lane's staged E4M3 row with scales `asc`, or null past the staged rows (zero strip).
// A's operand order: lane 16 kb + m holds K = 16 kb .. 16 kb + 15 and 64 + 16 kb .. 64 + 16 kb + 15 of the tile.
// wsc = the staged scale row of output row n.  The half tile (t = 22) holds groups 88 and 89 in its first 64 K.
template <int MT>
NA_DEVICE void block_compute(const CodeRegs<MT>& r, const uint8_t* wsc, const uint8_t* arow, const uint8_t* asc,
                             const uint8_t* zero, int lane, int t0, int t1, f32x4_t& acc) {
  const int kb = lane >> 4;
#pragma unroll
  for (int i = 0; i < MT; ++i) {
    const int t = slot_tile(t0, t1, i);
    const int g = 4 * t + kb;                              // B: this lane's group; A: this lane's first K block
    const bool ok = t0 + i < t1 && g < kGK;
    const uint32_t w0 = ok ? r.c[i].x : 0u, w1 = ok ? r.c[i].y : 0u, w2 = ok ? r.c[i].z : 0u, w3 = ok ? r.c[i].w : 0u;
    const int sb = wsc[g];                                 // groups 90, 91: the row's zero padding (codes are 0)
    const int sa = arow ? asc[min(g, kGK - 1)] : 127;
    const uint8_t* ap = arow ? arow + 128 * t : zero;
    const uint4 a0 = *reinterpret_cast<const uint4*>(ap + 16 * kb);
    const uint4 a1 = t < kTFull ? *reinterpret_cast<const uint4*>(ap + 64 + 16 * kb) : make_uint4(0, 0, 0, 0);
    const mfma_i32x8_t A = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
    const mfma_i32x8_t Bv = {(int)w0, (int)w1, (int)w2, (int)w3, 0, 0, 0, 0};
    acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bv, acc, 0, 4, 0, sa, 0, sb);
  }
}

// D rows 2u, 2u + 1 = hi and lo of token u: lane 16 i + n holds D[4i .. 4i + 3][n], i.e. tokens 2i (elements 0, 1)
// and 2i + 1 (elements 2, 3).  The two sums of this lane.
NA_DEVICE void token_sums(const f32x4_t& acc, float& y0, float& y1) {
  y0 = acc[0] + acc[1];
  y1 = acc[2] + acc[3];
}

// Store the bf16 values v held as D columns n = lane % 16 (16 lanes per D row) as 32-bit pairs: even lanes write
// (v[n], v[n + 1]) to row_ptr + n.  All lanes must call it (it exchanges values between neighbouring lanes).
NA_DEVICE void store_row_pairs(uint16_t* row_ptr, uint16_t v, bool ok) {
  const int lane = threadIdx.x & 63;
  const uint32_t hi = (uint32_t)__shfl_xor((int)v, 1) & 0xffff;
  if (ok && !(lane & 1)) *reinterpret_cast<uint32_t*>(row_ptr + (lane & 15)) = (uint32_t)v | (hi << 16);
}
// h of D column n = lane % 16 (row 16b + n) of `pair` as bf16 pairs (store_row_pairs: every lane calls it).
NA_DEVICE void store_h(uint8_t* h, int pair, int b, uint16_t hv, bool ok) {
  store_row_pairs(reinterpret_cast<uint16_t*>(h + (long long)pair * kHRow) + 16 * b, hv, ok);
}

// ... as tagged words: even lanes write (v[n], v[n + 1]) as word n / 2 of w.
NA_DEVICE void tag_row_pairs(uint64_t* w, uint16_t v, bool ok, uint32_t tag) {
  const int lane = threadIdx.x & 63;
  const uint32_t hi = (uint32_t)__shfl_xor((int)v, 1) & 0xffff;
  if (ok && !(lane & 1)) tag_store(w + ((lane & 15) >> 1), (uint32_t)v | (hi << 16), tag);
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
// to the expert, <= B); pair_at(users, u) is the u-th user in ascending order.  The staged tokens are the users; each
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

// The u-th pair (ascending) of a route's mask, 0 <= u < kMaxTokT; the mask is uniform, the walk is scalar.
NA_DEVICE int pair_at(uint64_t users, int u) {
  int p = __ffsll((long long)users) - 1;
  uint64_t m = users;
#pragma unroll
  for (int t = 1; t < kMaxTokT; ++t) {
    m &= m - 1;
    const int pt = __ffsll((long long)m) - 1;
    p = (t == u) ? pt : p;
  }
  return p;
}

// The duplicate pairs' h: for token u = 2 (lane / 16) + e < nt (user pair p), the same value v[e] also goes to every
// other pair of p's token that `all` routes to the expert (columns 16b .. 16b + 15).  Kept out of line of the common
// path, which stores only the users' rows.
__device__ __noinline__ void dup_rows_store_h(uint8_t* h, uint64_t users, uint64_t all, int nt, int b, uint16_t v0,
                                              uint16_t v1) {
  const int lane = threadIdx.x & 63;
  const uint16_t v[2] = {v0, v1};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int u = 2 * (lane >> 4) + e;
    const int p = pair_at(users, min(u, nt - 1));
    const uint32_t dm = token_dups(all, p) & ~(1u << (p & 3));
    for (int k = 0; k < 4; ++k) store_h(h, (p & ~3) + k, b, v[e], u < nt && ((dm >> k) & 1));
  }
}

// As dup_rows_store for the down outputs: pair q gets bf16(y[e] x w[q]) with its own routing weight (TAG: as tagged
// words of tg, in place of yw).
template <bool TAG>
__device__ __noinline__ void dup_rows_store_w(uint16_t* yw, uint64_t users, uint64_t all, int nt, int b, float y0,
                                              float y1, const uint16_t* wts, OneTags tg, uint32_t tag) {
  const int lane = threadIdx.x & 63;
  const float y[2] = {y0, y1};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int u = 2 * (lane >> 4) + e;
    const int p = pair_at(users, min(u, nt - 1));
    const uint32_t dm = token_dups(all, p) & ~(1u << (p & 3));
    for (int k = 0; k < 4; ++k) {
      const int q = (p & ~3) + k;
      const uint16_t v = f32_to_bf16(y[e] * bf16_to_f32(wts[q]));
      if constexpr (TAG) tag_row_pairs(one_y_words(tg, q, b), v, u < nt && ((dm >> k) & 1), tag);
      else store_row_pairs(yw + (long long)q * kH + 16 * b, v, u < nt && ((dm >> k) & 1));
    }
  }
}

// This lane's A row: staged row m = lane % 16 while m < 2 nt, else none (the zero strip).
template <int NR>
NA_DEVICE const uint8_t* a_row(const X8Lds<NR>& L, int lane, int nt) {
  const int m = lane & 15;
  return m < 2 * nt ? L.row[min(m, NR - 1)] : nullptr;
}
template <int NR>
NA_DEVICE const uint8_t* a_scales(const X8Lds<NR>& L, int lane) {
  return L.sc[min(lane & 15, NR - 1)];
}

// LDS of one expert-major decode workgroup: the staged E4M3 rows, the weight scale rows, and the KS partial sums
// [KS][2 matrices][64 lanes][2 tokens].  With 4 or more staged tokens the partial sums reuse the rows' space (after a
// barrier that ends every wave's reads of them), which keeps three workgroups per CU at 8 tokens.
template <int KS, int XT>
struct DecodeLds {
  static constexpr bool kAliasRed = XT >= 4;
  static constexpr int kRedBytes = (KS > 1 ? KS : 1) * 2 * 64 * 2 * 4;
  static_assert(!kAliasRed || kRedBytes <= (int)sizeof(X8Lds<2 * XT>::row), "partial sums must fit in the rows");
  X8Lds<2 * XT> x;
  __align__(16) uint8_t sc[2 * kScLds];
  __align__(16) uint8_t red_own[kAliasRed ? 16 : kRedBytes];
  NA_DEVICE float* red() { return reinterpret_cast<float*>(kAliasRed ? &x.row[0][0] : red_own); }
};

// gate_up: output block b (rows j = 16b .. 16b + 15 of gate and of up) of the item-th distinct expert -> h[pair, j]
// (bf16).
// Order: route and slot -> every global load (codes, scales, x, bias) -> x quantised to E4M3 and the scales to LDS,
// barrier -> one MFMA per tile (each waits only for its own codes) -> fixed-order sum of the KS partial sums through
// LDS -> epilogue in wave 0, which reads nothing from global memory.
// The body of workgroup (item, b); every wave returns from it (waves past the first right after the K reduction).
// TAG (the single-launch expert body, batch 1): h is written as tagged words of tg (the users' rows only: down reads
// an expert's first user's row), not to h8.
template <int KS, int XT, bool TAG>
NA_DEVICE void gate_up_body(DecodeLds<KS, XT>& L, int item, int b, long long rid, int B,
                            const uint8_t* __restrict__ pool, long long slot_bytes,
                            const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ x,
                            const uint16_t* __restrict__ bias_gu, uint8_t* __restrict__ h8, float alpha, float limit,
                            const OneTags& tg = OneTags{}, const OnePre* pre = nullptr) {
  static_assert(!TAG || XT == 1, "tagged h: one token");
  constexpr int MT = (kTTiles + KS - 1) / KS;
  constexpr int NTH = 64 * KS;
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, 4 * B, item, nt, users, all, distinct, valid);
  if (e < 0 || e == 128) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long long gid = expert_base + e;
  const long long slot = TAG ? (pre->slot >= 0 ? pre->slot : gid) : slot_tab ? slot_tab[gid] : gid;
  const uint8_t* gblk = pool + slot * slot_bytes + (long long)b * kTBlock;
  const uint8_t* ublk = gblk + (long long)kTUpBlock0 * kTBlock;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  ScaleRegs<2, NTH> sr;
  scale_load<2, NTH>(tid, gblk, ublk, sr);
  XRegs<XT, NTH> xr;
  if constexpr (TAG) xr = pre->x;                      // batch 1: token 0's row, loaded at the kernel's entry
  else x_load<XT, NTH>(tid, x, kH, [users](int t) { return pair_at(users, t) >> 2; }, nt, xr);
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
  x8_store<XT, NTH>(tid, L.x, nt, xr);
  scale_store<2, NTH>(tid, L.sc, sr);
  __syncthreads();
  const uint8_t* arow = a_row(L.x, lane, nt);
  const uint8_t* asc = a_scales(L.x, lane);
  const uint8_t* srow = L.sc + (lane & 15) * kScPitch;
  f32x4_t ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rg, srow, arow, asc, L.x.zero, lane, t0, t1, ag);
  block_compute<MT>(ru, srow + kScLds, arow, asc, L.x.zero, lane, t0, t1, au);
  float g2[2], u2[2];
  token_sums(ag, g2[0], g2[1]);
  token_sums(au, u2[0], u2[1]);
  if constexpr (KS > 1) {
    float* red = L.red();                                  // [KS][2][64][2]
    if constexpr (DecodeLds<KS, XT>::kAliasRed) __syncthreads();   // every wave is done with the staged rows
    if (XT > 1 || lane < 16) {
      *reinterpret_cast<float2*>(red + ((2 * wave) * 64 + lane) * 2) = make_float2(g2[0], g2[1]);
      *reinterpret_cast<float2*>(red + ((2 * wave + 1) * 64 + lane) * 2) = make_float2(u2[0], u2[1]);
    }
    __syncthreads();
    if (wave != 0) return;
    if (XT > 1 || lane < 16) {
      float2 gs = *reinterpret_cast<const float2*>(red + lane * 2);
      float2 us = *reinterpret_cast<const float2*>(red + (64 + lane) * 2);
#pragma unroll
      for (int w = 1; w < KS; ++w) {
        const float2 gw = *reinterpret_cast<const float2*>(red + ((2 * w) * 64 + lane) * 2);
        const float2 uw = *reinterpret_cast<const float2*>(red + ((2 * w + 1) * 64 + lane) * 2);
        gs.x += gw.x;
        gs.y += gw.y;
        us.x += uw.x;
        us.y += uw.y;
      }
      g2[0] = gs.x;
      g2[1] = gs.y;
      u2[0] = us.x;
      u2[1] = us.y;
    }
  }
  uint16_t hv[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = 2 * (lane >> 4) + q;
    float gb = rb(g2[q]), ub = rb(u2[q]);
    if (bg) {
      gb = rb(gb + bf16_to_f32(bgj));
      ub = rb(ub + bf16_to_f32(buj));
    }
    hv[q] = f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit));
    if constexpr (!TAG) store_h(h8, pair_at(users, min(u, nt - 1)), b, hv[q], u < nt);
  }
  if constexpr (TAG) {
    // lanes 0..15 hold the token's 16 values: even lanes write them as 8 words of bf16 pairs
    tag_row_pairs(one_h_words(tg, pair_at(users, 0), b), hv[0], lane < 16, one_tag(tg));
  } else if (all != users) {
    dup_rows_store_h(h8, users, all, nt, b, hv[0], hv[1]);   // rare
  }
}

template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_gate_up_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ bias_gu, uint8_t* __restrict__ h8, float alpha, float limit) {
  __shared__ DecodeLds<KS, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(x, bias_gu, h8, alpha, limit);       // past the preloaded arguments: fetched while ids fly
  gate_up_body<KS, XT, false>(L, blockIdx.x, blockIdx.y, rid, B, pool, slot_bytes, slot_tab, expert_base, x, bias_gu,
                              h8, alpha, limit);
}

// down, expert-major: output block b (rows n = 16b .. 16b + 15) of the item-th distinct expert from each routed
// token's own h row (bf16 from the gate_up kernel, quantised to E4M3 hi + lo rows while staged), + bias, x routing
// weight -> yw[pair, n].  An invalid id (128)
// writes +0 for its pairs and reads no weights.  The top-k sum is left to k_combine_t950.  Load order as in the
// gate_up kernel.  Every wave returns from the body (waves past the first right after the K reduction).
// TAG (the single-launch expert body, batch 1): h was written earlier in the same launch as tagged words of tg, so
// the weight rows are loaded first, then thread 0 polls the last word of the expert's h row (from its last gate_up
// workgroup), then every thread reads its 8 words of the row (ordinary loads first: all 180 down workgroups of the
// expert read that row, and an XCD's L2 serves all but the first), polling again any word not yet tagged; yw is
// written as tagged words of tg (by wave 0), not to yw.
template <int KS, int XT, bool TAG>
NA_DEVICE void down_body(DecodeLds<KS, XT>& L, int item, int b, long long rid, int B, const uint8_t* __restrict__ pool,
                         long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
                         const uint8_t* __restrict__ h8, const uint16_t* __restrict__ wts,
                         const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw,
                         const OneTags& tg = OneTags{}, const OnePre* pre = nullptr) {
  static_assert(!TAG || XT == 1, "tagged h: one token");
  constexpr int MT = (kTTiles + KS - 1) / KS;
  constexpr int NTH = 64 * KS;
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, 4 * B, item, nt, users, all, distinct, valid);
  if (e < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (e == 128) {                                      // invalid ids: each of their pairs contributes +0
    if constexpr (TAG) {
      if (wave != 0) return;
      const uint32_t tag = one_tag(tg);
      if (lane < 4 * (kTRows / 2) && ((all >> (lane >> 3)) & 1))
        tag_store(one_y_words(tg, lane >> 3, b) + (lane & 7), 0u, tag);
      return;
    }
    for (int i = tid; i < 4 * B * (kTRows / 2); i += NTH) {
      const int q = i / (kTRows / 2), c = i - q * (kTRows / 2);
      if ((all >> q) & 1) *reinterpret_cast<uint32_t*>(yw + (long long)q * kH + 16 * b + 2 * c) = 0u;
    }
    return;
  }
  const long long gid = expert_base + e;
  const long long slot = TAG ? (pre->slot >= 0 ? pre->slot : gid) : slot_tab ? slot_tab[gid] : gid;
  const uint8_t* blk = pool + slot * slot_bytes + kTDownOff + (long long)b * kTBlock;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  ScaleRegs<1, NTH> sr;
  scale_load<1, NTH>(tid, blk, blk, sr);
  XRegs<XT, NTH> xr;
  const auto pair_of = [users](int t) { return pair_at(users, t); };
  if constexpr (!TAG) h8_load<XT, NTH>(tid, h8, pair_of, nt, xr);
  const int n = 16 * b + (lane & 15);
  // epilogue operands are loaded now and converted at their use, so no wait is placed before the barrier
  const uint16_t bdn = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  uint16_t wr[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) wr[q] = wts[pair_at(users, min(2 * (lane >> 4) + q, nt - 1))];
  CodeRegs<MT> rd;
  code_load<MT>(blk, lane, t0, t1, rd);
  if constexpr (TAG) {
    static_assert(XRegs<XT, NTH>::XP == 2, "two 16-byte pieces of the h row per thread");
    __shared__ uint32_t tag_lds;                       // thread 0's number, for every thread after the barrier
    const uint64_t* hrow = one_h_words(tg, pair_at(users, 0), 0);
    if (tid == 0) {
      const uint32_t t0 = one_tag(tg);
      tag_wait1(hrow + (kTDownBlocks - 1) * 8 + 7, t0, tg.err);
      tag_lds = t0;
    }
    __syncthreads();
    const uint32_t tag = tag_lds;
    // piece q (values 8q .. 8q + 7 of the row) = words 4 (q % 2) .. 4 (q % 2) + 3 of block q / 2
    const uint64_t* src[8];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int q = min(tid + NTH * k, kHPieces - 1);
      const uint64_t* w = hrow + (q >> 1) * 8 + 4 * (q & 1);
#pragma unroll
      for (int i = 0; i < 4; ++i) src[4 * k + i] = w + i;
    }
    uint32_t hw[8];
    tag_read_at<8, true>(src, tag, hw, tg.err);
    xr.v[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
    xr.v[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
  }
  __builtin_amdgcn_sched_barrier(0);
  x8_store<XT, NTH>(tid, L.x, nt, xr);
  scale_store<1, NTH>(tid, L.sc, sr);
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(rd, L.sc + (lane & 15) * kScPitch, a_row(L.x, lane, nt), a_scales(L.x, lane), L.x.zero, lane, t0,
                    t1, acc);
  float y2[2];
  token_sums(acc, y2[0], y2[1]);
  if constexpr (KS > 1) {
    float* red = L.red();                                  // [KS][64][2]
    if constexpr (DecodeLds<KS, XT>::kAliasRed) __syncthreads();   // every wave is done with the staged rows
    if (XT > 1 || lane < 16) *reinterpret_cast<float2*>(red + (wave * 64 + lane) * 2) = make_float2(y2[0], y2[1]);
    __syncthreads();
    if (wave != 0) return;
    if (XT > 1 || lane < 16) {
      float2 s = *reinterpret_cast<const float2*>(red + lane * 2);
#pragma unroll
      for (int w = 1; w < KS; ++w) {
        const float2 v = *reinterpret_cast<const float2*>(red + (w * 64 + lane) * 2);
        s.x += v.x;
        s.y += v.y;
      }
      y2[0] = s.x;
      y2[1] = s.y;
    }
  }
  float yb[2];
  const uint32_t ytag = TAG ? one_tag(tg) : 0u;
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int u = 2 * (lane >> 4) + q;
    float y = rb(y2[q]);
    if (bias_dn) y = rb(y + bf16_to_f32(bdn));
    yb[q] = y;
    const uint16_t v = f32_to_bf16(y * bf16_to_f32(wr[q]));
    const int pr = pair_at(users, min(u, nt - 1));
    if constexpr (TAG) tag_row_pairs(one_y_words(tg, pr, b), v, u < nt, ytag);
    else store_row_pairs(yw + (long long)pr * kH + 16 * b, v, u < nt);
  }
  if (all != users) dup_rows_store_w<TAG>(yw, users, all, nt, b, yb[0], yb[1], wts, tg, ytag);   // uniform, rare
}

// down for batches of several tokens, two row blocks per workgroup (b and b + 90, grid items x 90): the staging of
// the tokens' h rows, the routing, the barrier, the K reduction and the epilogue are shared by twice the weight bytes
// (like gate_up's gate and up blocks), so half as many workgroups carry the same stream, each with twice its bytes in
// flight.  Each block's arithmetic is down_body's (the same MFMA sums, reduction order and epilogue): the outputs
// are bit-identical.
template <int KS, int XT>
NA_DEVICE void down_body2(DecodeLds<KS, XT>& L, int item, int bb, long long rid, int B, const uint8_t* __restrict__ pool,
                          long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
                          const uint8_t* __restrict__ h8, const uint16_t* __restrict__ wts,
                          const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  static_assert(KS > 1 && XT > 1, "several tokens, K split over the waves");
  constexpr int MT = (kTTiles + KS - 1) / KS;
  constexpr int NTH = 64 * KS;
  constexpr int kHalf = kTDownBlocks / 2;
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4 * XT>(rid, 4 * B, item, nt, users, all, distinct, valid);
  if (e < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int bl[2] = {bb, bb + kHalf};
  if (e == 128) {                                      // invalid ids: each of their pairs contributes +0
    for (int i = tid; i < 2 * 4 * B * (kTRows / 2); i += NTH) {
      const int k = i / (4 * B * (kTRows / 2)), r = i - k * (4 * B * (kTRows / 2));
      const int q = r / (kTRows / 2), c = r - q * (kTRows / 2);
      if ((all >> q) & 1) *reinterpret_cast<uint32_t*>(yw + (long long)q * kH + 16 * bl[k] + 2 * c) = 0u;
    }
    return;
  }
  const long long gid = expert_base + e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* blk0 = pool + slot * slot_bytes + kTDownOff + (long long)bl[0] * kTBlock;
  const uint8_t* blk1 = blk0 + (long long)kHalf * kTBlock;
  int t0, t1;
  ktile_range<KS>(wave, t0, t1);
  ScaleRegs<2, NTH> sr;
  scale_load<2, NTH>(tid, blk0, blk1, sr);
  XRegs<XT, NTH> xr;
  h8_load<XT, NTH>(tid, h8, [users](int t) { return pair_at(users, t); }, nt, xr);
  // epilogue operands are loaded now and converted at their use, so no wait is placed before the barrier
  uint16_t bdn[2];
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int n = 16 * bl[k] + (lane & 15);
    bdn[k] = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  }
  uint16_t wr[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) wr[q] = wts[pair_at(users, min(2 * (lane >> 4) + q, nt - 1))];
  CodeRegs<MT> r0, r1;
  code_load<MT>(blk0, lane, t0, t1, r0);
  code_load<MT>(blk1, lane, t0, t1, r1);
  __builtin_amdgcn_sched_barrier(0);
  x8_store<XT, NTH>(tid, L.x, nt, xr);
  scale_store<2, NTH>(tid, L.sc, sr);
  __syncthreads();
  const uint8_t* arow = a_row(L.x, lane, nt);
  const uint8_t* asc = a_scales(L.x, lane);
  const uint8_t* srow = L.sc + (lane & 15) * kScPitch;
  f32x4_t a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
  block_compute<MT>(r0, srow, arow, asc, L.x.zero, lane, t0, t1, a0);
  block_compute<MT>(r1, srow + kScLds, arow, asc, L.x.zero, lane, t0, t1, a1);
  float y[2][2];
  token_sums(a0, y[0][0], y[0][1]);
  token_sums(a1, y[1][0], y[1][1]);
  float* red = L.red();                                // [KS][2 blocks][64][2]
  if constexpr (DecodeLds<KS, XT>::kAliasRed) __syncthreads();   // every wave is done with the staged rows
#pragma unroll
  for (int k = 0; k < 2; ++k)
    *reinterpret_cast<float2*>(red + ((2 * wave + k) * 64 + lane) * 2) = make_float2(y[k][0], y[k][1]);
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float2 sm = *reinterpret_cast<const float2*>(red + (k * 64 + lane) * 2);
#pragma unroll
    for (int w = 1; w < KS; ++w) {
      const float2 v = *reinterpret_cast<const float2*>(red + ((2 * w + k) * 64 + lane) * 2);
      sm.x += v.x;
      sm.y += v.y;
    }
    y[k][0] = sm.x;
    y[k][1] = sm.y;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    float yb[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int u = 2 * (lane >> 4) + q;
      float v = rb(y[k][q]);
      if (bias_dn) v = rb(v + bf16_to_f32(bdn[k]));
      yb[q] = v;
      const uint16_t o = f32_to_bf16(v * bf16_to_f32(wr[q]));
      store_row_pairs(yw + (long long)pair_at(users, min(u, nt - 1)) * kH + 16 * bl[k], o, u < nt);
    }
    if (all != users) dup_rows_store_w<false>(yw, users, all, nt, bl[k], yb[0], yb[1], wts, OneTags{}, 0u);   // rare
  }
}

template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_down2_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint8_t* __restrict__ h8,
    const uint16_t* __restrict__ wts, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  __shared__ DecodeLds<KS, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(h8, wts, bias_dn, yw);                // past the preloaded arguments: fetched while the ids fly
  down_body2<KS, XT>(L, blockIdx.x, blockIdx.y, rid, B, pool, slot_bytes, slot_tab, expert_base, h8, wts, bias_dn,
                     yw);
}

template <int KS, int XT>
__global__ __launch_bounds__(64 * KS) void k_moe_down_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint8_t* __restrict__ h8,
    const uint16_t* __restrict__ wts, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  __shared__ DecodeLds<KS, XT> L;
  const long long rid = route_ids_load(ids, 4 * B);
  args_at_entry(h8, wts, bias_dn, yw);                // past the preloaded arguments: fetched while the ids fly
  down_body<KS, XT, false>(L, blockIdx.x, blockIdx.y, rid, B, pool, slot_bytes, slot_tab, expert_base, h8, wts,
                           bias_dn, yw);
}

__global__ __launch_bounds__(256) void k_combine_t950(const uint32_t* __restrict__ yw, int B,
                                                      uint32_t* __restrict__ out) {
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

// down + combine, row-block-major, for one token: one workgroup of 16 waves per output block b holds the token's
// (up to 4) distinct experts (4 groups of KSD = 4 waves; group g serves the g-th distinct expert), so the top-k sum
// needs no third kernel and no cross-workgroup exchange.  The 4 pairs' h rows are staged in LDS once (as E4M3 hi + lo);
// each group runs the expert-major down arithmetic on its pair's rows; the group leaders leave each pair's
// bf16(y x w) slice in LDS; after a barrier, out[16b + n] = bf16(sum_k yw[k][n]) in top-k order.
constexpr int kDcWaves = 16, kDcKS = 4;

struct DownCombLds {
  X8Lds<8> x;                                          // pair p's h row: E4M3 rows 2p (hi), 2p + 1 (lo)
  __align__(16) uint8_t sc[kDcWaves / kDcKS][kScLds];
  float red[kDcWaves][16];
  float yw[4][kTRows];
};

__global__ __launch_bounds__(64 * kDcWaves) void k_moe_down_comb_t950(
    const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint8_t* __restrict__ h8,
    const uint16_t* __restrict__ wts, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ out) {
  constexpr int MT = (kTTiles + kDcKS - 1) / kDcKS;
  constexpr int NTH = 64 * kDcWaves;
  constexpr int GTH = 64 * kDcKS;
  __shared__ DownCombLds L;
  const long long rid = route_ids_load(ids, 4);
  args_at_entry(h8, wts, bias_dn, out);               // past the preloaded arguments: fetched while the ids fly
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = wave / kDcKS, kw = wave - g * kDcKS, gtid = tid - g * GTH;
  const int b = blockIdx.x;
  int nt, distinct, valid;
  uint64_t users, all;
  const int e = route_t950<4>(rid, 4, g, nt, users, all, distinct, valid);
  const bool live = e >= 0 && e != 128;
  const long long gid = expert_base + (live ? e : 0);
  // groups without a live expert load slot 0's block (valid memory) with every tile slot zeroed, so that the loads
  // stay unconditional and are all issued before the first wait
  const long long slot = live ? (slot_tab ? slot_tab[gid] : gid) : 0;
  const uint8_t* blk = pool + slot * slot_bytes + kTDownOff + (long long)b * kTBlock;
  int t0, t1;
  ktile_range<kDcKS>(kw, t0, t1);
  ScaleRegs<1, GTH> sr;
  scale_load<1, GTH>(gtid, blk, blk, sr);
  XRegs<4, NTH> xr;                                    // all 4 pairs' h rows: staged token t = pair t
  h8_load<4, NTH>(tid, h8, [](int t) { return t; }, 4, xr);
  const int n = 16 * b + (lane & 15);
  const uint16_t bdn = (bias_dn ? bias_dn + gid * kH : wts)[bias_dn ? n : 0];   // unconditional load
  const uint16_t wr = wts[live ? pair_at(users, 0) : 0];
  CodeRegs<MT> rd;
  code_load<MT>(blk, lane, t0, live ? t1 : t0, rd);
  __builtin_amdgcn_sched_barrier(0);
  x8_store<4, NTH>(tid, L.x, 4, xr);
  scale_store<1, GTH>(gtid, L.sc[g], sr);
  if (e == 128 && kw == 0) {                           // invalid ids: each of their pairs contributes +0
    for (int i = lane; i < 4 * kTRows; i += 64)
      if ((all >> (i / kTRows)) & 1) L.yw[i / kTRows][i % kTRows] = 0.f;
  }
  __syncthreads();
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  const int p = live ? pair_at(users, 0) : 0;          // the pair of this group's expert (one token)
  const int m = lane & 15;
  const uint8_t* arow = m < 2 ? L.x.row[2 * p + m] : nullptr;
  if (live) block_compute<MT>(rd, L.sc[g] + m * kScPitch, arow, L.x.sc[2 * p + (m & 1)], L.x.zero, lane, t0, t1, acc);
  if (lane < 16) L.red[wave][lane] = acc[0] + acc[1];
  __syncthreads();
  if (live && kw == 0 && lane < 16) {
    float s = L.red[wave][lane];
#pragma unroll
    for (int w = 1; w < kDcKS; ++w) s += L.red[wave + w][lane];
    float y = rb(s);
    if (bias_dn) y = rb(y + bf16_to_f32(bdn));
    if (all == users) {                                // uniform: the token lists this expert once
      L.yw[p][lane] = rb(y * bf16_to_f32(wr));
    } else {
      const uint32_t dm = token_dups(all, p);
      for (int k = 0; k < 4; ++k)
        if ((dm >> k) & 1) L.yw[(p & ~3) + k][lane] = rb(y * bf16_to_f32(wts[(p & ~3) + k]));
    }
  }
  __syncthreads();
  if (tid < kTRows) {
    float a = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) a += L.yw[k][tid];
    out[16 * b + tid] = f32_to_bf16(a);
  }
}

// ---- the expert body of one token in a single launch (na_moe_decode_t950_one): 720 workgroups.  Workgroup blk =
// 180 i + b runs k_moe_gate_up_t950<4, 1>'s (i-th distinct expert, gate_up row block b), writing its 16 h values as
// tagged words (handoff.h), then k_moe_down_t950<4, 1>'s (i-th expert, down row block b): its weight rows are loaded
// before it polls the expert's h row, and its weighted outputs are written as tagged words; workgroup 540 + b (the
// fourth expert's) then reads the four pairs' outputs of block b and sums them in k_combine_t950's order.  The order
// is expert-major: workgroups are dispatched, and their weight loads served, roughly in id order, so the first
// experts' h rows are complete (and their down parts run) while the later experts' gate_up rows still stream, where
// an interleaved order released every expert's h only near the end of the stream (0.9 us slower per launch).  Bit-identical to the two- and
// three-launch paths.  The launch's number: workgroup blk owns counter word blk, reads it at entry (n after n
// launches), tags with n + 1 and stores n + 1 back before it ends: the same number in every workgroup of a launch,
// one more than the previous launch's, with no atomic, no shared word and nothing to reset.
// A down workgroup waits for the gate_up parts of its expert's 180 workgroups, so all 720 must be resident at once:
// the host launches this kernel only where the occupancy query allows it (3 workgroups per CU x 256 CUs = 768 on
// MI355X).  The waits are bounded (handoff.h): a broken assumption shows as the error word, never as a hang.
// sync: kOneSyncLines lines of kLine uint32, zero before the first launch: line 0 the error word (raised by a wait
// that gave up, never cleared here), the workgroups' counter words (720 uint32), then the tagged words of h
// (4 x 180 x 8) and of the weighted outputs (4 x 180 x 8).
constexpr int kOneErr = 0, kOneCtr = 1, kOneTagH = kOneCtr + (kOneWgs + kLine - 1) / kLine;
constexpr int kOneTagWords = 4 * kTDownBlocks * 8;                     // 5760 per area
constexpr int kOneTagY = kOneTagH + kOneTagWords * 2 / kLine;
constexpr int kOneSyncLines = kOneTagY + kOneTagWords * 2 / kLine;     // 373 lines, 95,488 bytes

// LOGITS (na_moe_decode_t950_one_logits): the routing comes from the layer's 128 router logits instead of ids and
// weights: every wave selects the top 4 itself (topk.h, the router's own selection and softmax), the weights go to
// LDS for the down part, and workgroup 0 writes the ids and weights out (ids_out / wts_out, when given).
template <bool LOGITS>
__global__ __launch_bounds__(256) void k_moe_one_t950(
    const int64_t* __restrict__ ids, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ x,
    const uint16_t* __restrict__ bias_gu, const uint16_t* __restrict__ bias_dn, const uint16_t* __restrict__ wts,
    uint16_t* __restrict__ out, float alpha, float limit, uint32_t* __restrict__ sync, const float* __restrict__ logits,
    int64_t* __restrict__ ids_out, uint16_t* __restrict__ wts_out) {
  __shared__ DecodeLds<4, 1> L;
  __shared__ uint16_t wts_lds[4];
  long long rid;
  float lv0 = 0.f, lv1 = 0.f;
  if constexpr (LOGITS) {
    lv0 = logits[threadIdx.x & 63];
    lv1 = logits[64 + (threadIdx.x & 63)];
  } else {
    rid = route_ids_load(ids, 4);
  }
  args_at_entry(x, bias_gu, bias_dn, wts, out, alpha, limit, sync, ids_out, wts_out);
  const int blk = blockIdx.x, item = blk / kTDownBlocks, b = blk - item * kTDownBlocks;   // expert-major
  const int tid = threadIdx.x, lane = tid & 63;
  // loads that do not depend on the routing, issued while the ids are in flight: token 0's x, the layer's slots
  OnePre pre;
  x_load<1, 256>(tid, x, kH, [](int) { return 0; }, 1, pre.x);
  int64_t srow[2] = {0, 0};
  if (slot_tab) {
    srow[0] = slot_tab[expert_base + lane];
    srow[1] = slot_tab[expert_base + 64 + lane];
  }
  // the launch count: loaded by thread 0 now, first needed at the end of the gate_up part (one_tag)
  uint32_t* ctr = sync + kOneCtr * kLine + blk;
  const uint32_t raw = tid == 0 ? load_coherent(ctr) : 0u;
  const OneTags tg{reinterpret_cast<uint64_t*>(sync + kOneTagH * kLine),
                   reinterpret_cast<uint64_t*>(sync + kOneTagY * kLine), raw, sync + kOneErr * kLine};
  if constexpr (LOGITS) {                              // the top 4 of the logits, in every wave
    float tv[4];
    int ti[4];
    top4_select(lv0, lv1, lane, tv, ti);
    rid = top4_id(ti, min(lane, 3));
    if (tid < 4) {
      const uint16_t wv = top4_weight(tv, tid);
      wts_lds[tid] = wv;                               // read by the down part, after gate_up's first barrier
      if (blk == 0 && ids_out) {
        ids_out[tid] = rid;
        wts_out[tid] = wv;
      }
    }
    wts = wts_lds;
  }
  {                                                    // this workgroup's expert -> its slot (a lane read, uniform)
    int nt, distinct, valid;
    uint64_t users, all;
    const int e = __builtin_amdgcn_readfirstlane(route_t950<4>(rid, 4, item, nt, users, all, distinct, valid));
    pre.slot = -1;
    if (slot_tab && e >= 0 && e < 128) {
      const int64_t v = srow[e >> 6];
      const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, e & 63);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)v >> 32), e & 63);
      pre.slot = (long long)(((uint64_t)hi << 32) | lo);
    }
  }
  gate_up_body<4, 1, true>(L, item, b, rid, 1, pool, slot_bytes, slot_tab, expert_base, x, bias_gu, nullptr, alpha,
                           limit, tg, &pre);
  down_body<4, 1, true>(L, item, b, rid, 1, pool, slot_bytes, slot_tab, expert_base, nullptr, wts, bias_dn, nullptr, tg,
                        &pre);
  if (tid >= 64) return;
  const uint32_t tag = one_tag(tg);
  if (tid == 0) store_coherent(ctr, tag);              // the count for the next launch
  if (item != 3) return;
  // block b's sum: thread t < 8 reads word t of the four pairs' outputs (k_combine_t950's arithmetic)
  if (tid >= kTRows / 2) return;
  const uint64_t* src[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) src[k] = one_y_words(tg, k, b) + tid;
  uint32_t w[4];
  tag_read_at<4>(src, tag, w, tg.err);
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a0 += bf16_to_f32((uint16_t)(w[k] & 0xffff));
    a1 += bf16_to_f32((uint16_t)(w[k] >> 16));
  }
  reinterpret_cast<uint32_t*>(out + 16 * b)[tid] = (uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16);
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
                        const uint16_t*, uint8_t*, float, float);
typedef void (*DownT)(const int64_t*, int, const uint8_t*, long long, const int64_t*, long long, const uint8_t*,
                      const uint16_t*, const uint16_t*, uint16_t*);

// The clamped SwiGLU's parameters: positive and finite (the decode kernels' argument check).
static bool act_args_ok(float alpha, float limit) {
  return alpha > 0.f && limit > 0.f && std::isfinite(alpha) && std::isfinite(limit);
}

template <int KS>
static GateUpT gate_up_t950_xt(int xt) {
  return xt == 1 ? k_moe_gate_up_t950<KS, 1> : xt == 2 ? k_moe_gate_up_t950<KS, 2>
       : xt == 4 ? k_moe_gate_up_t950<KS, 4> : k_moe_gate_up_t950<KS, 8>;
}
static GateUpT pick_gate_up_t950(int ks, int xt) {
  return ks == 4 ? gate_up_t950_xt<4>(xt) : gate_up_t950_xt<8>(xt);
}
template <int KS>
static DownT down_t950_xt(int xt) {
  return xt == 1 ? k_moe_down_t950<KS, 1> : xt == 2 ? k_moe_down_t950<KS, 2>
       : xt == 4 ? k_moe_down_t950<KS, 4> : k_moe_down_t950<KS, 8>;
}
static DownT pick_down_t950(int ks, int xt) {
  return ks == 4 ? down_t950_xt<4>(xt) : down_t950_xt<8>(xt);
}

// The t950 decode expert body of na_moe_decode_t950 with its scratch given: h (bf16 rows of the 4 B pairs,
// 5,760 B each) and yw (bf16 weighted expert outputs of the pairs, 5,760 B each).
static int decode_t950(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                       long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                       const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha, float limit,
                       int k_split, int down_mode, void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !h_scratch || !yw_scratch || B <= 0) return kErrArgs;
  if (down_mode != 0 && down_mode != 1) return kErrArgs;
  if (B > 8) return kErrTooLarge;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if (k_split <= 0) k_split = 4;                    // automatic: the fastest measured on MI355X at every batch size
  if (k_split != 4 && k_split != 8) return kErrArgs;
  // down_mode 0, B = 1, with an output: gate_up, then down + combine (two launches); else gate_up, down, combine
  // (at B = 2 the row-block kernel's 16-wave workgroups with two waves per expert measured slower than three launches)
  const bool two = down_mode == 0 && out != nullptr && B == 1;
  hipEvent_t ev[6] = {};
  if (events)
    for (int i = 0; i < (two ? 4 : 6); ++i) ev[i] = (hipEvent_t)events[i];
  if (!act_args_ok(alpha, limit)) return kErrArgs;
  const int items = 4 * B;
  const dim3 g1(items, kTDownBlocks);
  const dim3 blk(64 * k_split);
  const int xt = B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8;
  launch_t(pick_gate_up_t950(k_split, xt), g1, blk, stream, ev[0], ev[1], topk_ids, B, (const uint8_t*)pool,
           slot_bytes, slot_tab, expert_base, (const uint16_t*)x, (const uint16_t*)bias_gu, (uint8_t*)h_scratch,
           alpha, limit);
  if (two) {
    launch_t(k_moe_down_comb_t950, dim3(kTDownBlocks), dim3(64 * kDcWaves), stream, ev[2], ev[3], topk_ids, B,
             (const uint8_t*)pool, slot_bytes, slot_tab, expert_base, (const uint8_t*)h_scratch,
             (const uint16_t*)topk_w, (const uint16_t*)bias_dn, (uint16_t*)out);
    return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
  }
  if (xt == 8) {                                      // two row blocks per workgroup
    launch_t(k_split == 4 ? k_moe_down2_t950<4, 8> : k_moe_down2_t950<8, 8>, dim3(items, kTDownBlocks / 2), blk,
             stream, ev[2], ev[3], topk_ids, B, (const uint8_t*)pool, slot_bytes, slot_tab, expert_base,
             (const uint8_t*)h_scratch, (const uint16_t*)topk_w, (const uint16_t*)bias_dn, (uint16_t*)yw_scratch);
  } else {
    launch_t(pick_down_t950(k_split, xt), g1, blk, stream, ev[2], ev[3], topk_ids, B, (const uint8_t*)pool,
             slot_bytes, slot_tab, expert_base, (const uint8_t*)h_scratch, (const uint16_t*)topk_w,
             (const uint16_t*)bias_dn, (uint16_t*)yw_scratch);
  }
  if (out)
    launch_t(k_combine_t950, dim3((B * kH / 2 + 255) / 256), dim3(256), stream, ev[4], ev[5],
             (const uint32_t*)yw_scratch, B, (uint32_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

// Scratch of na_moe_decode_t950_noalloc: h then yw of up to 8 tokens (32 pairs x 5,760 B each), 368,640 B per
// device, held from the library's load until the process ends.  Every call on a device uses the same bytes: calls
// that overlap on one device race.  Both parts are written before they are read in every call, so nothing needs
// to start at zero.
constexpr int kNoAllocMaxB = 8;
constexpr long long kNoAllocPart = 4LL * kNoAllocMaxB * 2 * kH;
static __device__ __align__(256) uint8_t scratch[2 * kNoAllocPart];

// Device address of `scratch` on the current device, looked up once per device with hipGetSymbolAddress (the array's
// host-side name is only a stand-in); nullptr if the lookup fails.
static void* scratch_address() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
    addr[dev] = p;
  }
  return addr[dev];
}

// Whether the current device holds all kOneWgs workgroups of k_moe_one_t950 at once (the occupancy query times the
// CU count), asked once per device.
static bool one_resident_ok() {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static int8_t ok[kMaxDevices] = {};                 // 0 unknown, 1 yes, -1 no
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  std::lock_guard<std::mutex> lock(mu);
  if (!ok[dev]) {
    int per_cu = 0, per_cu_l = 0, cus = 0;               // both forms (ids, logits) of the kernel
    const bool q = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k_moe_one_t950<false>, 256, 0) == hipSuccess &&
                   hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu_l, k_moe_one_t950<true>, 256, 0) == hipSuccess &&
                   hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess;
    ok[dev] = q && (long long)min(per_cu, per_cu_l) * cus >= kOneWgs ? 1 : -1;
  }
  return ok[dev] > 0;
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
  return decode_t950(x, topk_ids, topk_w, B, pool, slot_bytes, slot_tab, expert_base, bias_gu, bias_dn, h_scratch,
                     yw_scratch, out, alpha, limit, k_split, down_mode, events, stream);
}

long long na_moe_one_sync_words(void) { return (long long)kOneSyncLines * kLine; }

int na_moe_decode_t950_one(const void* x, const int64_t* topk_ids, const void* topk_w, const void* pool,
                           long long slot_bytes, const int64_t* slot_tab, long long expert_base, const void* bias_gu,
                           const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha,
                           float limit, unsigned int* sync, void* const* events, hipStream_t stream) {
  (void)h_scratch;                                     // h and the weighted outputs travel as tagged words in sync
  (void)yw_scratch;
  if (!x || !topk_ids || !topk_w || !pool || !out || !sync) return kErrArgs;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(sync)) & 15) return kErrArgs;
  if (!act_args_ok(alpha, limit)) return kErrArgs;
  if (!one_resident_ok()) return kErrResident;
  launch_t(k_moe_one_t950<false>, dim3(kOneWgs), dim3(256), stream, events ? (hipEvent_t)events[0] : nullptr,
           events ? (hipEvent_t)events[1] : nullptr, topk_ids, (const uint8_t*)pool, slot_bytes, slot_tab,
           expert_base, (const uint16_t*)x, (const uint16_t*)bias_gu, (const uint16_t*)bias_dn,
           (const uint16_t*)topk_w, (uint16_t*)out, alpha, limit, (uint32_t*)sync, nullptr, nullptr, nullptr);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_moe_decode_t950_one_logits(const void* x, const float* logits, int64_t* ids_out, void* wts_out,
                                  const void* pool, long long slot_bytes, const int64_t* slot_tab,
                                  long long expert_base, const void* bias_gu, const void* bias_dn, void* out,
                                  float alpha, float limit, unsigned int* sync, void* const* events,
                                  hipStream_t stream) {
  if (!x || !logits || !pool || !out || !sync || !ids_out != !wts_out) return kErrArgs;
  if (slot_bytes < kTSlot || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(sync)) & 15) return kErrArgs;
  if (!act_args_ok(alpha, limit)) return kErrArgs;
  if (!one_resident_ok()) return kErrResident;
  launch_t(k_moe_one_t950<true>, dim3(kOneWgs), dim3(256), stream, events ? (hipEvent_t)events[0] : nullptr,
           events ? (hipEvent_t)events[1] : nullptr, nullptr, (const uint8_t*)pool, slot_bytes, slot_tab, expert_base,
           (const uint16_t*)x, (const uint16_t*)bias_gu, (const uint16_t*)bias_dn, nullptr, (uint16_t*)out, alpha,
           limit, (uint32_t*)sync, logits, ids_out, (uint16_t*)wts_out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_moe_one_resident(void) { return one_resident_ok() ? 1 : 0; }

int na_moe_decode_t950_noalloc(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                               long long slot_bytes, const int64_t* slot_tab, long long expert_base,
                               const void* bias_gu, const void* bias_dn, void* out, float alpha, float limit,
                               int k_split, int down_mode, hipStream_t stream) {
  if (!out) return kErrArgs;                         // the result must leave the shared scratch
  if (B > kNoAllocMaxB) return kErrTooLarge;
  uint8_t* base = static_cast<uint8_t*>(scratch_address());
  if (!base) return kErrLaunch;
  return decode_t950(x, topk_ids, topk_w, B, pool, slot_bytes, slot_tab, expert_base, bias_gu, bias_dn, base,
                     base + kNoAllocPart, out, alpha, limit, k_split, down_mode, nullptr, stream);
}

}  // extern "C"
