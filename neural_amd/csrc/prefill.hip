// MXFP4 GEMMs on gfx950 for prompt processing: the reference's mxfp4_gemm / grouped GEMM arithmetic (per 32-element
// group, E2M1 x 2^(s-127) dequantised exactly to bf16, bf16 x bf16 products accumulated in fp32, one bf16 rounding of
// each output; reference neural/q80/mxfp4_kernels.py:87-126, 242-295) and the fused MoE prefill layer (reference
// server.py:1837-1936, _expert_gemms :1977-2040).
//
// The fused layer (k_prefill_gate_up / k_prefill_down) runs on the block-scaled v_mfma_scale_f32_16x16x128_f8f6f4:
// E2M1 codes and E8M0 scales as stored, activations as two E4M3 rows (hi, lo) with one E8M0 scale per 32 elements
// each (x per 32-element block of a row; h per 32 columns of a row, quantised in the gate_up epilogue).  hi w + lo w
// is the reference's bf16 x E2M1 product exactly for every element within 2^13 of its block's largest magnitude m;
// an element further below m is reproduced to within 2^-21 m (the remainder's 4 significant bits on the lo grid),
// so an output deviates from the reference's by at most 2^-21 sum_k |w_k| m_k before its bf16 rounding (t950.h
// states the quantiser).
//
// The plain and grouped GEMM entry points (bf16 activations, no workspace) run the same tiles, the activations
// quantised into hi + lo rows while they are staged.
//
// Weight layouts (template W): the store's raw and PS4 slots (row r: 1,440 code bytes, then a raw 90-byte or PS4
// 46-byte scale row; lane (q, n) reads the 16 bytes of group 4t + q of row n, already the MFMA's B order) and the t950
// tiles (lane (q, n) reads the 16 bytes at 1024 t + 16 (16 q + n) of the row block: the same operand).
#include "common.h"
#include "t950.h"

#include <hip/hip_ext.h>

namespace na {

enum WLayout : int { kWRaw = 0, kWPs4 = 1, kWT950 = 2 };

constexpr int kPBM = 64;                 // tokens per tile
constexpr int kPKT = 128;                // K elements per k-tile
constexpr int kPTiles = kTTiles;         // 23 k-tiles: 22 full + groups 88, 89

// One matrix (gate_up or down) of one expert, as the kernels address it.
struct WSrc {
  const uint8_t* codes;     // raw/PS4: row 0's code bytes (row pitch 1,440); t950: block 0 of the matrix
  const uint8_t* scales;    // raw/PS4: row 0's scale row (pitch 90 or 46); t950: unused
};

// Store layouts (raw, PS4): the 16 code bytes of (row n, group 4t + q) of row block rblk for lane 16 q + n, and that
// group's E8M0 scale.
template <int W>
NA_DEVICE void w_load(const WSrc& s, int rblk, int t, int lane, uint4& c, uint32_t& sc) {
  const int q = lane >> 4, n = lane & 15;
  const int r = rblk * 16 + n;
  const int g = min(4 * t + q, kGK - 1);             // groups 90, 91 of the last k-tile: zeroed at the use
  c = load16<true>(s.codes + (long long)r * kRowBytes + 16 * g);
  if constexpr (W == kWRaw) {
    sc = s.scales[(long long)r * kGK + g];
  } else {
    const uint8_t* row = s.scales + (long long)r * kPs4Row;
    const uint32_t nib = row[1 + (g >> 1)];
    sc = row[0] + ((g & 1) ? (nib >> 4) : (nib & 15));
  }
}

constexpr int kPNB = 3;                  // row blocks per wave in the plain, grouped and down kernels
constexpr int kPRows = 4 * kPNB * 16;    // 192 weight rows per workgroup

template <int W>
NA_DEVICE WSrc w_src(const uint8_t* blocks, long long sb_slot, const uint8_t* scales, long long ss_slot,
                     long long slot) {
  return WSrc{blocks + slot * sb_slot, scales ? scales + slot * ss_slot : nullptr};
}

// ------------------------------------------------------------------------------------ fused MoE prefill layer
// Routing: pairs p = 4 t + k (token t, rank k); valid expert ids in [0, 128).  counts[e], then a stable order of the
// pairs by expert (order[offs[e] + i] = the i-th pair of expert e in increasing p) and a tile table
// tiles[i] = (expert, first sorted position, rows <= 64), ntiles.  Invalid ids are in no expert's list and
// contribute +0 (the combine skips them).
// Quantised row ("q row", kQRow bytes): hi codes [0, 2880), lo codes [2880, 5760), hi scales [5760, 5856) and lo
// scales [5856, 5952), scale bytes 90..95 of each half zero (the last k-tile's groups 90, 91 are padding).
constexpr int kQRow = 2 * kH + 2 * kX8ScPitch;        // 5,952
constexpr int kQLo = kH;
constexpr int kQSh = 2 * kH;
constexpr int kQSl = 2 * kH + kX8ScPitch;

struct PTile {
  int e, p0, cnt, pad;
};

// Blocks 0..127: counts[e] = pairs routed to expert e.  Blocks 128..: x quantised into q rows, one 8-element chunk
// per thread (4 consecutive threads = one 32-element block; 360 chunks per row, so a block never straddles rows).
__global__ __launch_bounds__(256) void k_prefill_count(const int64_t* __restrict__ ids, int P, int* __restrict__ counts,
                                                       const uint16_t* __restrict__ x, int T, uint8_t* __restrict__ xq) {
  if (blockIdx.x >= 128) {
    const long long g = (long long)(blockIdx.x - 128) * 256 + threadIdx.x;
    const bool ok = g < (long long)T * kChunks;
    const long long row = ok ? g / kChunks : 0;
    const int c = ok ? (int)(g - row * kChunks) : 0;
    const uint4 v = ok ? *reinterpret_cast<const uint4*>(x + row * kH + 8 * c) : make_uint4(0, 0, 0, 0);
    uint2 hi, lo;
    uint32_t sh, sl;
    x8_quant_chunk(v, hi, lo, sh, sl);
    if (ok) {
      uint8_t* dst = xq + row * kQRow;
      *reinterpret_cast<uint2*>(dst + 8 * c) = hi;
      *reinterpret_cast<uint2*>(dst + kQLo + 8 * c) = lo;
      if ((c & 3) == 0) {
        dst[kQSh + (c >> 2)] = (uint8_t)sh;
        dst[kQSl + (c >> 2)] = (uint8_t)sl;
      }
      if (c < kX8ScPitch - kGK) {
        dst[kQSh + kGK + c] = 0;
        dst[kQSl + kGK + c] = 0;
      }
    }
    return;
  }
  const int e = blockIdx.x;
  __shared__ int part[4];
  int c = 0;
  for (int p = threadIdx.x; p < P; p += 256) c += ids[p] == e;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = c;
  __syncthreads();
  if (threadIdx.x == 0) counts[e] = part[0] + part[1] + part[2] + part[3];
}

// Block e: the expert's tiles and its pairs in increasing p.  The prefix over the experts before e comes from one
// wave's shuffles; the pairs are walked 8,192 at a time, wave w taking 2,048 consecutive ones in 32 coalesced steps of
// 64: one ballot per step gives each lane its place among the wave's hits, and a 4-entry scan places the waves.
__global__ __launch_bounds__(256) void k_prefill_order(const int64_t* __restrict__ ids, int P,
                                                       const int* __restrict__ counts, int* __restrict__ order,
                                                       PTile* __restrict__ tiles, int* __restrict__ ntiles) {
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int wcnt[4];
  __shared__ int base_s[2];
  if (wave == 0) {
    const int c0 = counts[lane], c1 = counts[64 + lane];
    const int t0 = (c0 + kPBM - 1) / kPBM, t1 = (c1 + kPBM - 1) / kPBM;
    int off = (lane < e ? c0 : 0) + (64 + lane < e ? c1 : 0);
    int tb = (lane < e ? t0 : 0) + (64 + lane < e ? t1 : 0);
    int tt = t0 + t1;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      off += __shfl_xor(off, o);
      tb += __shfl_xor(tb, o);
      tt += __shfl_xor(tt, o);
    }
    if (lane == 0) {
      base_s[0] = off;
      base_s[1] = tb;
      if (e == 0) *ntiles = tt;
    }
  }
  __syncthreads();
  const int off = base_s[0], tb = base_s[1], c = counts[e];
  for (int m = tid; m * kPBM < c; m += 256) tiles[tb + m] = PTile{e, off + m * kPBM, min(kPBM, c - m * kPBM), 0};
  const uint64_t lt = (1ull << lane) - 1;
  int run = 0;                                        // pairs of expert e before this round
  for (int p0 = 0; p0 < P; p0 += 8192) {
    const int wp0 = p0 + 2048 * wave;
    uint64_t bal[32];
    int wn = 0;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const int p = wp0 + 64 * j + lane;
      bal[j] = __ballot(p < P && ids[p] == e);
      wn += __popcll(bal[j]);
    }
    if (lane == 0) wcnt[wave] = wn;
    __syncthreads();
    int pos = off + run;
    for (int w = 0; w < wave; ++w) pos += wcnt[w];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      if ((bal[j] >> lane) & 1) order[pos + __popcll(bal[j] & lt)] = wp0 + 64 * j + lane;
      pos += __popcll(bal[j]);
    }
    run += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    __syncthreads();
  }
}

// ---------------------------------------------------------------- block-scaled products of the fused layer
// The layer's two GEMMs run on v_mfma_scale_f32_16x16x128_f8f6f4 with the E2M1 codes and E8M0 scales as stored (B)
// and the activations as two exact E4M3 rows (A: hi and lo, one E8M0 scale per 32-element block each; the exactness
// argument is the one of x8_quant_chunk in t950.h).  Each k-tile of 128 elements is one MFMA per (16 tokens, 16 weight
// rows) and activation row (hi, lo): the hi + lo products are the reference's bf16 x E2M1 products, accumulated in
// fp32.  Activations are quantised once per row, not per workgroup: x per token by the first launch, h per sorted pair
// by the gate_up epilogue.
//
constexpr int kQPitch = 2 * kPKT + 16;                 // LDS bytes per staged row: hi 128 | lo 128 | pad 16
constexpr int kQStage = kPBM * kQPitch + kPBM * 8;     // one k-tile: 64 rows, then 8 scale bytes per row
constexpr int kGuSlots = 3;                            // gate_up: 23 column groups over 8 XCDs, 3 per XCD
constexpr int kDnSlots = 2;                            // down: 15 column groups, 2 per XCD
constexpr int kYPitch = 2 * kPRows + 16;              // LDS bytes per row of a staged down output tile
constexpr int kOhPitch = 2 * kPKT + 8;                 // LDS bytes per row of gate_up's staged h codes (rows 4 apart
                                                       // start 8 banks apart)

// Staging of one k-tile of 64 q rows: pieces of 16 B, thread tid owns piece (tid & 15) of rows (tid >> 4) + 16 i
// (pieces 0..7 hi, 8..15 lo); threads 0..63 also own the 4 hi and 4 lo scale bytes of row tid, stored interleaved
// (hi g, lo g) per group g of the k-tile.
struct QStage {
  uint4 v[4];
  uint2 s;
};

// Activation rows that arrive quantised (q rows): rp[i] = q row of staged row (tid >> 4) + 16 i, srow = q row of
// staged row tid & 63.
struct QRows {
  using Stage = QStage;
  const uint8_t* rp[4];
  const uint8_t* srow;

  NA_DEVICE void load(int t, int tid, QStage& a) const {
    const int c16 = tid & 15, e0 = t * kPKT + 16 * (c16 & 7), half = (c16 >> 3) * kQLo;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a.v[i] = e0 < kH ? *reinterpret_cast<const uint4*>(rp[i] + half + e0) : make_uint4(0, 0, 0, 0);
    if (tid < 64) {
      a.s.x = *reinterpret_cast<const uint32_t*>(srow + kQSh + 4 * t);
      a.s.y = *reinterpret_cast<const uint32_t*>(srow + kQSl + 4 * t);
    }
  }
  NA_DEVICE void store(uint8_t* buf, int tid, const QStage& a) const {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<uint4*>(buf + ((tid >> 4) + 16 * i) * kQPitch + 16 * (tid & 15)) = a.v[i];
    if (tid < 64)                                      // interleaved at the store, so the loads are not waited on early
      *reinterpret_cast<uint2*>(buf + kPBM * kQPitch + 8 * tid) =
          make_uint2(__byte_perm(a.s.x, a.s.y, 0x5140), __byte_perm(a.s.x, a.s.y, 0x7362));
  }
};

// bf16 activation rows quantised while they are staged (the GEMM entry points, which have no workspace): thread tid
// owns the 8-element piece tid & 15 of rows (tid >> 4) + 16 i, so the 4 pieces of a 32-element block sit in 4
// consecutive lanes, as x8_quant_chunk needs.  rp[i] = bf16 row of staged row (tid >> 4) + 16 i.
struct XStage {
  uint4 v[4];
};

struct XRows {
  using Stage = XStage;
  const uint16_t* rp[4];

  NA_DEVICE void load(int t, int tid, XStage& a) const {
    const int e0 = t * kPKT + 8 * (tid & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a.v[i] = e0 < kH ? *reinterpret_cast<const uint4*>(rp[i] + e0) : make_uint4(0, 0, 0, 0);
  }
  NA_DEVICE void store(uint8_t* buf, int tid, const XStage& a) const {
    const int c16 = tid & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint2 hi, lo;
      uint32_t sh, sl;
      x8_quant_chunk(a.v[i], hi, lo, sh, sl);
      const int row = (tid >> 4) + 16 * i;
      *reinterpret_cast<uint2*>(buf + row * kQPitch + 8 * c16) = hi;
      *reinterpret_cast<uint2*>(buf + row * kQPitch + kPKT + 8 * c16) = lo;
      if ((c16 & 3) == 0)
        *reinterpret_cast<uint16_t*>(buf + kPBM * kQPitch + row * 8 + 2 * (c16 >> 2)) = (uint16_t)(sh | (sl << 8));
    }
  }
};

// FP4 B operand of k-tile t in the MFMA order (lane 16 kb + n: the 16 code bytes of group 4t + kb of row n), groups
// beyond K zeroed.  Every layout's load already is in that order.
NA_DEVICE mfma_i32x8_t w_operand8(uint4 c, int t, int lane) {
  if (4 * t + (lane >> 4) >= kGK) c = make_uint4(0, 0, 0, 0);
  return mfma_i32x8_t{(int)c.x, (int)c.y, (int)c.z, (int)c.w, 0, 0, 0, 0};
}

constexpr int kWScBytes = kTRows * kTScalePitch;      // 1,536 E8M0 bytes of one t950 row block

// One wave's weight stream over its NB row blocks.  t950: the code bytes of a k-tile per load (the E8M0 rows of the
// blocks are staged once in the wave's LDS area wsc and read per k-tile from there); raw / PS4: codes and the lane's
// scale per load.
template <int W, int NB>
struct WStream {
  WSrc src;
  const int* blk;
  const uint8_t* wsc;
  int lane;

  NA_DEVICE void load(int t, uint4 (&c)[NB], uint32_t (&sc)[NB]) const {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      if constexpr (W == kWT950) {
        const uint8_t* bk = src.codes + (long long)blk[nb] * kTBlock;
        c[nb] = load16(bk + t * 1024 + 16 * lane);
        sc[nb] = 0;
      } else {
        w_load<W>(src, blk[nb], t, lane, c[nb], sc[nb]);
      }
    }
  }
  NA_DEVICE int scale(int t, int nb, uint32_t sc) const {
    if constexpr (W == kWT950)
      return wsc[nb * kWScBytes + (lane & 15) * kTScalePitch + 4 * t + (lane >> 4)];
    else
      return (int)(sc & 0xff);
  }
};

// One k-tile of gemm8_tile.  A of k-tile t is staged in LDS at cur and the weights of k-tile t are in (c, sc).  It
// issues the loads of A of k-tile t + 2 (into a_in) and of the weights of k-tile t + 2 (into (c2, sc2)), runs the
// MFMAs, stores A of k-tile t + 1 (loaded one step earlier, a_out) at nxt and meets the barrier.
template <int W, int NB, int NT, typename S>
NA_DEVICE void gemm8_step(int t, const WStream<W, NB>& ws, bool live, const S& st, const uint8_t* cur, uint8_t* nxt,
                          const typename S::Stage& a_out, typename S::Stage& a_in,
                          const uint4 (&c)[NB], const uint32_t (&sc)[NB], uint4 (&c2)[NB], uint32_t (&sc2)[NB],
                          f32x4_t (&acc)[4][NB]) {
  const int tid = threadIdx.x, lane = tid & 63, kb = lane >> 4, m = lane & 15;
  if (t + 2 < kPTiles) {
    st.load(t + 2, tid, a_in);
    ws.load(t + 2, c2, sc2);
  }
  if (live) {
    mfma_i32x8_t b[NB];
    int sb[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      b[nb] = w_operand8(c[nb], t, lane);
      sb[nb] = ws.scale(t, nb, sc[nb]);
    }
    __builtin_amdgcn_s_setprio(1);                     // the MFMA burst issues ahead of the other wave's staging
#pragma unroll
    for (int tt = 0; tt < NT; ++tt) {
      const uint8_t* row = cur + (16 * tt + m) * kQPitch + 16 * kb;
      const uint4 h0 = *reinterpret_cast<const uint4*>(row), h1 = *reinterpret_cast<const uint4*>(row + 64);
      const uint4 l0 = *reinterpret_cast<const uint4*>(row + 128), l1 = *reinterpret_cast<const uint4*>(row + 192);
      const uint32_t s2 = *reinterpret_cast<const uint16_t*>(cur + kPBM * kQPitch + (16 * tt + m) * 8 + 2 * kb);
      const int sh = (int)(s2 & 0xff), sl = (int)(s2 >> 8);
      const mfma_i32x8_t ah = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
      const mfma_i32x8_t al = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc[tt][nb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(ah, b[nb], acc[tt][nb], 0, 4, 0, sh, 0, sb[nb]);
        acc[tt][nb] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(al, b[nb], acc[tt][nb], 0, 4, 0, sl, 0, sb[nb]);
      }
    }
  }
  // The MFMAs are issued before the LDS stores, which wait for their k-tile's loads: an empty asm that takes every
  // accumulator (and orders memory) keeps the compiler from sinking the MFMAs below those stores.
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) asm volatile("" : "+v"(acc[tt][nb])::"memory");
  __builtin_amdgcn_s_setprio(0);
  if (t + 1 < kPTiles) st.store(nxt, tid, a_out);
  __syncthreads();
}

// acc[tt][nb] = D of tokens 16 tt .. 16 tt + 15 x row block blk[nb] (lane (q, n): tokens 16 tt + 4 q + r, row n),
// over the 23 k-tiles for tt < NT (the 16-token blocks that hold rows; the others stay zero); st stages the
// activation rows (QRows or XRows).  Both
// operand streams run two k-tiles ahead of the MFMAs: the activations through three LDS buffers of a k-tile (64 rows'
// 256 code bytes and 8 scale bytes each, loaded into registers two steps before and stored one step before their
// use), each wave's weight codes through three register sets; the k-loop is unrolled by 3 so that every buffer and
// register set is fixed at compile time.  Each wave reads one token tile's hi and lo fragments at a time and feeds
// them to its NB row blocks.  lds: 3 x kQStage bytes; wsc: this wave's LDS area of NB x 1,536 bytes (t950 scale
// rows).  A wave without work (live = false) stages and meets every barrier but runs no MFMA.  All 256 threads must
// call it.
template <int W, int NB, int NT, typename S>
NA_DEVICE void gemm8_tile_n(const WSrc& src, const int (&blk)[NB], bool live, const S& st, uint8_t* lds, uint8_t* wsc,
                            f32x4_t (&acc)[4][NB]) {
  const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[tt][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const WStream<W, NB> ws{src, blk, wsc, lane};
  if constexpr (W == kWT950) {                         // the blocks' E8M0 rows: 96 pieces of 16 B each
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint8_t* sp = src.codes + (long long)blk[nb] * kTBlock + kTCodes;
      const uint4 v0 = load16(sp + 16 * lane);
      *reinterpret_cast<uint4*>(wsc + nb * kWScBytes + 16 * lane) = v0;
      if (lane < kWScBytes / 16 - 64) {
        const uint4 v1 = load16(sp + 1024 + 16 * lane);
        *reinterpret_cast<uint4*>(wsc + nb * kWScBytes + 1024 + 16 * lane) = v1;
      }
    }
  }
  uint8_t* const b0 = lds;
  uint8_t* const b1 = lds + kQStage;
  uint8_t* const b2 = lds + 2 * kQStage;
  uint4 c0[NB], c1[NB], c2[NB];
  uint32_t s0[NB], s1[NB], s2[NB];
  typename S::Stage a0, a1, a2;                        // a_k: A of the k-tiles = k (mod 3) while in flight
  st.load(0, tid, a0);
  ws.load(0, c0, s0);
  st.load(1, tid, a1);
  ws.load(1, c1, s1);
  st.store(b0, tid, a0);
  __syncthreads();
  int t = 0;
  for (; t + 3 <= kPTiles; t += 3) {                   // k-tiles 0 .. 20
    gemm8_step<W, NB, NT, S>(t, ws, live, st, b0, b1, a1, a2, c0, s0, c2, s2, acc);
    gemm8_step<W, NB, NT, S>(t + 1, ws, live, st, b1, b2, a2, a0, c1, s1, c0, s0, acc);
    gemm8_step<W, NB, NT, S>(t + 2, ws, live, st, b2, b0, a0, a1, c2, s2, c1, s1, acc);
  }
  gemm8_step<W, NB, NT, S>(t, ws, live, st, b0, b1, a1, a2, c0, s0, c2, s2, acc);       // 21
  gemm8_step<W, NB, NT, S>(t + 1, ws, live, st, b1, b2, a2, a0, c1, s1, c0, s0, acc);   // 22
}

// gemm8_tile_n for a tile whose rows fill ntt (1..4) 16-token blocks: the MFMAs of empty blocks are not issued
// (variants for 1, 2 and 4 blocks; 3 runs as 4).  ntt is workgroup-uniform.
template <int W, int NB, typename S>
NA_DEVICE void gemm8_tile(const WSrc& src, const int (&blk)[NB], bool live, int ntt, const S& st, uint8_t* lds,
                          uint8_t* wsc, f32x4_t (&acc)[4][NB]) {
  if (ntt > 2)
    gemm8_tile_n<W, NB, 4, S>(src, blk, live, st, lds, wsc, acc);
  else if (ntt == 2)
    gemm8_tile_n<W, NB, 2, S>(src, blk, live, st, lds, wsc, acc);
  else
    gemm8_tile_n<W, NB, 1, S>(src, blk, live, st, lds, wsc, acc);
}

// Workgroup b -> (tile, column group): the dispatcher deals workgroups to the 8 XCDs in turn (XCD b % 8), so XCD x
// is given column groups slots * x .. slots * x + slots - 1 of every tile, tiles in order.  Each XCD's L2 then holds
// the weight rows of its few column groups while the tiles of one expert pass through it, and every weight byte
// crosses from HBM about once.
template <int SLOTS>
NA_DEVICE void xcd_tile(int b, int& tile, int& col) {
  const int s = b >> 3;
  tile = s / SLOTS;
  col = SLOTS * (b & 7) + s % SLOTS;
}

// gate_up + bias + clamped SwiGLU on the block-scaled MFMA: tile i, column group y (128 intermediate columns).
// Wave w owns intermediate blocks jb, jb + 1 (jb = 8 y + 2 w) and reads their gate rows (blocks jb, jb + 1) and up
// rows (blocks 180 + jb, 181 + jb), so the SwiGLU pairs registers of one lane.  x rows come quantised (xq, one q row
// per token) and are gathered through the pair order; h leaves as q rows in sorted pair order, each 32-column block
// (one wave's columns of one row) with its own E8M0 scales.  Grid: max tiles x 24 (xcd_tile<3>); in column group 22
// waves 2 and 3 have no blocks.
template <int W>
__global__ __launch_bounds__(256, W == kWT950 ? 2 : 1) void k_prefill_gate_up(
    const uint8_t* __restrict__ xq, const int* __restrict__ order, const PTile* __restrict__ tiles,
    const int* __restrict__ ntiles, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ bias_gu,
    uint8_t* __restrict__ hq, float alpha, float limit) {
  __shared__ __align__(16) uint8_t lds[3 * kQStage + 4 * 4 * kWScBytes];
  int ti, y;
  xcd_tile<kGuSlots>(blockIdx.x, ti, y);
  if (ti >= *ntiles || y >= 23) return;
  const PTile tl = tiles[ti];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, q = lane >> 4,
            n = lane & 15;
  const int jb = 8 * y + 2 * wave;
  const bool live = jb < kTUpBlock0;
  const int jl = live ? jb : 0;
  const int blk[4] = {jl, jl + 1, kTUpBlock0 + jl, kTUpBlock0 + jl + 1};
  const long long gid = expert_base + tl.e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sb = pool + slot * slot_bytes;
  const WSrc src = W == kWT950 ? WSrc{sb, nullptr} : WSrc{sb, sb + kOffGateScales};
  QRows st;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    st.rp[i] = xq + (long long)(order[tl.p0 + min((tid >> 4) + 16 * i, tl.cnt - 1)] >> 2) * kQRow;
  st.srow = xq + (long long)(order[tl.p0 + min(tid & 63, tl.cnt - 1)] >> 2) * kQRow;
  f32x4_t acc[4][4];
  const int ntt = (tl.cnt + 15) >> 4;
  gemm8_tile<W, 4>(src, blk, live, ntt, st, lds, lds + 3 * kQStage + wave * 4 * kWScBytes, acc);
  // h = bf16(SwiGLU(bf16(acc) + bias)) (the reference's bf16 rounding points), quantised per (row, 32-column block)
  // into LDS: oh[row] = hi codes of the workgroup's 128 columns | lo codes, os[row] = 4 hi | 4 lo scale bytes.
  uint8_t* oh = lds;
  uint8_t* os = lds + kPBM * kOhPitch;
  if (live) {
    const uint16_t* bg = bias_gu ? bias_gu + gid * kGU : nullptr;
    float bgv[2], buv[2];
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      const int j = 16 * (jl + hb) + n;
      bgv[hb] = bg ? bf16_to_f32(bg[j]) : 0.f;
      buv[hb] = bg ? bf16_to_f32(bg[kI + j]) : 0.f;
    }
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      if (tt >= ntt) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float hv[2];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          float g = rb(acc[tt][hb][r]), u = rb(acc[tt][2 + hb][r]);
          if (bg) {
            g = rb(g + bgv[hb]);
            u = rb(u + buv[hb]);
          }
          hv[hb] = rb(swiglu_clamp_bf16(g, u, alpha, limit));
        }
        const float mx = row16_max(fmaxf(fabsf(hv[0]), fabsf(hv[1])));
        const uint32_t sh = x8_scale_byte(mx);
        const float s_hi = e8m0_f32(sh);
        fp8x2_t o2 = {0, 0};
        o2 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(o2, hv[0], hv[1], s_hi, false);
        const uint32_t hc = __builtin_bit_cast(uint32_t, o2);
        const auto d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(hc, s_hi, false);
        const float r0 = hv[0] - d[0], r1 = hv[1] - d[1];
        const float mr = row16_max(fmaxf(fabsf(r0), fabsf(r1)));
        const uint32_t sl = x8_scale_byte(mr);
        fp8x2_t l2 = {0, 0};
        l2 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(l2, r0, r1, e8m0_f32(sl), false);
        const uint32_t lc = __builtin_bit_cast(uint32_t, l2);
        const int row = 16 * tt + 4 * q + r, c = 32 * wave + n;
        oh[row * kOhPitch + c] = (uint8_t)hc;
        oh[row * kOhPitch + c + 16] = (uint8_t)(hc >> 8);
        oh[row * kOhPitch + kPKT + c] = (uint8_t)lc;
        oh[row * kOhPitch + kPKT + c + 16] = (uint8_t)(lc >> 8);
        if (n == 0) {
          os[row * 8 + wave] = (uint8_t)sh;
          os[row * 8 + 4 + wave] = (uint8_t)sl;
        }
      }
    }
  }
  __syncthreads();
  // q rows out: 16-byte pieces of the valid columns (64 in column group 22), scale bytes 4 y .. 4 y + 3 (group 22:
  // bytes 88, 89 and the zero padding 90..95).
  const int ncol = y == 22 ? 64 : 128;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pc = tid + 256 * i, row = pc >> 4, c16 = pc & 15, c8 = c16 & 7;
    if (row < tl.cnt && 16 * c8 < ncol) {
      const uint2 a0 = *reinterpret_cast<const uint2*>(oh + row * kOhPitch + 16 * c16);
      const uint2 a1 = *reinterpret_cast<const uint2*>(oh + row * kOhPitch + 16 * c16 + 8);
      *reinterpret_cast<uint4*>(hq + (long long)(tl.p0 + row) * kQRow + (c16 >> 3) * kQLo + kPKT * y + 16 * c8) =
          make_uint4(a0.x, a0.y, a1.x, a1.y);
    }
  }
  if (tid < tl.cnt && tid < kPBM) {
    uint8_t* dst = hq + (long long)(tl.p0 + tid) * kQRow;
    const uint32_t sh4 = *reinterpret_cast<const uint32_t*>(os + tid * 8);
    const uint32_t sl4 = *reinterpret_cast<const uint32_t*>(os + tid * 8 + 4);
    if (y < 22) {
      *reinterpret_cast<uint32_t*>(dst + kQSh + 4 * y) = sh4;
      *reinterpret_cast<uint32_t*>(dst + kQSl + 4 * y) = sl4;
    } else {
      *reinterpret_cast<uint2*>(dst + kQSh + 88) = make_uint2(sh4 & 0xffff, 0);
      *reinterpret_cast<uint2*>(dst + kQSl + 88) = make_uint2(sl4 & 0xffff, 0);
    }
  }
}

// down + bias, x routing weight, scattered back to pair order: ys[p][n] = bf16(bf16(bf16(y) + b) * w[p]) with p the
// pair of sorted position p0 + m.  A = the h q rows of the tile (consecutive sorted positions).  Grid: max tiles x 16
// (xcd_tile<2>); wave w: row blocks 12 y + 3 w + i.
template <int W>
__global__ __launch_bounds__(256, W == kWT950 ? 2 : 1) void k_prefill_down(
    const uint8_t* __restrict__ hq, const int* __restrict__ order, const PTile* __restrict__ tiles,
    const int* __restrict__ ntiles, const uint16_t* __restrict__ wts, const uint8_t* __restrict__ pool,
    long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
    const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ ys) {
  __shared__ __align__(16) uint8_t lds[3 * kQStage + 4 * kPNB * kWScBytes];
  int ti, y;
  xcd_tile<kDnSlots>(blockIdx.x, ti, y);
  if (ti >= *ntiles || y >= kH / kPRows) return;
  const PTile tl = tiles[ti];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, q = lane >> 4,
            n = lane & 15;
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = y * (4 * kPNB) + kPNB * wave + i;
  const long long gid = expert_base + tl.e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sb = pool + slot * slot_bytes;
  const WSrc src = W == kWT950 ? WSrc{sb + kTDownOff, nullptr}
                               : WSrc{sb + kOffDownCodes, sb + kOffGateScales + (long long)kGU * (W == kWRaw ? kGK : kPs4Row)};
  QRows st;
#pragma unroll
  for (int i = 0; i < 4; ++i) st.rp[i] = hq + (long long)(tl.p0 + min((tid >> 4) + 16 * i, tl.cnt - 1)) * kQRow;
  st.srow = hq + (long long)(tl.p0 + min(tid & 63, tl.cnt - 1)) * kQRow;
  f32x4_t acc[4][kPNB];
  const int ntt = (tl.cnt + 15) >> 4;
  gemm8_tile<W, kPNB>(src, blk, true, ntt, st, lds, lds + 3 * kQStage + wave * kPNB * kWScBytes, acc);
  // y = bf16(bf16(bf16(acc) + b) * w[p]) per element, staged as the tile's 64 rows x 192 columns in LDS (the A stages
  // are free after the last k-tile's barrier), then written back with 16-byte stores: one 384-byte piece per pair.
  uint8_t* yt = lds;
  float wv[4][4];                                     // routing weight of each of the lane's 16 tokens
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) wv[tt][r] = bf16_to_f32(wts[order[tl.p0 + min(16 * tt + 4 * q + r, tl.cnt - 1)]]);
#pragma unroll
  for (int nb = 0; nb < kPNB; ++nb) {
    const int cl = 16 * (kPNB * wave + nb) + n;        // column within the workgroup's 192
    const float bd = bias_dn ? bf16_to_f32(bias_dn[gid * kH + 16 * blk[nb] + n]) : 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      if (tt >= ntt) break;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float yv = rb(acc[tt][nb][r]);
        if (bias_dn) yv = rb(yv + bd);
        const uint32_t v = f32_to_bf16(yv * wv[tt][r]);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false) & 0xffff;
        if (!(n & 1))
          *reinterpret_cast<uint32_t*>(yt + (16 * tt + 4 * q + r) * kYPitch + 2 * cl) = v | (hi << 16);
      }
    }
  }
  __syncthreads();
  constexpr int kPieces = kPRows * 2 / 16;            // 24 pieces of 16 bytes per row
#pragma unroll
  for (int i = 0; i < kPBM * kPieces / 256; ++i) {
    const int pc = tid + 256 * i, row = pc / kPieces, piece = pc - row * kPieces;
    if (row < tl.cnt)
      *reinterpret_cast<uint4*>(ys + (long long)order[tl.p0 + row] * kH + kPRows * y + 8 * piece) =
          *reinterpret_cast<const uint4*>(yt + row * kYPitch + 16 * piece);
  }
}

// ------------------------------------------------------------------------------- plain GEMM (mxfp4_gemm)
// out[e][m][n] = bf16(sum_k x[m][k] w_e[n][k]); grid (E * ceil(M / 64), N / 192); wave w: row blocks 12 y + 3 w + i.
// The same block-scaled tiles as the fused layer, the activations quantised into hi + lo rows while staged.
NA_DEVICE void store_tile(uint16_t* out_row0, long long pitch, const f32x4_t (&acc)[4][kPNB], const int (&blk)[kPNB],
                          int m_limit) {
  const int lane = threadIdx.x & 63, q = lane >> 4, n = lane & 15;
#pragma unroll
  for (int nb = 0; nb < kPNB; ++nb)
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * tt + 4 * q + r;
        const uint32_t v = f32_to_bf16(acc[tt][nb][r]);
        const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false) & 0xffff;
        if (m < m_limit && !(n & 1))
          *reinterpret_cast<uint32_t*>(out_row0 + (long long)m * pitch + 16 * blk[nb] + n) = (uint32_t)v | (hi << 16);
      }
}

template <int W>
__global__ __launch_bounds__(256, 2) void k_mxfp4_gemm(const uint16_t* __restrict__ x, int M,
                                                       const uint8_t* __restrict__ blocks, long long sb_slot,
                                                       const uint8_t* __restrict__ scales, long long ss_slot,
                                                       const int64_t* __restrict__ slots, uint16_t* __restrict__ out,
                                                       int N) {
  __shared__ __align__(16) uint8_t lds[3 * kQStage + 4 * kPNB * kWScBytes];
  const int mt = (M + kPBM - 1) / kPBM;
  const int e = blockIdx.x / mt, m0 = (blockIdx.x - e * mt) * kPBM;
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = blockIdx.y * (4 * kPNB) + kPNB * wave + i;
  const WSrc src = w_src<W>(blocks, sb_slot, scales, ss_slot, slots[e]);
  XRows st;
#pragma unroll
  for (int i = 0; i < 4; ++i) st.rp[i] = x + (long long)min(m0 + (tid >> 4) + 16 * i, M - 1) * kH;
  f32x4_t acc[4][kPNB];
  gemm8_tile_n<W, kPNB, 4>(src, blk, true, st, lds, lds + 3 * kQStage + wave * kPNB * kWScBytes, acc);
  store_tile(out + ((long long)e * M + m0) * N, N, acc, blk, M - m0);
}

// --------------------------------------------------------------- grouped GEMM (GroupedGemmPlan descriptors)
// tiles int64 [ntiles][5] = (x address, out address, slot, pair M, pm); rows [pm * block_m, min(M, pm * block_m +
// block_m)) of the pair, walked in 64-row sub-tiles (block_m <= 64: one).  grid (ntiles, N / 192).
template <int W>
__global__ __launch_bounds__(256) void k_mxfp4_gemm_grouped(const uint8_t* __restrict__ blocks, long long sb_slot,
                                                               const uint8_t* __restrict__ scales, long long ss_slot,
                                                               const int64_t* __restrict__ tiles, int block_m, int N) {
  __shared__ __align__(16) uint8_t lds[3 * kQStage + 4 * kPNB * kWScBytes];
  const int64_t* d = tiles + (long long)blockIdx.x * 5;
  const uint16_t* x = reinterpret_cast<const uint16_t*>(d[0]);
  uint16_t* out = reinterpret_cast<uint16_t*>(d[1]);
  const long long slot = d[2];
  const int M = (int)d[3], pm = (int)d[4];
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = blockIdx.y * (4 * kPNB) + kPNB * wave + i;
  const WSrc src = w_src<W>(blocks, sb_slot, scales, ss_slot, slot);
  const int r0 = pm * block_m, r1 = min(M, r0 + block_m);
  for (int m0 = r0; m0 < r1; m0 += kPBM) {
    XRows st;
#pragma unroll
    for (int i = 0; i < 4; ++i) st.rp[i] = x + (long long)min(m0 + (tid >> 4) + 16 * i, r1 - 1) * kH;
    f32x4_t acc[4][kPNB];
    gemm8_tile_n<W, kPNB, 4>(src, blk, true, st, lds, lds + 3 * kQStage + wave * kPNB * kWScBytes, acc);
    store_tile(out + (long long)m0 * N, N, acc, blk, r1 - m0);
    __syncthreads();                                   // the next sub-tile restages the scale rows and buffers
  }
}

// out[t][n] = bf16(sum_k ys[4 t + k][n]) over the valid ranks k, fp32 sum in top-k order (server.py:2340-2341).
// One thread per 8 columns of a token: 16-byte loads of the four ranks' rows, one 16-byte store.
__global__ __launch_bounds__(256) void k_prefill_combine(const uint16_t* __restrict__ ys, const int64_t* __restrict__ ids,
                                                         int T, uint16_t* __restrict__ out) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)T * (kH / 8)) return;
  const int t = (int)(i / (kH / 8)), c8 = (int)(i - (long long)t * (kH / 8));
  float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  uint4 v[4];
  bool ok[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {                       // all four loads in flight before the sums
    const long long e = ids[4 * t + k];
    ok[k] = e >= 0 && e < 128;
    v[k] = ok[k] ? *reinterpret_cast<const uint4*>(ys + (long long)(4 * t + k) * kH + 8 * c8) : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (!ok[k]) continue;
    const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[2 * j] += bf16_to_f32((uint16_t)(w[j] & 0xffff));
      a[2 * j + 1] += bf16_to_f32((uint16_t)(w[j] >> 16));
    }
  }
  uint4 o;
  o.x = (uint32_t)f32_to_bf16(a[0]) | ((uint32_t)f32_to_bf16(a[1]) << 16);
  o.y = (uint32_t)f32_to_bf16(a[2]) | ((uint32_t)f32_to_bf16(a[3]) << 16);
  o.z = (uint32_t)f32_to_bf16(a[4]) | ((uint32_t)f32_to_bf16(a[5]) << 16);
  o.w = (uint32_t)f32_to_bf16(a[6]) | ((uint32_t)f32_to_bf16(a[7]) << 16);
  *reinterpret_cast<uint4*>(out + (long long)t * kH + 8 * c8) = o;
}

// Workspace of the fused prefill layer for T tokens (P = 4 T pairs): byte offsets, 256-aligned.
struct PrefillWs {
  long long counts, ntiles, order, tiles, xq, h, ys, total;
  int max_tiles;
};

static long long align256(long long v) { return (v + 255) & ~255LL; }

static PrefillWs prefill_ws(int T) {
  PrefillWs w;
  const long long P = 4LL * T;
  w.max_tiles = (int)(P / kPBM + 128);
  w.counts = 0;
  w.ntiles = 512;
  w.order = 1024;
  w.tiles = align256(w.order + P * 4);
  w.xq = align256(w.tiles + (long long)w.max_tiles * sizeof(PTile));
  w.h = align256(w.xq + (long long)T * kQRow);
  w.ys = align256(w.h + P * kQRow);
  w.total = align256(w.ys + P * kH * 2);
  return w;
}

template <typename... KArgs, typename... Args>
static void launch_p(void (*kern)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                     Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, e0, e1, 0, static_cast<KArgs>(args)...);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, stream, static_cast<KArgs>(args)...);
}

}  // namespace na

using namespace na;

extern "C" {

long long na_moe_prefill_workspace_bytes(int T) {
  if (T <= 0 || T > (1 << 20)) return -1;
  return prefill_ws(T).total;
}

int na_moe_prefill_workspace_layout(int T, long long* offsets) {
  if (T <= 0 || T > (1 << 20) || !offsets) return kErrArgs;
  const PrefillWs w = prefill_ws(T);
  const long long v[9] = {w.counts, w.ntiles, w.order, w.tiles, w.xq, w.h, w.ys, w.total, w.max_tiles};
  for (int i = 0; i < 9; ++i) offsets[i] = v[i];
  return kOk;
}

int na_moe_prefill(const void* x, const int64_t* topk_ids, const void* topk_w, int T, const void* pool,
                   long long slot_bytes, int layout, const int64_t* slot_tab, long long expert_base,
                   const void* bias_gu, const void* bias_dn, void* workspace, long long ws_bytes, void* out,
                   float alpha, float limit, void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !workspace || !out || T <= 0 || T > (1 << 20)) return kErrArgs;
  if (layout < kWRaw || layout > kWT950) return kErrArgs;
  const long long need = layout == kWT950 ? kTSlot : layout == kWPs4 ? kSlotPs4 : kSlotRaw;
  if (slot_bytes < need || (slot_bytes & 15) || (reinterpret_cast<uintptr_t>(pool) & 15)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(out)) & 15)
    return kErrArgs;
  const PrefillWs w = prefill_ws(T);
  if (ws_bytes < w.total) return kErrTooLarge;
  uint8_t* ws = (uint8_t*)workspace;
  int* counts = (int*)(ws + w.counts);
  int* ntiles = (int*)(ws + w.ntiles);
  int* order = (int*)(ws + w.order);
  PTile* tiles = (PTile*)(ws + w.tiles);
  uint8_t* xq = ws + w.xq;
  uint8_t* hq = ws + w.h;
  uint16_t* ys = (uint16_t*)(ws + w.ys);
  hipEvent_t ev[10] = {};
  if (events)
    for (int i = 0; i < 10; ++i) ev[i] = (hipEvent_t)events[i];
  const int P = 4 * T;
  const long long qblocks = ((long long)T * kChunks + 255) / 256;
  launch_p(k_prefill_count, dim3((unsigned)(128 + qblocks)), dim3(256), stream, ev[0], ev[1], topk_ids, P, counts,
           (const uint16_t*)x, T, xq);
  launch_p(k_prefill_order, dim3(128), dim3(256), stream, ev[2], ev[3], topk_ids, P, (const int*)counts, order, tiles,
           ntiles);
  const dim3 gg(w.max_tiles * 8 * kGuSlots), gd(w.max_tiles * 8 * kDnSlots), blk(256);
#define NA_PREFILL_GEMMS(W)                                                                                          \
  launch_p(k_prefill_gate_up<W>, gg, blk, stream, ev[4], ev[5], (const uint8_t*)xq, (const int*)order,                \
           (const PTile*)tiles, (const int*)ntiles, (const uint8_t*)pool, slot_bytes, slot_tab, expert_base,          \
           (const uint16_t*)bias_gu, hq, alpha, limit);                                                                \
  launch_p(k_prefill_down<W>, gd, blk, stream, ev[6], ev[7], (const uint8_t*)hq, (const int*)order,                    \
           (const PTile*)tiles, (const int*)ntiles, (const uint16_t*)topk_w, (const uint8_t*)pool, slot_bytes,        \
           slot_tab, expert_base, (const uint16_t*)bias_dn, ys);
  if (layout == kWT950) {
    NA_PREFILL_GEMMS(kWT950)
  } else if (layout == kWPs4) {
    NA_PREFILL_GEMMS(kWPs4)
  } else {
    NA_PREFILL_GEMMS(kWRaw)
  }
#undef NA_PREFILL_GEMMS
  const long long nc = (long long)T * (kH / 8);
  launch_p(k_prefill_combine, dim3((unsigned)((nc + 255) / 256)), dim3(256), stream, ev[8], ev[9],
           (const uint16_t*)ys, topk_ids, T, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_mxfp4_gemm(const void* x, int M, int K, const void* blocks, long long sb_slot, const void* scales,
                  long long ss_slot, int layout, const int64_t* slots, int E, void* out, int N, hipStream_t stream) {
  if (!x || !blocks || !slots || !out || M <= 0 || E <= 0 || N <= 0) return kErrArgs;
  if (K != kH || N % kPRows || layout < kWRaw || layout > kWT950 || (layout != kWT950 && !scales)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out)) & 15) return kErrArgs;
  const long long mt = (M + kPBM - 1) / kPBM;
  if (mt * E > 0x7fffffff) return kErrTooLarge;
  const dim3 grid((unsigned)(mt * E), N / kPRows), blk(256);
  auto kern = layout == kWT950 ? k_mxfp4_gemm<kWT950> : layout == kWPs4 ? k_mxfp4_gemm<kWPs4> : k_mxfp4_gemm<kWRaw>;
  hipLaunchKernelGGL(kern, grid, blk, 0, stream, (const uint16_t*)x, M, (const uint8_t*)blocks, sb_slot,
                     (const uint8_t*)scales, ss_slot, slots, (uint16_t*)out, N);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_mxfp4_gemm_grouped(const void* blocks, long long sb_slot, const void* scales, long long ss_slot, int layout,
                          const int64_t* tiles, int ntiles, int block_m, int N, int K, hipStream_t stream) {
  if (!blocks || !tiles || ntiles < 0 || N <= 0) return kErrArgs;
  if (K != kH || N % kPRows || layout < kWRaw || layout > kWT950 || (layout != kWT950 && !scales)) return kErrArgs;
  if (block_m < 16 || (block_m & (block_m - 1)) || block_m > 4096) return kErrArgs;
  if (ntiles == 0) return kOk;
  const dim3 grid(ntiles, N / kPRows), blk(256);
  auto kern = layout == kWT950 ? k_mxfp4_gemm_grouped<kWT950>
            : layout == kWPs4 ? k_mxfp4_gemm_grouped<kWPs4> : k_mxfp4_gemm_grouped<kWRaw>;
  hipLaunchKernelGGL(kern, grid, blk, 0, stream, (const uint8_t*)blocks, sb_slot, (const uint8_t*)scales, ss_slot,
                     tiles, block_m, N);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
