// MXFP4 GEMM on gfx950 for prompt processing: the reference's mxfp4_gemm / grouped GEMM arithmetic (per 32-element
// group, E2M1 x 2^(s-127) dequantised exactly to bf16, bf16 x bf16 products accumulated in fp32, one bf16 rounding of
// each output; reference neural/q80/mxfp4_kernels.py:87-126, 242-295) on v_mfma_f32_16x16x32_bf16, and the fused
// MoE prefill layer built on it (reference server.py:1837-1936, _expert_gemms :1977-2040).
//
// Workgroup tile: 64 tokens x (4 waves x NB row blocks of 16 weight rows; NB = 3, or 4 in the SwiGLU gate_up
// kernel), K walked in k-tiles of 4 groups (128 elements).  Per k-tile the workgroup stages the 64 x 128 activation
// tile in LDS (double buffered, gathered through a row map: token-permuted rows for the MoE path), each wave loads
// its blocks' codes and scales (next k-tile in flight while the current one computes), reads its 16 A fragments
// once, dequantises each block's codes in registers with v_cvt_scalef32_pk_bf16_fp4 and runs 16 NB MFMAs.  The activations stay bf16: an FP4 or
// FP8 MFMA would need quantised activations and would no longer give the reference's results.
//
// Weight layouts (template W): the store's raw and PS4 slots (row r: 1,440 code bytes, then a raw 90-byte or PS4
// 46-byte scale row; lane (q, n) reads the 16 bytes of group 4t + q of row n, so MFMA j covers elements 8j..8j+7 of
// each lane's group) and the t950 tiles (lane (q, n) reads the 16 bytes of its tile: MFMA j covers group 4t + j,
// elements 8q..8q+7).  The A operand follows the same K mapping, so every product pairs the right x and w.
#include "common.h"
#include "t950.h"

#include <hip/hip_ext.h>

namespace na {

enum WLayout : int { kWRaw = 0, kWPs4 = 1, kWT950 = 2 };

constexpr int kPBM = 64;                 // tokens per tile
constexpr int kPKT = 128;                // K elements per k-tile
constexpr int kPApitch = kPKT * 2 + 16;  // LDS bytes per staged activation row (padded)
constexpr int kPTiles = kTTiles;         // 23 k-tiles: 22 full + groups 88, 89

// One matrix (gate_up or down) of one expert, as the kernels address it.
struct WSrc {
  const uint8_t* codes;     // raw/PS4: row 0's code bytes (row pitch 1,440); t950: block 0 of the matrix
  const uint8_t* scales;    // raw/PS4: row 0's scale row (pitch 90 or 46); t950: unused
};

// Codes (4 dwords, one per MFMA j) and E8M0 scales (one byte per MFMA j) of k-tile t for lane (q, n) of row block rblk.
template <int W>
NA_DEVICE void w_load(const WSrc& s, int rblk, int t, int lane, uint4& c, uint32_t& sc) {
  const int q = lane >> 4, n = lane & 15;
  if constexpr (W == kWT950) {
    const uint8_t* blk = s.codes + (long long)rblk * kTBlock;
    const int off = t < kTFull ? t * 1024 + 16 * lane : kTFull * 1024 + 8 * lane;   // half tile: 16 B at 8 B stride
    c = load16<true>(blk + off);
    sc = *reinterpret_cast<const uint32_t*>(blk + kTCodes + n * kTScalePitch + 4 * t);
  } else {
    const int r = rblk * 16 + n;
    const int g = min(4 * t + q, kGK - 1);           // groups 90, 91 of the last k-tile: zeroed at the use
    c = load16<true>(s.codes + (long long)r * kRowBytes + 16 * g);
    uint32_t e;
    if constexpr (W == kWRaw) {
      e = s.scales[(long long)r * kGK + g];
    } else {
      const uint8_t* row = s.scales + (long long)r * kPs4Row;
      const uint32_t nib = row[1 + (g >> 1)];
      e = row[0] + ((g & 1) ? (nib >> 4) : (nib & 15));
    }
    sc = e * 0x01010101u;                             // the same scale for the lane's 4 MFMAs
  }
}

// B operand of MFMA j from the lane's codes, with the groups beyond K zeroed.
template <int W>
NA_DEVICE bf16x8_t w_operand(const uint4& c, uint32_t sc, int t, int j, int lane) {
  const uint32_t w[4] = {c.x, c.y, c.z, c.w};
  const int q = lane >> 4;
  const int g = W == kWT950 ? 4 * t + j : 4 * t + q;
  const uint32_t code = g < kGK ? w[j] : 0u;
  return dequant8(code, e8m0_f32((sc >> (8 * j)) & 0xff));
}

// LDS byte offset, within a staged activation row, of the 8 A elements of MFMA j for lane group q.
template <int W>
NA_DEVICE int a_offset(int j, int q) {
  return W == kWT950 ? (32 * j + 8 * q) * 2 : (32 * q + 8 * j) * 2;
}

// Activation tile staging: piece p = tid + 256 i (i < 4) of the 64 x 16 pieces of 16 bytes; row = p / 16.
struct AStage {
  uint4 v[4];
};

template <typename RowPtr>
NA_DEVICE void a_load(RowPtr row_ptr, int t, int tid, AStage& a) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i, row = p >> 4, c16 = p & 15;
    const int e0 = t * kPKT + 8 * c16;               // first element of the piece
    a.v[i] = e0 < kH ? *reinterpret_cast<const uint4*>(row_ptr(row) + e0) : make_uint4(0, 0, 0, 0);
  }
}

NA_DEVICE void a_store(uint8_t* lds, int tid, const AStage& a) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = tid + 256 * i, row = p >> 4, c16 = p & 15;
    *reinterpret_cast<uint4*>(lds + row * kPApitch + 16 * c16) = a.v[i];
  }
}

// acc[tt][nb] = D of token tile tt (tokens 16 tt .. 16 tt + 15) x row block blk[nb] of this wave: lane (q, n)
// holds tokens 16 tt + 4 q + r, r = 0..3, row n of the block.  Per k-tile the wave reads its 16 A fragments from LDS
// once and feeds each to NB MFMAs per group (one per row block), so LDS traffic per MFMA falls as 1 / NB.  A wave
// without work (live = false) still stages activations and meets every barrier; its loads use block blk[0] (valid
// memory) and it runs no MFMA.  All 256 threads must call it (barriers inside).
template <int W, int NB, typename RowPtr>
NA_DEVICE void gemm_tile(const WSrc& src, const int (&blk)[NB], bool live, RowPtr row_ptr,
                         uint8_t* lds_a /* 2 x 64 x kPApitch */, f32x4_t (&acc)[4][NB]) {
  const int tid = threadIdx.x, lane = tid & 63, q = lane >> 4, n = lane & 15;
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[tt][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  AStage an;
  uint4 cn[NB];
  uint32_t sn[NB];
  a_load(row_ptr, 0, tid, an);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) w_load<W>(src, blk[nb], 0, lane, cn[nb], sn[nb]);
  a_store(lds_a, tid, an);
  __syncthreads();
  for (int t = 0; t < kPTiles; ++t) {
    uint4 c[NB];
    uint32_t sc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      c[nb] = cn[nb];
      sc[nb] = sn[nb];
    }
    const uint8_t* cur = lds_a + (t & 1) * (kPBM * kPApitch);
    if (t + 1 < kPTiles) {                           // next k-tile in flight during this one's MFMAs
      a_load(row_ptr, t + 1, tid, an);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) w_load<W>(src, blk[nb], t + 1, lane, cn[nb], sn[nb]);
    }
    bf16x8_t a[4][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        a[tt][j] = *reinterpret_cast<const bf16x8_t*>(cur + (16 * tt + n) * kPApitch + a_offset<W>(j, q));
    if (live) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const bf16x8_t b = w_operand<W>(c[nb], sc[nb], t, j, lane);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            acc[tt][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[tt][j], b, acc[tt][nb], 0, 0, 0);
        }
    }
    if (t + 1 < kPTiles) a_store(lds_a + ((t + 1) & 1) * (kPBM * kPApitch), tid, an);
    __syncthreads();
  }
}

constexpr int kPNB = 3;                  // row blocks per wave in the plain, grouped and down kernels
constexpr int kPRows = 4 * kPNB * 16;    // 192 weight rows per workgroup

template <int W>
NA_DEVICE WSrc w_src(const uint8_t* blocks, long long sb_slot, const uint8_t* scales, long long ss_slot,
                     long long slot) {
  return WSrc{blocks + slot * sb_slot, scales ? scales + slot * ss_slot : nullptr};
}

// ------------------------------------------------------------------------------- plain GEMM (mxfp4_gemm)
// out[e][m][n] = bf16(sum_k x[m][k] w_e[n][k]); grid (E * ceil(M / 64), N / 192); wave w: row blocks
// 12 y + 3 w + i.
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
        const uint16_t v = f32_to_bf16(acc[tt][nb][r]);
        const uint32_t hi = (uint32_t)__shfl_xor((int)v, 1) & 0xffff;
        if (m < m_limit && !(n & 1))
          *reinterpret_cast<uint32_t*>(out_row0 + (long long)m * pitch + 16 * blk[nb] + n) = (uint32_t)v | (hi << 16);
      }
}

template <int W>
__global__ __launch_bounds__(256) void k_mxfp4_gemm(const uint16_t* __restrict__ x, int M,
                                                    const uint8_t* __restrict__ blocks, long long sb_slot,
                                                    const uint8_t* __restrict__ scales, long long ss_slot,
                                                    const int64_t* __restrict__ slots, uint16_t* __restrict__ out,
                                                    int N) {
  __shared__ __align__(16) uint8_t lds_a[2 * kPBM * kPApitch];
  const int mt = (M + kPBM - 1) / kPBM;
  const int e = blockIdx.x / mt, m0 = (blockIdx.x - e * mt) * kPBM;
  const int wave = threadIdx.x >> 6;
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = blockIdx.y * (4 * kPNB) + kPNB * wave + i;
  const WSrc src = w_src<W>(blocks, sb_slot, scales, ss_slot, slots[e]);
  f32x4_t acc[4][kPNB];
  gemm_tile<W, kPNB>(src, blk, true, [=](int row) { return x + (long long)min(m0 + row, M - 1) * kH; }, lds_a, acc);
  store_tile(out + ((long long)e * M + m0) * N, N, acc, blk, M - m0);
}

// --------------------------------------------------------------- grouped GEMM (GroupedGemmPlan descriptors)
// tiles int64 [ntiles][5] = (x address, out address, slot, pair M, pm); rows [pm * block_m, min(M, pm * block_m +
// block_m)) of the pair, walked in 64-row sub-tiles (block_m <= 64: one).  grid (ntiles, N / 192).
template <int W>
__global__ __launch_bounds__(256) void k_mxfp4_gemm_grouped(const uint8_t* __restrict__ blocks, long long sb_slot,
                                                            const uint8_t* __restrict__ scales, long long ss_slot,
                                                            const int64_t* __restrict__ tiles, int block_m, int N) {
  __shared__ __align__(16) uint8_t lds_a[2 * kPBM * kPApitch];
  const int64_t* d = tiles + (long long)blockIdx.x * 5;
  const uint16_t* x = reinterpret_cast<const uint16_t*>(d[0]);
  uint16_t* out = reinterpret_cast<uint16_t*>(d[1]);
  const long long slot = d[2];
  const int M = (int)d[3], pm = (int)d[4];
  const int wave = threadIdx.x >> 6;
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = blockIdx.y * (4 * kPNB) + kPNB * wave + i;
  const WSrc src = w_src<W>(blocks, sb_slot, scales, ss_slot, slot);
  const int r0 = pm * block_m, r1 = min(M, r0 + block_m);
  for (int m0 = r0; m0 < r1; m0 += kPBM) {
    f32x4_t acc[4][kPNB];
    gemm_tile<W, kPNB>(src, blk, true, [=](int row) { return x + (long long)min(m0 + row, r1 - 1) * kH; }, lds_a,
                       acc);
    store_tile(out + (long long)m0 * N, N, acc, blk, r1 - m0);
  }
}

// ------------------------------------------------------------------------------------ fused MoE prefill layer
// Routing: pairs p = 4 t + k (token t, rank k); valid expert ids in [0, 128).  counts[e], then a stable order of the
// pairs by expert (order[offs[e] + i] = the i-th pair of expert e in increasing p) and a tile table
// tiles[i] = (expert, first sorted position, rows <= 64), ntiles.  Invalid ids are in no expert's list and
// contribute +0 (the combine skips them).
struct PTile {
  int e, p0, cnt, pad;
};

__global__ __launch_bounds__(256) void k_prefill_count(const int64_t* __restrict__ ids, int P,
                                                       int* __restrict__ counts) {
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

__global__ __launch_bounds__(256) void k_prefill_order(const int64_t* __restrict__ ids, int P,
                                                       const int* __restrict__ counts, int* __restrict__ order,
                                                       PTile* __restrict__ tiles, int* __restrict__ ntiles) {
  const int e = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ int wcnt[4];
  __shared__ int base_s[2];
  if (tid == 0) {
    int off = 0, tb = 0, tt = 0;
    for (int i = 0; i < 128; ++i) {
      const int c = counts[i];
      if (i < e) {
        off += c;
        tb += (c + kPBM - 1) / kPBM;
      }
      tt += (c + kPBM - 1) / kPBM;
    }
    base_s[0] = off;
    base_s[1] = tb;
    if (e == 0) *ntiles = tt;
  }
  __syncthreads();
  const int off = base_s[0], tb = base_s[1], c = counts[e];
  for (int m = tid; m * kPBM < c; m += 256) tiles[tb + m] = PTile{e, off + m * kPBM, min(kPBM, c - m * kPBM), 0};
  int run = 0;                                        // pairs of expert e before this chunk
  for (int p0 = 0; p0 < P; p0 += 256) {
    const int p = p0 + tid;
    const bool hit = p < P && ids[p] == e;
    const uint64_t bal = __ballot(hit);
    const int before = __popcll(bal & ((1ull << lane) - 1));
    if (lane == 0) wcnt[wave] = __popcll(bal);
    __syncthreads();
    int wbase = run;
    for (int w = 0; w < wave; ++w) wbase += wcnt[w];
    if (hit) order[off + wbase + before] = p;
    run += wcnt[0] + wcnt[1] + wcnt[2] + wcnt[3];
    __syncthreads();
  }
}

// gate_up + bias + clamped SwiGLU: tile i, column group a.  Wave w owns intermediate blocks jb, jb + 1
// (jb = 8 a + 2 w; columns 16 jb .. 16 jb + 31) and reads their gate rows (blocks jb, jb + 1) and up rows (blocks
// 180 + jb, 181 + jb), so the SwiGLU pairs registers of one lane.  h rows are in sorted pair order: h[p0 + m][j].
// grid (max tiles, 23); in the last column group waves 2 and 3 have no blocks.
template <int W>
__global__ __launch_bounds__(256) void k_prefill_gate_up(
    const uint16_t* __restrict__ x, const int* __restrict__ order, const PTile* __restrict__ tiles,
    const int* __restrict__ ntiles, const uint8_t* __restrict__ pool, long long slot_bytes,
    const int64_t* __restrict__ slot_tab, long long expert_base, const uint16_t* __restrict__ bias_gu,
    uint16_t* __restrict__ h, float alpha, float limit) {
  __shared__ __align__(16) uint8_t lds_a[2 * kPBM * kPApitch];
  if ((int)blockIdx.x >= *ntiles) return;
  const PTile tl = tiles[blockIdx.x];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, n = lane & 15;
  const int jb = 8 * blockIdx.y + 2 * wave;
  const bool live = jb < kTUpBlock0;
  const int jl = live ? jb : 0;
  const int blk[4] = {jl, jl + 1, kTUpBlock0 + jl, kTUpBlock0 + jl + 1};
  const long long gid = expert_base + tl.e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sb = pool + slot * slot_bytes;
  const WSrc src = W == kWT950 ? WSrc{sb, nullptr} : WSrc{sb, sb + kOffGateScales};
  f32x4_t acc[4][4];
  gemm_tile<W, 4>(src, blk, live,
                  [=](int row) { return x + (long long)(order[tl.p0 + min(row, tl.cnt - 1)] >> 2) * kH; }, lds_a,
                  acc);
  if (!live) return;
  // gu = bf16(acc) + bias (bf16 rounding of each op, as the reference's torch ops), then the clamped SwiGLU
  const uint16_t* bg = bias_gu ? bias_gu + gid * kGU : nullptr;
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    const int j = 16 * (jl + hb) + n;
    const float bgv = bg ? bf16_to_f32(bg[j]) : 0.f, buv = bg ? bf16_to_f32(bg[kI + j]) : 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * tt + 4 * q + r;
        float g = rb(acc[tt][hb][r]), u = rb(acc[tt][2 + hb][r]);
        if (bg) {
          g = rb(g + bgv);
          u = rb(u + buv);
        }
        const uint16_t hv = f32_to_bf16(swiglu_clamp_bf16(g, u, alpha, limit));
        const uint32_t hi = (uint32_t)__shfl_xor((int)hv, 1) & 0xffff;
        if (m < tl.cnt && !(n & 1))
          *reinterpret_cast<uint32_t*>(h + (long long)(tl.p0 + m) * kI + j) = (uint32_t)hv | (hi << 16);
      }
  }
}

// down + bias, x routing weight, scattered back to pair order: ys[p][n] = bf16(bf16(bf16(y) + b) * w[p]) with p the
// pair of sorted position p0 + m.  grid (max tiles, 15); wave w: row blocks 12 y + 3 w + i.
template <int W>
__global__ __launch_bounds__(256) void k_prefill_down(
    const uint16_t* __restrict__ h, const int* __restrict__ order, const PTile* __restrict__ tiles,
    const int* __restrict__ ntiles, const uint16_t* __restrict__ wts, const uint8_t* __restrict__ pool,
    long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
    const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ ys) {
  __shared__ __align__(16) uint8_t lds_a[2 * kPBM * kPApitch];
  if ((int)blockIdx.x >= *ntiles) return;
  const PTile tl = tiles[blockIdx.x];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, n = lane & 15;
  int blk[kPNB];
#pragma unroll
  for (int i = 0; i < kPNB; ++i) blk[i] = blockIdx.y * (4 * kPNB) + kPNB * wave + i;
  const long long gid = expert_base + tl.e;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* sb = pool + slot * slot_bytes;
  const WSrc src = W == kWT950 ? WSrc{sb + kTDownOff, nullptr}
                               : WSrc{sb + kOffDownCodes, sb + kOffGateScales + (long long)kGU * (W == kWRaw ? kGK : kPs4Row)};
  f32x4_t acc[4][kPNB];
  gemm_tile<W, kPNB>(src, blk, true, [=](int row) { return h + (long long)(tl.p0 + min(row, tl.cnt - 1)) * kI; },
                     lds_a, acc);
  int pr[4][4];                                       // pair of each of the lane's 16 tokens
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int r = 0; r < 4; ++r) pr[tt][r] = order[tl.p0 + min(16 * tt + 4 * q + r, tl.cnt - 1)];
#pragma unroll
  for (int nb = 0; nb < kPNB; ++nb) {
    const int col = 16 * blk[nb] + n;
    const float bd = bias_dn ? bf16_to_f32(bias_dn[gid * kH + col]) : 0.f;
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = 16 * tt + 4 * q + r;
        const int p = pr[tt][r];
        float y = rb(acc[tt][nb][r]);
        if (bias_dn) y = rb(y + bd);
        const uint16_t v = f32_to_bf16(y * bf16_to_f32(wts[p]));
        const uint32_t hi = (uint32_t)__shfl_xor((int)v, 1) & 0xffff;
        if (m < tl.cnt && !(n & 1))
          *reinterpret_cast<uint32_t*>(ys + (long long)p * kH + 16 * blk[nb] + n) = (uint32_t)v | (hi << 16);
      }
  }
}

// out[t][n] = bf16(sum_k ys[4 t + k][n]) over the valid ranks k, fp32 sum in top-k order (server.py:2340-2341).
__global__ __launch_bounds__(256) void k_prefill_combine(const uint32_t* __restrict__ ys, const int64_t* __restrict__ ids,
                                                         int T, uint32_t* __restrict__ out) {
  const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long long)T * (kH / 2)) return;
  const int t = (int)(i / (kH / 2)), c = (int)(i - (long long)t * (kH / 2));
  float a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const long long e = ids[4 * t + k];
    if (e < 0 || e >= 128) continue;
    const uint32_t v = ys[(long long)(4 * t + k) * (kH / 2) + c];
    a0 += bf16_to_f32((uint16_t)(v & 0xffff));
    a1 += bf16_to_f32((uint16_t)(v >> 16));
  }
  out[i] = (uint32_t)f32_to_bf16(a0) | ((uint32_t)f32_to_bf16(a1) << 16);
}

// Workspace of the fused prefill layer for T tokens (P = 4 T pairs): byte offsets, 256-aligned.
struct PrefillWs {
  long long counts, ntiles, order, tiles, h, ys, total;
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
  w.h = align256(w.tiles + (long long)w.max_tiles * sizeof(PTile));
  w.ys = align256(w.h + P * kI * 2);
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
  uint16_t* h = (uint16_t*)(ws + w.h);
  uint16_t* ys = (uint16_t*)(ws + w.ys);
  hipEvent_t ev[10] = {};
  if (events)
    for (int i = 0; i < 10; ++i) ev[i] = (hipEvent_t)events[i];
  const int P = 4 * T;
  launch_p(k_prefill_count, dim3(128), dim3(256), stream, ev[0], ev[1], topk_ids, P, counts);
  launch_p(k_prefill_order, dim3(128), dim3(256), stream, ev[2], ev[3], topk_ids, P, (const int*)counts, order, tiles,
           ntiles);
  const dim3 gg(w.max_tiles, (kTUpBlock0 + 7) / 8), gd(w.max_tiles, kH / kPRows), blk(256);
#define NA_PREFILL_GEMMS(W)                                                                                          \
  launch_p(k_prefill_gate_up<W>, gg, blk, stream, ev[4], ev[5], (const uint16_t*)x, (const int*)order,                \
           (const PTile*)tiles, (const int*)ntiles, (const uint8_t*)pool, slot_bytes, slot_tab, expert_base,          \
           (const uint16_t*)bias_gu, h, alpha, limit);                                                                 \
  launch_p(k_prefill_down<W>, gd, blk, stream, ev[6], ev[7], (const uint16_t*)h, (const int*)order,                   \
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
  const long long nc = (long long)T * (kH / 2);
  launch_p(k_prefill_combine, dim3((unsigned)((nc + 255) / 256)), dim3(256), stream, ev[8], ev[9],
           (const uint32_t*)ys, topk_ids, T, (uint32_t*)out);
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
