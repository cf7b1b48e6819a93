// Decode-time MXFP4 expert products for GPT-OSS-120B on gfx950 (MI355X): bandwidth kernels.
//
// What the reference does (Triton): neural/q80/mxfp4_kernels.py:430-569 (_mxfp4_gemv / _mxfp4_gemv_masked) and the
// decode expert body server.py:508-518 (gate_up GEMV -> +bias -> clamped SwiGLU -> down GEMV -> +bias -> weighted sum).
//
// How this file does it:
//   * A wavefront streams one ROW PAIR at a time: 2 x 1440 code bytes = 180 16-byte chunks (one chunk = one group of
//     32 E2M1 codes).  Lane l loads chunks c = 64k + l (k = 0..2, c < 180) with 128-bit global loads: every load
//     instruction is a contiguous run of 16-byte chunks of one row (or of the two rows when they are adjacent).
//   * The lane -> (row of the pair, group) map is the same for every row pair, so a lane touches only 3 of the 90
//     groups of x; x sits in LDS (padded to dodge bank conflicts) or, for <= 2 tokens, in registers.
//   * Dequantisation is in registers: v_cvt_scalef32_pk_bf16_fp4 (exact) + v_dot2_f32_bf16 per code byte, then the
//     group partial is scaled by 2^(s-127) with v_ldexp_f32 (exact) and accumulated in fp32.
//   * Each row-pair's two sums are reduced across the wavefront; bf16 rounding points of the epilogues follow the
//     reference's torch op sequence (common.h).
//   * Decode routing is read on the device (top-k expert ids), so a step never syncs with the host and is
//     hipGraph-capturable: work item w of a launch is the w-th DISTINCT expert of the batch (first-appearance order);
//     it reads that expert's weights once for every token routed to it.
#include "common.h"
#include <hip/hip_ext.h>

namespace na {

constexpr int kWave = 64;
constexpr int kWaves = 4;                 // waves per workgroup
constexpr int kThreads = kWave * kWaves;
constexpr int kXG = 20;                   // LDS dwords per x group (16 used, padded: 80 B stride, conflict-free b128)
constexpr int kXTok = kGK * kXG;          // LDS dwords per staged token
constexpr int kMaxTok = 8;                // tokens per expert per launch (decode batch <= 8)
constexpr int kExpertsPerLayer = 128;

// ----------------------------------------------------------------------------------------------- scales
template <int PS4>
NA_DEVICE int load_scale(const uint8_t* srow, int g) {
  if (PS4) {
    const int base = srow[0];
    const int b = srow[1 + (g >> 1)];
    return base + ((g & 1) ? (b >> 4) : (b & 15));
  }
  return srow[g];
}

// Lane -> chunk map of a row pair (GK = 90: 180 chunks over 3 wave-wide loads).  Lanes past chunk 179 (k = 2,
// lanes 52..63) load a valid chunk (group 0 of row A) and drop its contribution with a select, so the whole load
// burst is branch-free.
struct LaneMap {
  int g[3];
  bool isB[3];
  bool valid[3];
};

NA_DEVICE LaneMap lane_map(int lane) {
  LaneMap m;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    const int c = 64 * k + lane;
    m.valid[k] = c < 2 * kGK;
    m.isB[k] = m.valid[k] && c >= kGK;
    m.g[k] = !m.valid[k] ? 0 : (m.isB[k] ? c - kGK : c);
  }
  return m;
}

// Stage token vectors [nt][2880] bf16 into LDS groups of kXG dwords.
NA_DEVICE void stage_x(uint32_t* xs, const uint16_t* const* xsrc, int nt) {
  for (int t = 0; t < nt; ++t) {
    const uint32_t* src = reinterpret_cast<const uint32_t*>(xsrc[t]);
    for (int i = threadIdx.x; i < kGK * 4; i += kThreads) {      // 16-byte pieces: 4 per group
      const int g = i >> 2, q = i & 3;
      const uint4 v = *reinterpret_cast<const uint4*>(src + g * 16 + q * 4);
      *reinterpret_cast<uint4*>(xs + t * kXTok + g * kXG + q * 4) = v;
    }
  }
}

// One row pair: A and B are two code rows (1440 B each) with their scale rows.  Loading and computing are separate
// phases so that a wave puts all of its row pairs' loads in flight before it consumes the first one.
struct PairLoad {
  uint4 c[3];
  int s[3];
};

template <int PS4>
NA_DEVICE void pair_load(const LaneMap& m, const uint8_t* cA, const uint8_t* cB, const uint8_t* sA, const uint8_t* sB,
                         PairLoad& d) {
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    d.c[k] = load16((m.isB[k] ? cB : cA) + 16 * m.g[k]);
    d.s[k] = load_scale<PS4>(m.isB[k] ? sB : sA, m.g[k]);
  }
}

// Lane-partial sums of the pair for the NT token slots: acc[t][0] (row A), acc[t][1] (row B).  Slots t >= nt hold
// duplicate inputs; their sums are computed and ignored (uniform control flow, no divergent loads).
template <int NT, bool XREG>
NA_DEVICE void pair_compute(const LaneMap& m, const PairLoad& d, const uint32_t* xs, const uint32_t (*xr)[3][16],
                            float (*acc)[2]) {
#pragma unroll
  for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = 0.f;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t* xv;
      if constexpr (XREG) xv = xr[t][k];
      else xv = xs + t * kXTok + m.g[k] * kXG;
      float p = e8m0_scale(group_dot(d.c[k], xv), d.s[k]);
      p = m.valid[k] ? p : 0.f;
      acc[t][0] += m.isB[k] ? 0.f : p;
      acc[t][1] += m.isB[k] ? p : 0.f;
    }
  }
}

// x of the lane's three groups straight from global memory (L2-resident) into registers.
template <int NT>
NA_DEVICE void load_xreg_global(const LaneMap& m, const uint16_t* const* xsrc, uint32_t (*xr)[3][16]) {
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const uint32_t* src = reinterpret_cast<const uint32_t*>(xsrc[t]) + m.g[k] * 16;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint4 v = load16(src + 4 * q);
        xr[t][k][4 * q + 0] = v.x;
        xr[t][k][4 * q + 1] = v.y;
        xr[t][k][4 * q + 2] = v.z;
        xr[t][k][4 * q + 3] = v.w;
      }
    }
}

// ----------------------------------------------------------------------------- routing of a decode batch
// Pairs are (token b, rank k) flattened as p = 4b + k.  Work item w of a launch is the w-th distinct expert of the
// batch in first-appearance order.  Expert ids outside [0, 128) are gathered into one item with status kBadExpert.
// An item's rows are its tokens (the first pair of each token routed to it); a token that lists the expert twice
// gets the result written to each of those pairs.
enum RouteStatus { kNoItem = 0, kItem = 1, kBadExpert = 2 };

struct Route {
  int expert;            // expert id within the layer
  int nt;                // tokens routed to it
  int distinct;          // distinct experts in the batch (= work items with status != kNoItem)
  int pair[kMaxTok];     // the first pair of each of those tokens, ascending (0 past nt)
  uint64_t all;          // every pair routed to it
};

// The ranks k of pair p's token that `all` routes to the same expert, as a 4-bit mask.
NA_DEVICE uint32_t token_dup_mask(uint64_t all, int p) { return (uint32_t)(all >> (p & ~3)) & 0xFu; }

NA_DEVICE int route_item(const int64_t* ids, int npairs, int item, Route& r) {
  const int lane = threadIdx.x & 63;
  int my = kExpertsPerLayer + 1;                       // lanes past the pairs: a value no pair holds
  if (lane < npairs) {
    const long long v = ids[lane];
    my = (v >= 0 && v < kExpertsPerLayer) ? (int)v : kExpertsPerLayer;
  }
  bool dup = false;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    const int o = __builtin_amdgcn_readlane(my, j);
    dup |= (j < lane) && (o == my);
  }
  const bool first = lane < npairs && !dup;
  uint64_t fm = __ballot(first);
  r.distinct = __popcll(fm);
  if (item >= r.distinct) return kNoItem;
  for (int i = 0; i < item; ++i) fm &= fm - 1;         // drop the lowest `item` set bits
  const int leader = __ffsll((long long)fm) - 1;
  r.expert = __builtin_amdgcn_readlane(my, leader);
  r.all = __ballot(lane < npairs && my == r.expert);
  uint64_t users = first_per_token(r.all);
  r.nt = 0;
#pragma unroll
  for (int t = 0; t < kMaxTok; ++t) {
    r.pair[t] = 0;
    if (users) {
      r.pair[t] = __ffsll((long long)users) - 1;
      users &= users - 1;
      r.nt = t + 1;
    }
  }
  return r.expert == kExpertsPerLayer ? kBadExpert : kItem;
}

// ======================================================================= generic GEMV (reference API mirror)
// out[e, n] = bf16(sum_k x_e[k] w_e[n, k]),  rows processed as adjacent pairs (2i, 2i+1), R pairs per wave.
// active (optional): a zero weight writes +0 and reads no weights (reference mxfp4_kernels.py:492-539).
template <int PS4, int R>
__global__ __launch_bounds__(kThreads) void k_mxfp4_gemv(
    const uint16_t* __restrict__ x, long long x_estride, const uint8_t* __restrict__ blocks, long long sb_slot,
    const uint8_t* __restrict__ scales, long long ss_slot, const int64_t* __restrict__ slots,
    const void* __restrict__ active, int active_dtype, uint16_t* __restrict__ out, int N) {
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int npairs = N / 2;
  const int p0 = blockIdx.y * (kWaves * R) + wave * R;
  bool on = true;
  if (active_dtype == 1) on = (reinterpret_cast<const uint16_t*>(active)[e] & 0x7fff) != 0;
  if (active_dtype == 2) on = reinterpret_cast<const float*>(active)[e] != 0.0f;
  if (!on) {
    for (int i = lane; i < 2 * R; i += 64)
      if (2 * p0 + i < N) out[(long long)e * N + 2 * p0 + i] = 0;
    return;
  }
  const LaneMap m = lane_map(lane);
  const long long slot = slots[e];
  const uint8_t* cb = blocks + slot * sb_slot;
  const int srow = PS4 ? kPs4Row : kGK;
  const uint8_t* sb = scales + slot * ss_slot;
  PairLoad d[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int p = min(p0 + i, npairs - 1);
    pair_load<PS4>(m, cb + (long long)(2 * p) * kRowBytes, cb + (long long)(2 * p + 1) * kRowBytes,
                   sb + (long long)(2 * p) * srow, sb + (long long)(2 * p + 1) * srow, d[i]);
  }
  const uint16_t* xe = x + (long long)e * x_estride;
  uint32_t xr[1][3][16];
  load_xreg_global<1>(m, &xe, xr);
#pragma unroll
  for (int i = 0; i < R; ++i) {
    float acc[1][2];
    pair_compute<1, true>(m, d[i], nullptr, xr, acc);
    const float a = wave_total(acc[0][0]);
    const float b = wave_total(acc[0][1]);
    const int p = p0 + i;
    if (lane == 0 && p < npairs) {
      const uint32_t packed = (uint32_t)f32_to_bf16(a) | ((uint32_t)f32_to_bf16(b) << 16);
      *reinterpret_cast<uint32_t*>(out + (long long)e * N + 2 * p) = packed;
    }
  }
}

// ================================================================ fused decode expert body (server.py:508-518)
// Kernel 1: gate_up GEMV for row pairs (gate j, up 2880 + j) of the distinct expert of this work item, for every
// token routed to it, then + bias (bf16), clamped SwiGLU (bf16 op by op) -> h[pair, j].  R row pairs per wave.
template <int NT, int PS4, int R>
__global__ __launch_bounds__(kThreads) void k_moe_gate_up(
    const uint16_t* __restrict__ x, const int64_t* __restrict__ ids, int B, const uint8_t* __restrict__ pool,
    long long slot_bytes, const int64_t* __restrict__ slot_tab, long long expert_base,
    const uint16_t* __restrict__ bias_gu, uint16_t* __restrict__ h, float alpha, float limit) {
  constexpr bool XREG = NT <= 2;
  __shared__ uint32_t xs[XREG ? 1 : NT * kXTok];
  args_at_entry(x, ids, B, pool, slot_bytes, slot_tab, expert_base, bias_gu, h, alpha, limit);
  Route r;
  if (route_item(ids, 4 * B, blockIdx.x, r) != kItem) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const LaneMap m = lane_map(lane);
  const long long gid = expert_base + r.expert;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* base = pool + slot * slot_bytes;
  const uint8_t* sb = base + kOffGateScales;
  const int srow = PS4 ? kPs4Row : kGK;
  const int j0 = blockIdx.y * (kWaves * R) + wave * R;
  PairLoad d[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int j = min(j0 + i, kI - 1);
    pair_load<PS4>(m, base + (long long)j * kRowBytes, base + (long long)(kI + j) * kRowBytes,
                   sb + (long long)j * srow, sb + (long long)(kI + j) * srow, d[i]);
  }
  const int nt = min(r.nt, NT);
  const uint16_t* xsrc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) xsrc[t] = x + (long long)(r.pair[t] >> 2) * kH;
  uint32_t xr[XREG ? NT : 1][3][16];
  if constexpr (XREG) {
    load_xreg_global<NT>(m, xsrc, xr);
  } else {
    stage_x(xs, xsrc, NT);
    __syncthreads();
  }
  const uint16_t* bg = bias_gu ? bias_gu + gid * kGU : nullptr;
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int j = j0 + i;
    float acc[NT][2];
    pair_compute<NT, XREG>(m, d[i], xs, xr, acc);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        const float g = wave_total(acc[t][0]);
        const float u = wave_total(acc[t][1]);
        if (lane == t && j < kI) {
          float gb = rb(g), ub = rb(u);
          if (bg) {
            gb = rb(gb + bf16_to_f32(bg[j]));
            ub = rb(ub + bf16_to_f32(bg[kI + j]));
          }
          const uint16_t hv = f32_to_bf16(swiglu_clamp_bf16(gb, ub, alpha, limit));
          const uint32_t dm = token_dup_mask(r.all, r.pair[t]);
          for (int k = 0; k < 4; ++k)
            if ((dm >> k) & 1) h[(long long)((r.pair[t] & ~3) + k) * kI + j] = hv;
        }
      }
    }
  }
}

// Kernel 2: down GEMV for row pairs (2i, 2i+1) from each routed token's own h, + bias, x routing weight (bf16
// product, server.py:518) -> yw[pair, n].  R row pairs per wave.
template <int NT, int PS4, int R>
__global__ __launch_bounds__(kThreads) void k_moe_down(
    const uint16_t* __restrict__ h, const int64_t* __restrict__ ids, const uint16_t* __restrict__ wts, int B,
    const uint8_t* __restrict__ pool, long long slot_bytes, const int64_t* __restrict__ slot_tab,
    long long expert_base, const uint16_t* __restrict__ bias_dn, uint16_t* __restrict__ yw) {
  constexpr bool XREG = NT <= 2;
  __shared__ uint32_t xs[XREG ? 1 : NT * kXTok];
  args_at_entry(h, ids, wts, B, pool, slot_bytes, slot_tab, expert_base, bias_dn, yw);
  Route r;
  const int st = route_item(ids, 4 * B, blockIdx.x, r);
  if (st == kNoItem) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pb0 = blockIdx.y * (kWaves * R);             // first row pair of this workgroup
  const int p0 = pb0 + wave * R;
  const int nt = min(r.nt, NT);
  if (st == kBadExpert) {                                // each of its pairs contributes +0; no weights are read
    for (int q = 0; q < 4 * B; ++q)
      if ((r.all >> q) & 1)
        for (int n = 2 * pb0 + threadIdx.x; n < min(2 * (pb0 + kWaves * R), kH); n += kThreads)
          yw[(long long)q * kH + n] = 0;
    return;
  }
  const LaneMap m = lane_map(lane);
  const long long gid = expert_base + r.expert;
  const long long slot = slot_tab ? slot_tab[gid] : gid;
  const uint8_t* base = pool + slot * slot_bytes;
  const int srow = PS4 ? kPs4Row : kGK;
  const uint8_t* cd = base + kOffDownCodes;
  const uint8_t* sd = base + kOffGateScales + (long long)kGU * srow;
  PairLoad d[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int na = 2 * min(p0 + i, kH / 2 - 1);
    pair_load<PS4>(m, cd + (long long)na * kRowBytes, cd + (long long)(na + 1) * kRowBytes,
                   sd + (long long)na * srow, sd + (long long)(na + 1) * srow, d[i]);
  }
  const uint16_t* xsrc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) xsrc[t] = h + (long long)r.pair[t] * kI;
  uint32_t xr[XREG ? NT : 1][3][16];
  if constexpr (XREG) {
    load_xreg_global<NT>(m, xsrc, xr);
  } else {
    stage_x(xs, xsrc, NT);
    __syncthreads();
  }
  const uint16_t* bd = bias_dn ? bias_dn + gid * kH : nullptr;
  float wt[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t) wt[t] = bf16_to_f32(wts[r.pair[t]]);
  const bool dups = r.all != first_per_token(r.all);    // uniform: some token lists this expert twice
#pragma unroll
  for (int i = 0; i < R; ++i) {
    const int na = 2 * (p0 + i);
    float acc[NT][2];
    pair_compute<NT, XREG>(m, d[i], xs, xr, acc);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if (t < nt) {
        const float a = wave_total(acc[t][0]);
        const float b = wave_total(acc[t][1]);
        if (lane == t && na < kH) {
          float ya = rb(a), yb = rb(b);
          if (bd) {
            ya = rb(ya + bf16_to_f32(bd[na]));
            yb = rb(yb + bf16_to_f32(bd[na + 1]));
          }
          if (!dups) {
            *reinterpret_cast<uint32_t*>(yw + (long long)r.pair[t] * kH + na) = pack_bf16x2(ya * wt[t], yb * wt[t]);
          } else {
            const uint32_t dm = token_dup_mask(r.all, r.pair[t]);
            for (int k = 0; k < 4; ++k)
              if ((dm >> k) & 1) {
                const int q = (r.pair[t] & ~3) + k;
                const float wq = bf16_to_f32(wts[q]);
                *reinterpret_cast<uint32_t*>(yw + (long long)q * kH + na) = pack_bf16x2(ya * wq, yb * wq);
              }
          }
        }
      }
    }
  }
}

// Kernel 3: out[b, n] = bf16(sum_k fp32(yw[4b + k, n])) in top-k order (server.py:518; prefill twin :2340-2341).
// Two outputs per thread.
__global__ __launch_bounds__(256) void k_moe_combine(const uint32_t* __restrict__ yw, int B,
                                                     uint32_t* __restrict__ out) {
  const int i = blockIdx.x * 256 + threadIdx.x;      // bf16 pair index
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

// ===================================================================================== router + top-k
// logits[b, e] = bf16(xn_b . Wr[e] + br[e]) (fused_core.py:431-441); the LAST workgroup to finish (atomic counter,
// no spinning) selects top-4 per token by repeated argmax (lowest index on ties) and writes softmax weights
// bf16(exp(v_i - v_0) / sum) (fused_core.py:460-486) and int64 ids.  The counter is reset by that workgroup, so the
// launch can be replayed in a graph.
constexpr int kRouterRowsPerWg = 8;   // 2 rows per wave

__global__ __launch_bounds__(kThreads) void k_router(const uint16_t* __restrict__ xn, int B,
                                                     const uint16_t* __restrict__ wr, const uint16_t* __restrict__ br,
                                                     int n_exp, float* __restrict__ logits,
                                                     unsigned int* __restrict__ counter, int64_t* __restrict__ ids_out,
                                                     uint16_t* __restrict__ w_out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int rr = 0; rr < kRouterRowsPerWg / kWaves; ++rr) {
    const int e = blockIdx.x * kRouterRowsPerWg + wave * (kRouterRowsPerWg / kWaves) + rr;
    if (e >= n_exp) break;
    const uint4* wrow = reinterpret_cast<const uint4*>(wr + (long long)e * kH);   // 360 x 16 B
    for (int b = 0; b < B; ++b) {
      const uint4* xrow = reinterpret_cast<const uint4*>(xn + (long long)b * kH);
      float a = 0.f;
      for (int i = lane; i < kH / 8; i += 64) {
        const uint4 w4 = wrow[i], x4 = xrow[i];
        a = dot2_bf16(w4.x, x4.x, a);
        a = dot2_bf16(w4.y, x4.y, a);
        a = dot2_bf16(w4.z, x4.z, a);
        a = dot2_bf16(w4.w, x4.w, a);
      }
      a = wave_sum_lane0(a);
      if (lane == 0) logits[b * n_exp + e] = rb(a + (br ? bf16_to_f32(br[e]) : 0.f));
    }
  }
  __threadfence();
  __syncthreads();
  __shared__ unsigned int last;
  if (threadIdx.x == 0) last = (atomicAdd(counter, 1u) == gridDim.x - 1);
  __syncthreads();
  if (!last) return;
  __threadfence();
  if (threadIdx.x == 0) *counter = 0u;
  if (wave != 0) return;
  for (int b = 0; b < B; ++b) {
    // each lane holds experts lane and lane + 64 (n_exp <= 128)
    const volatile float* lg = logits + b * n_exp;
    float v0 = lane < n_exp ? lg[lane] : -__builtin_inff();
    float v1 = lane + 64 < n_exp ? lg[lane + 64] : -__builtin_inff();
    float top_v[4];
    int top_i[4];
    for (int k = 0; k < 4; ++k) {
      // (value, -index) max over the wave: larger value wins, then smaller index
      float bv = v0;
      int bi = lane;
      if (v1 > bv) { bv = v1; bi = lane + 64; }
      for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off, 64);
        const int oi = __shfl_xor(bi, off, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      top_v[k] = bv;
      top_i[k] = bi;
      if (bi == lane) v0 = -__builtin_inff();
      if (bi == lane + 64) v1 = -__builtin_inff();
    }
    if (lane == 0) {
      float ex[4], s = 0.f;
      for (int k = 0; k < 4; ++k) { ex[k] = expf(top_v[k] - top_v[0]); s += ex[k]; }
      for (int k = 0; k < 4; ++k) {
        ids_out[b * 4 + k] = top_i[k];
        w_out[b * 4 + k] = f32_to_bf16(ex[k] / s);
      }
    }
  }
}

// ======================================================================================= host launchers
static int pick_nt(int B) { return B <= 1 ? 1 : B <= 2 ? 2 : B <= 4 ? 4 : 8; }

// Launch on `stream`; with a start/stop event pair the dispatch itself timestamps the kernel (hipExtLaunchKernel),
// so the measured interval is the kernel's execution whatever the host does between launches.
template <typename... KArgs, typename... Args>
static void launch(void (*kern)(KArgs...), dim3 grid, dim3 block, hipStream_t stream, hipEvent_t e0, hipEvent_t e1,
                   Args... args) {
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, e0, e1, 0, static_cast<KArgs>(args)...);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, stream, static_cast<KArgs>(args)...);
}

typedef void (*GateUpFn)(const uint16_t*, const int64_t*, int, const uint8_t*, long long, const int64_t*, long long,
                         const uint16_t*, uint16_t*, float, float);
typedef void (*DownFn)(const uint16_t*, const int64_t*, const uint16_t*, int, const uint8_t*, long long,
                       const int64_t*, long long, const uint16_t*, uint16_t*);
typedef void (*GemvFn)(const uint16_t*, long long, const uint8_t*, long long, const uint8_t*, long long,
                       const int64_t*, const void*, int, uint16_t*, int);

template <int PS4, int R>
static GateUpFn gate_up_nt(int nt) {
  switch (nt) {
    case 1: return k_moe_gate_up<1, PS4, R>;
    case 2: return k_moe_gate_up<2, PS4, R>;
    case 4: return k_moe_gate_up<4, PS4, R>;
    default: return k_moe_gate_up<8, PS4, R>;
  }
}
template <int PS4>
static GateUpFn gate_up_kernel(int nt, int r) {
  switch (r) {
    case 1: return gate_up_nt<PS4, 1>(nt);
    case 2: return gate_up_nt<PS4, 2>(nt);
    default: return gate_up_nt<PS4, 4>(nt);
  }
}
template <int PS4, int R>
static DownFn down_nt(int nt) {
  switch (nt) {
    case 1: return k_moe_down<1, PS4, R>;
    case 2: return k_moe_down<2, PS4, R>;
    case 4: return k_moe_down<4, PS4, R>;
    default: return k_moe_down<8, PS4, R>;
  }
}
template <int PS4>
static DownFn down_kernel(int nt, int r) {
  switch (r) {
    case 1: return down_nt<PS4, 1>(nt);
    case 2: return down_nt<PS4, 2>(nt);
    default: return down_nt<PS4, 4>(nt);
  }
}
template <int PS4>
static GemvFn gemv_kernel(int r) {
  switch (r) {
    case 1: return k_mxfp4_gemv<PS4, 1>;
    case 2: return k_mxfp4_gemv<PS4, 2>;
    default: return k_mxfp4_gemv<PS4, 4>;
  }
}
static bool valid_r(int r) { return r == 1 || r == 2 || r == 4; }

}  // namespace na

using namespace na;

extern "C" {

int na_mxfp4_gemv(const void* x, int per_expert_x, const void* blocks, long long sb_slot, const void* scales,
                  long long ss_slot, int packed, const int64_t* slots, int E, const void* active, int active_dtype,
                  void* out, int N, int K, int pairs_per_wave, void* const* events, hipStream_t stream) {
  if (!x || !blocks || !scales || !slots || !out || E <= 0 || N <= 0 || (N & 1) || K != kH) return kErrArgs;
  if (active_dtype < 0 || active_dtype > 2 || (active_dtype && !active)) return kErrArgs;
  if (pairs_per_wave <= 0) pairs_per_wave = 2;
  if (!valid_r(pairs_per_wave)) return kErrArgs;
  const int per_wg = kWaves * pairs_per_wave;
  dim3 grid(E, (N / 2 + per_wg - 1) / per_wg);
  const long long xs = per_expert_x ? K : 0;
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  launch(packed ? gemv_kernel<1>(pairs_per_wave) : gemv_kernel<0>(pairs_per_wave), grid, dim3(kThreads), stream,
         e0, e1, (const uint16_t*)x, xs, (const uint8_t*)blocks, sb_slot, (const uint8_t*)scales, ss_slot,
         slots, active, active_dtype, (uint16_t*)out, N);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_moe_decode(const void* x, const int64_t* topk_ids, const void* topk_w, int B, const void* pool,
                  long long slot_bytes, int packed, const int64_t* slot_tab, long long expert_base,
                  const void* bias_gu, const void* bias_dn, void* h_scratch, void* yw_scratch, void* out, float alpha,
                  float limit, int gu_pairs_per_wave, int dn_pairs_per_wave, void* const* events, hipStream_t stream) {
  if (!x || !topk_ids || !topk_w || !pool || !h_scratch || !yw_scratch || B <= 0) return kErrArgs;
  if (B > kMaxTok) return kErrTooLarge;
  if (slot_bytes < (packed ? kSlotPs4 : kSlotRaw)) return kErrArgs;
  if (gu_pairs_per_wave <= 0) gu_pairs_per_wave = 4;
  if (dn_pairs_per_wave <= 0) dn_pairs_per_wave = 2;
  if (!valid_r(gu_pairs_per_wave) || !valid_r(dn_pairs_per_wave)) return kErrArgs;
  hipEvent_t ev[6] = {};
  if (events)
    for (int i = 0; i < 6; ++i) ev[i] = (hipEvent_t)events[i];
  const int nt = pick_nt(B);
  const int items = 4 * B;
  dim3 g1(items, kI / (kWaves * gu_pairs_per_wave));
  launch(packed ? gate_up_kernel<1>(nt, gu_pairs_per_wave) : gate_up_kernel<0>(nt, gu_pairs_per_wave), g1,
         dim3(kThreads), stream, ev[0], ev[1], (const uint16_t*)x, topk_ids, B, (const uint8_t*)pool, slot_bytes,
         slot_tab, expert_base, (const uint16_t*)bias_gu, (uint16_t*)h_scratch, alpha, limit);
  dim3 g2(items, (kH / 2) / (kWaves * dn_pairs_per_wave));
  launch(packed ? down_kernel<1>(nt, dn_pairs_per_wave) : down_kernel<0>(nt, dn_pairs_per_wave), g2, dim3(kThreads),
         stream, ev[2], ev[3], (const uint16_t*)h_scratch, topk_ids, (const uint16_t*)topk_w, B,
         (const uint8_t*)pool, slot_bytes, slot_tab, expert_base, (const uint16_t*)bias_dn, (uint16_t*)yw_scratch);
  if (out)
    launch(k_moe_combine, dim3((B * kH / 2 + 255) / 256), dim3(256), stream, ev[4], ev[5],
           (const uint32_t*)yw_scratch, B, (uint32_t*)out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_router_topk(const void* xn, int B, const void* w_router, const void* b_router, int n_exp, float* logits,
                   unsigned int* counter, int64_t* ids_out, void* w_out, hipStream_t stream) {
  if (!xn || !w_router || !logits || !counter || !ids_out || !w_out || B <= 0 || n_exp <= 4 || n_exp > 128)
    return kErrArgs;
  dim3 grid((n_exp + kRouterRowsPerWg - 1) / kRouterRowsPerWg);
  launch(k_router, grid, dim3(kThreads), stream, nullptr, nullptr, (const uint16_t*)xn, B, (const uint16_t*)w_router,
         (const uint16_t*)b_router, n_exp, logits, counter, ids_out, (uint16_t*)w_out);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
