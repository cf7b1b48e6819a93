// Prompt-processing (prefill) attention with learned sinks, causal + optional sliding window, GQA 64 query / 8 KV
// heads of 64, on gfx950.  The computation of reference fused_core.py:684-759 (k_prefill_attn): per query head and
// query position qp = p0 + t, keys j <= qp (and j > qp - window on sliding layers) of the cache; scores
// s = (q . k) * scaling in fp32; online softmax whose running state starts at (m = sink, l = 1), so the sink joins
// the denominator; P is rounded to bf16 for the P V product, the row sums use the unrounded P; o = bf16(acc / l).
//
// Work layout: one workgroup of 8 waves per (16-token query block, KV head h), two workgroups per CU; wave w is
// query head 8 h + w, so the eight query heads that share a KV head read each K / V tile from LDS, where it is
// staged once.  Tiles of 64 keys walk [lo, hi) with lo = max(first query - window + 1, 0) rounded down to 64 (0 on
// full layers) and hi = one past the block's last query; the next tile's global loads are in flight while the
// current tile is computed (two LDS buffers, one barrier per tile).  Tiles below the block's first query (and inside
// the window of its last) need no mask and take a path without one; the O rescale is skipped when no column's
// running maximum moved.  (Measured on MI355X: 32-token blocks at one workgroup per CU equal on causal layers and
// slower on sliding ones; 128-key tiles slower.)  Both products run on v_mfma_f32_16x16x32_bf16 with the queries as the columns:
//   S^T [key][query] = K [key][d] . Q^T [d][query]      (A = K rows from LDS, B = Q held in registers)
//   O^T [d][query]  += V^T [d][key] . P^T [key][query]   (A = V^T from LDS, B = P^T straight from the S^T registers)
// A lane then owns one query column in every tile, so the softmax state of that query (running max, the alpha
// rescale of O^T) stays in the lane; the only cross-lane steps are the max over the 4 lanes that share a column and
// the final row sum.  The k index of the P V product is a permutation of the 32 keys of a step (lane group g holds
// keys 4g..4g+3 and 16+4g..16+4g+3), the same permutation on both operands.
//
// Key sources: linear cache [NKV][cache_rows][64] holding every position below p0 + T, or (ring > 0, sliding
// layers) a rolling cache [NKV][ring][64] for keys j < p0 (row j % ring) plus the block's own K / V rows
// [T][NKV][64] (strided) for j >= p0.  Both modes run the same tiles in the same order with the same arithmetic, so
// their outputs are bit-identical when the caches hold the same values.  Keys past hi - 1 in the last tile are read
// from row hi - 1 and masked; a ring slot holding a position that no query can see is masked (its contents must be
// finite, as in the reference).
#include "common.h"

#include <hip/hip_ext.h>

#include <type_traits>

namespace na {

namespace pfa {

constexpr int kNQ = 64, kNKV = 8, kHD = 64, kRep = 8;
constexpr int kKPitch = kHD * 2 + 16;      // LDS bytes per K row: 144 (16-byte reads of 8 rows hit distinct banks)
constexpr int kVPitch = kHD * 2 + 16;      // LDS bytes per V row: 144 (read transposed, ds_read_b64_tr_b16)
typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
constexpr int kThreads = 512;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

template <int KEYS>
struct Lds {
  __align__(16) uint8_t k[2][KEYS * kKPitch];
  __align__(16) uint8_t v[2][KEYS * kVPitch];
};

NA_DEVICE bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

struct KeySrc {
  const uint16_t* kc;
  const uint16_t* vc;
  const uint16_t* kn;
  const uint16_t* vn;
  long long cache_rows, sk_t, sk_h, sv_t, sv_h, p0;
  int ring, h;

  // Row of key position j (0 <= j < p0 + T) for head h.
  NA_DEVICE const uint16_t* krow(long long j) const {
    if (ring > 0) {
      if (j < p0) return kc + ((long long)h * cache_rows + j % ring) * kHD;
      return kn + (j - p0) * sk_t + (long long)h * sk_h;
    }
    return kc + ((long long)h * cache_rows + j) * kHD;
  }
  NA_DEVICE const uint16_t* vrow(long long j) const {
    if (ring > 0) {
      if (j < p0) return vc + ((long long)h * cache_rows + j % ring) * kHD;
      return vn + (j - p0) * sv_t + (long long)h * sv_h;
    }
    return vc + ((long long)h * cache_rows + j) * kHD;
  }
};

// QT query tiles of 16 per wave: 16 * QT tokens per workgroup; KEYS keys per tile (64 or 128).
template <int QT, int KEYS>
__global__ __launch_bounds__(kThreads, QT == 1 ? 4 : 2) void k_prefill_attn(
    const uint16_t* __restrict__ q, KeySrc src, const uint16_t* __restrict__ sinks, uint16_t* __restrict__ out,
    int T, float scaling, int window) {
  constexpr int kQB = 16 * QT, kKeys = KEYS, KT = KEYS / 16, KS = KEYS / 32, KP = KEYS / 64;
  __shared__ Lds<KEYS> L;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, n = lane & 15;
  const int nqb = (T + kQB - 1) / kQB;
  const int h = blockIdx.x % kNKV;                    // consecutive workgroups: consecutive heads
  const int qb = nqb - 1 - (int)(blockIdx.x / kNKV);  // longest key ranges first
  src.h = h;
  const int hq = h * kRep + wave;
  const int q0 = qb * kQB;                            // block-relative first token
  const int qpos0 = (int)src.p0 + q0;                 // positions fit 31 bits (the host checks p0 + T)
  const int hi = (int)src.p0 + min(q0 + kQB, T);      // one past the last key any query of the block sees
  const int qlast = hi - 1;
  int lo = window > 0 ? qpos0 - window + 1 : 0;
  lo = lo < 0 ? 0 : (lo / kKeys) * kKeys;
  const int nt = (hi - lo + kKeys - 1) / kKeys;

  // Q^T as the B operand: lane (n, g) holds query q0 + 16 qt + n, dims 8g.. (step 0) and 32 + 8g.. (step 1).
  uint4 qf[QT][2];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    const int t = min(q0 + 16 * qt + n, T - 1);
    const uint16_t* qr = q + ((long long)t * kNQ + hq) * kHD;
    qf[qt][0] = *reinterpret_cast<const uint4*>(qr + 8 * g);
    qf[qt][1] = *reinterpret_cast<const uint4*>(qr + 32 + 8 * g);
  }
  // scores in the log2 domain: exp(s scaling - m) = exp2(s scaling log2e - m'), formed as exp2(fma(s, sl2, -m'));
  // the maximum is taken over the raw scores (s -> s sl2 is monotone, so max(s) sl2 = max(s sl2))
  const float sl2 = scaling * kLog2e;
  const float sink2 = bf16_to_f32(sinks[hq]) * kLog2e;
  float m[QT], l[QT];
  f32x4_t acc[4][QT];
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    m[qt] = sink2;
    l[qt] = g == 0 ? 1.f : 0.f;                       // the sink's exp(sink - m) = 1, counted once per column
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) acc[dt][qt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }

  // Staging, per 64 keys of a tile: K row key tid / 8, dims 8 (tid % 8) (a wave reads 8 whole rows); V key
  // tid % 64, dims 8 (tid / 64), stored as it is (the P V step reads it transposed).  Tile it + 1's loads are in
  // flight over tile it's work (two LDS buffers, one barrier per tile).  Every global load and LDS store is
  // unconditional: rows past hi - 1 read row hi - 1, and the store of tile it + 1 goes to buffer (it + 1) & 1, which
  // no wave reads in iteration it (its last reads were in iteration it - 1, before that iteration's barrier).
  const int kk = tid >> 3, kd = tid & 7;
  const int vk = tid & 63, vd = tid >> 6;
  uint4 kreg[KP], vreg[KP];
  auto load_k = [&](int s0) {
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int jk = s0 + 64 * p + kk;
      kreg[p] = *reinterpret_cast<const uint4*>(src.krow(jk < hi ? jk : hi - 1) + 8 * kd);
    }
  };
  auto load_v = [&](int s0) {
#pragma unroll
    for (int p = 0; p < KP; ++p) {
      const int jv = s0 + 64 * p + vk;
      vreg[p] = *reinterpret_cast<const uint4*>(src.vrow(jv < hi ? jv : hi - 1) + 8 * vd);
    }
  };
  auto store_k = [&](int buf) {
#pragma unroll
    for (int p = 0; p < KP; ++p) *reinterpret_cast<uint4*>(L.k[buf] + (64 * p + kk) * kKPitch + 16 * kd) = kreg[p];
  };
  auto store_v = [&](int buf) {
#pragma unroll
    for (int p = 0; p < KP; ++p) *reinterpret_cast<uint4*>(L.v[buf] + (64 * p + vk) * kVPitch + 16 * vd) = vreg[p];
  };

  // S^T = K Q^T of the tile in K buffer buf: tile (kt, qt), lane holds keys 16 kt + 4 g + r of query column n
  auto scores = [&](int buf, float (&s)[KT][QT][4]) {
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const uint8_t* kr = L.k[buf] + (16 * kt + n) * kKPitch + 16 * g;
      const uint4 ka0 = *reinterpret_cast<const uint4*>(kr);
      const uint4 ka1 = *reinterpret_cast<const uint4*>(kr + 64);
#pragma unroll
      for (int qt = 0; qt < QT; ++qt) {
        f32x4_t d = {0.f, 0.f, 0.f, 0.f};
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka0), as_bf16x8(qf[qt][0]), d, 0, 0, 0);
        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(ka1), as_bf16x8(qf[qt][1]), d, 0, 0, 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) s[kt][qt][r] = d[r];
      }
    }
  };

  // One tile (keys s0 .., buffer buf): S^T, the online softmax, then O^T += V^T P^T.  MASK = false: every key of
  // the tile is visible to every query of the block (below the first query, and inside the window of the last), so
  // no key is masked.
  auto tile = [&](auto mask_c, int buf, int s0) {
    constexpr bool MASK = decltype(mask_c)::value;
    float s[KT][QT][4];
    scores(buf, s);
    bool moved = false;
    float alpha[QT], mnew[QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      const int qp = qpos0 + 16 * qt + n;
      float mx = kNegInf;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (MASK) {
            const int j = s0 + 16 * kt + 4 * g + r;
            bool ok = j <= qp && j < hi;
            if (window > 0) ok = ok && j > qp - window;
            s[kt][qt][r] = ok ? s[kt][qt][r] : kNegInf;
          }
          mx = fmaxf(mx, s[kt][qt][r]);
        }
      }
      mx = fmaxf(mx, lane_xor16(mx));                 // the 4 lanes of column n (VALU lane swaps, no LDS)
      mx = fmaxf(mx, lane_xor32(mx));
      mnew[qt] = fmaxf(m[qt], mx * sl2);              // finite: m starts at the sink
      alpha[qt] = __builtin_amdgcn_exp2f(m[qt] - mnew[qt]);
      moved |= mnew[qt] != m[qt];
      m[qt] = mnew[qt];
    }
    // O^T *= alpha, skipped when no column of the wave moved its maximum (then every alpha is exactly 1)
    if (__builtin_amdgcn_ballot_w64(moved)) {
#pragma unroll
      for (int qt = 0; qt < QT; ++qt)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) acc[dt][qt] *= alpha[qt];
    }
    // P^T fragments: P = exp2(s sl2 - m') rounded to bf16; the row sums take the unrounded values
    uint4 pf[KS][QT];
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      float ls = l[qt] * alpha[qt];
      uint32_t pk[KT][2];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) {
        float e[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          e[r] = __builtin_amdgcn_exp2f(fmaf(s[kt][qt][r], sl2, -mnew[qt]));   // exp2(-inf) = +0 for masked keys
          ls += e[r];
        }
        pk[kt][0] = pack_bf16x2(e[0], e[1]);
        pk[kt][1] = pack_bf16x2(e[2], e[3]);
      }
      l[qt] = ls;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)                 // step ks: keys 32 ks + 4g.., 32 ks + 16 + 4g..
        pf[ks][qt] = make_uint4(pk[2 * ks][0], pk[2 * ks][1], pk[2 * ks + 1][0], pk[2 * ks + 1][1]);
    }
    // ---- O^T += V^T P^T over the 32-key steps.  V^T's A operand (lane (g, n): dim 16 dt + n, keys 32 ks + 4 g ..
    // + 3 and 32 ks + 16 + 4 g .. + 3) comes from two transposing LDS reads (ds_read_b64_tr_b16): in each 16-lane
    // group, lane 4 j + q points at key k0 + j, dims 16 dt + 4 q .. + 3, and lane n receives element n % 4 of lanes
    // n / 4, 4 + n / 4, 8 + n / 4, 12 + n / 4, i.e. keys k0 .. k0 + 3 of dim 16 dt + n.  One base per lane, every
    // (ks, dt) at a constant offset from it.
    lds_v4i16_t* const vt0 = reinterpret_cast<lds_v4i16_t*>(
        (__attribute__((address_space(3))) uint8_t*)(L.v[buf]) + (4 * g + ((lane & 15) >> 2)) * kVPitch +
        8 * (lane & 3));
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt0 + (32 * ks * kVPitch + 32 * dt) / 8);
        const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt0 + ((32 * ks + 16) * kVPitch + 32 * dt) / 8);
        const uint4 va = __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int qt = 0; qt < QT; ++qt)
          acc[dt][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(va), as_bf16x8(pf[ks][qt]), acc[dt][qt], 0,
                                                                 0, 0);
      }
    }
  };

  // Tiles [ia, ib) need no mask: s0 + kKeys <= qpos0 (it < nA) and, on sliding layers, s0 > qlast - window
  // (it >= nB).  Masking is exact for every tile, so the split only has to leave no masked key unmasked.
  const int nA = (qpos0 - lo) / kKeys;                // qpos0 >= lo
  int nB = 0;
  if (window > 0) {
    const int x = qlast - window - lo;
    nB = x < 0 ? 0 : x / kKeys + 1;
  }
  const int ia = min(nA, nB), ib = nA;

  load_k(lo);
  load_v(lo);
  store_k(0);
  store_v(0);
  __syncthreads();
  // the masked and unmasked tiles as separate loops (one code path per loop, no copies of the accumulators between
  // two paths at every tile)
  int it = 0;
  auto run = [&](auto mask_c, int end) {
    for (; it < end; ++it) {
      const int s0 = lo + it * kKeys, buf = it & 1;
      load_k(s0 + kKeys);
      load_v(s0 + kKeys);
      tile(mask_c, buf, s0);
      store_k(buf ^ 1);
      store_v(buf ^ 1);
      __syncthreads();
    }
  };
  run(std::true_type{}, ia);
  run(std::false_type{}, ib);
  run(std::true_type{}, nt);

  // ---- o = acc / l; lane holds dims 16 dt + 4 g + r of query column n
#pragma unroll
  for (int qt = 0; qt < QT; ++qt) {
    float lt = l[qt];
    lt += __shfl_xor(lt, 16);
    lt += __shfl_xor(lt, 32);
    const int t = q0 + 16 * qt + n;
    if (t < T) {
      const float inv = 1.f / lt;
      uint16_t* orow = out + ((long long)t * kNQ + hq) * kHD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const uint2 o = make_uint2(pack_bf16x2(acc[dt][qt][0] * inv, acc[dt][qt][1] * inv),
                                   pack_bf16x2(acc[dt][qt][2] * inv, acc[dt][qt][3] * inv));
        *reinterpret_cast<uint2*>(orow + 16 * dt + 4 * g) = o;
      }
    }
  }
}

// Ring write (reference fused_core.py:787-800): the last min(T, ring) positions of a block, K / V rows [T][NKV][64]
// with strides, into ring slots position % ring of [NKV][ring][64].  One thread per 16 bytes.
__global__ __launch_bounds__(256) void k_ring_write(uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int ring,
                                                    const uint16_t* __restrict__ kn, const uint16_t* __restrict__ vn,
                                                    long long sk_t, long long sk_h, long long sv_t, long long sv_h,
                                                    long long p0, int T) {
  const int n = min(T, ring);
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // over n x NKV x 8 pieces
  if (i >= (long long)n * kNKV * 8) return;
  const int piece = (int)(i & 7);
  const int hh = (int)((i >> 3) % kNKV);
  const int r = (int)(i / (8 * kNKV));
  const int t = T - n + r;                            // block-relative position
  const long long slot = (p0 + t) % ring;
  const long long dst = ((long long)hh * ring + slot) * kHD + 8 * piece;
  *reinterpret_cast<uint4*>(kc + dst) = *reinterpret_cast<const uint4*>(kn + t * sk_t + hh * sk_h + 8 * piece);
  *reinterpret_cast<uint4*>(vc + dst) = *reinterpret_cast<const uint4*>(vn + t * sv_t + hh * sv_h + 8 * piece);
}

}  // namespace pfa

}  // namespace na

using namespace na;
using namespace na::pfa;

extern "C" {

int na_prefill_attention(const void* q, const void* kc, const void* vc, long long cache_rows, const void* k_new,
                         const void* v_new, long long sk_t, long long sk_h, long long sv_t, long long sv_h,
                         const void* sinks, void* out, long long p0, int T, float scaling, int window, int ring,
                         void* const* events, hipStream_t stream) {
  if (T < 0 || p0 < 0 || window < 0 || ring < 0 || cache_rows <= 0) return kErrArgs;
  if (p0 + T >= (1LL << 31)) return kErrArgs;           // positions are 32-bit in the kernel
  if (T == 0) return kOk;                             // an empty prompt: nothing to read or write
  if (!q || !kc || !vc || !sinks || !out) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15)
    return kErrArgs;
  if (reinterpret_cast<uintptr_t>(out) & 7) return kErrArgs;
  if (ring > 0) {
    if (window <= 0 || ring < window || cache_rows != ring || !k_new || !v_new) return kErrArgs;
    if ((reinterpret_cast<uintptr_t>(k_new) | reinterpret_cast<uintptr_t>(v_new)) & 15) return kErrArgs;
    if (sk_t < 0 || sk_h < 0 || sv_t < 0 || sv_h < 0 || ((sk_t | sk_h | sv_t | sv_h) & 7)) return kErrArgs;
  } else if (p0 + T > cache_rows) {
    return kErrArgs;
  }
  KeySrc src{(const uint16_t*)kc, (const uint16_t*)vc, (const uint16_t*)k_new, (const uint16_t*)v_new,
             cache_rows, sk_t, sk_h, sv_t, sv_h, p0, ring, 0};
  constexpr int QT = 1;                               // 16 tokens per workgroup, two workgroups per CU
  const int qb = 16 * QT;
  const dim3 grid((unsigned)(((long long)T + qb - 1) / qb * kNKV)), block(kThreads);
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  auto kern = k_prefill_attn<QT, 64>;
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, grid, block, 0, stream, e0, e1, 0, (const uint16_t*)q, src, (const uint16_t*)sinks,
                          (uint16_t*)out, T, scaling, window);
  else
    hipLaunchKernelGGL(kern, grid, block, 0, stream, (const uint16_t*)q, src, (const uint16_t*)sinks, (uint16_t*)out,
                       T, scaling, window);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_ring_write(void* kc, void* vc, int ring, const void* k_new, const void* v_new, long long sk_t, long long sk_h,
                  long long sv_t, long long sv_h, long long p0, int T, hipStream_t stream) {
  if (ring <= 0 || T < 0 || p0 < 0) return kErrArgs;
  if (T == 0) return kOk;
  if (!kc || !vc || !k_new || !v_new) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc) | reinterpret_cast<uintptr_t>(k_new) |
       reinterpret_cast<uintptr_t>(v_new)) & 15)
    return kErrArgs;
  if (sk_t < 0 || sk_h < 0 || sv_t < 0 || sv_h < 0 || ((sk_t | sk_h | sv_t | sv_h) & 7)) return kErrArgs;
  const long long pieces = (long long)(T < ring ? T : ring) * kNKV * 8;
  hipLaunchKernelGGL(k_ring_write, dim3((unsigned)((pieces + 255) / 256)), dim3(256), 0, stream, (uint16_t*)kc,
                     (uint16_t*)vc, ring, (const uint16_t*)k_new, (const uint16_t*)v_new, sk_t, sk_h, sv_t, sv_h, p0,
                     T);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
