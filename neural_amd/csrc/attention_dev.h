// Device code of the GQA decode attention (64 query heads, 8 KV heads, head_dim 64, learned sinks), shared by the
// standalone kernel (attention.hip) and the fused attention block of a decode layer (core.hip).  The algorithm and
// its rounding points are described in attention.hip.
#pragma once
#include "common.h"
#include "handoff.h"

namespace na {

constexpr int kNQ = 64, kNKV = 8, kHD = 64, kRep = 8;
constexpr int kSub = 256;                          // keys per sub-chunk (4 waves x 64)
constexpr int kAttnMaxSplit = 64;
// Split-K partials of one (sequence, KV head) over its ns chunks: acc [8 rows][ns][64] (row r, chunk c at (r ns + c) 64),
// then m [ns][8] and S [ns][8]: ns x kPartFloats floats.  Chunk-minor acc rows put one lane's values of successive
// chunks 256 bytes apart, so the combine reads them at immediate offsets from a few base addresses.
constexpr int kPartFloats = kRep + kRep + kRep * kHD;
constexpr int kVPitch = kHD * 2 + 8;               // LDS bytes per V row (key): 136, 8-byte aligned
constexpr int kPPitch = kSub * 2 + 16;             // LDS bytes per P row
constexpr float kNegInf = -__builtin_huge_valf();

struct AttnLds {
  __align__(16) uint8_t v[kSub * kVPitch];         // V of the sub-chunk, bf16 [key][d] (read transposed)
  __align__(16) uint8_t p[kRep * kPPitch];         // P of the sub-chunk, bf16 [row][key]: the MFMA's A rows 8..15
                                                   // re-read rows 0..7, so D rows 8..15 repeat rows 0..7
  float mx[4][kRep];                               // per-wave row maxima
  float sm[4][kRep];                               // per-wave row sums
  float sink[kRep];                                // the KV group's sinks (written in the first pass)
  uint32_t last;                                   // split-K: this workgroup combines
};


NA_DEVICE bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }
typedef short v4i16_t __attribute__((ext_vector_type(4)));

// Key range [c0, c1) of chunk c (empty when c0 >= c1): the reference's split rule over 64-key blocks of [lo, hi].
NA_DEVICE void chunk_range(int lo, int hi, int c, int ns, int& c0, int& c1) {
  const int n = hi - lo + 1;
  const int nb = (n + 63) / 64;
  const int bps = (nb + ns - 1) / ns;
  c0 = lo + c * bps * 64;
  c1 = min(c0 + bps * 64, hi + 1);
}

// The attention of workgroup `blk` (grid B x 8 x ns).  FUSED (B = 1): q, and the K / V row of the step's own
// position, are produced earlier in the same launch as tagged words (handoff.h; word 32 r + d holds dims d and d + 32
// of QKV row r = head, q heads 0..63, K heads 64..71, V heads 72..79): the first sub-chunk's K / V loads are issued,
// then thread 0 polls the group's last word (V head h, dims 31 / 63, from the group's last QKV workgroup), then each
// lane reads its words.  The output is also written as tagged words (word i: elements 2i, 2i + 1 of the 4096).
struct AttnHandoff {
  const uint64_t* qkv;
  uint64_t* att;
  uint32_t gen;                                    // the generation word as loaded at entry (launch_tag)
  uint32_t* err;
};

// The KV group's 320 tagged QKV words (q heads 8h .. 8h + 7, then K head h, then V head h; 32 words each) read by
// the workgroup's threads (thread t: words t and 256 + t) into bf16 rows in LDS: [0, 512) the 8 q rows, [512, 576)
// K's row, [576, 640) V's row.
NA_DEVICE void tagged_group_rows(const uint64_t* qkv, int h, uint32_t gen, uint32_t* err, uint16_t* rows) {
  const int t = threadIdx.x;
  const int n = t + 256 < (kRep + 2) * 32 ? 2 : 1;
  const uint64_t* src[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int k = min(t + 256 * i, (kRep + 2) * 32 - 1);
    const int r = k >> 5, head = r < kRep ? h * kRep + r : r == kRep ? kNQ + h : kNQ + kNKV + h;
    src[i] = qkv + head * 32 + (k & 31);
  }
  uint32_t w[2];
  tag_read_at<2>(src, gen, w, err);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (i < n) {
      const int k = t + 256 * i, r = k >> 5, d = k & 31;
      rows[r * kHD + d] = (uint16_t)(w[i] & 0xffffu);
      rows[r * kHD + 32 + d] = (uint16_t)(w[i] >> 16);
    }
  }
}

// The split-K combine of one (sequence, KV head), run by the last of its ns chunk workgroups: head = the head's
// partials, orow = its 8 output rows; att (the fused block): also the output's tagged words, with tag.  Wave w
// finishes rows w and w + 4, lane l their column d = l, and the lower (upper) half of the wave stands for row w
// (w + 4): half-lane j reads chunk j's and chunk 32 + j's maximum and sum of that row.  The row's maximum m (the sink
// included) is the half's maximum; half-lane j forms its chunks' weights w_c = exp(m_c - m); then every lane takes
// the weights and sums by v_readlane (wave-uniform) and forms, in chunk order, S = exp(sink - m) + sum_c s_c w_c and
// o = sum_c acc_c[row][d] w_c for both rows over the live chunks; out = o / S.  One round of device-coherent loads
// (sc1), all in flight together (the partials were published with device-coherent stores before the count),
// through buffer resources that end where the live chunks end: a load past the end reads 0 without touching memory
// (the buffer's range check), so no load needs a branch or a clamped address.  No LDS, no barrier.
NA_DEVICE void attn_combine(const float* __restrict__ head, int ns, float sink, uint16_t* __restrict__ orow,
                            uint64_t* att, uint32_t tag) {
  const int lane = threadIdx.x & 63, jw = lane & 31;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), rh = w + 4 * (lane >> 5);
  auto rsrc = [](const float* base, int floats) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, max(floats, 0) * 4, kBufDword3);
  };
  auto ldr = [](__amdgpu_buffer_rsrc_t r, int off_bytes) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off_bytes, 0, kBufSc1));
  };
  // the head's maxima and sums; rows w and w + 4 of acc, chunks 0 .. ns - 1 and (second round) 32 .. ns - 1: a chunk
  // past ns reads 0 and moves no data
  const float* ms = head + kRep * kHD * ns;            // m [ns][8], then S [ns][8]
  const auto rm = rsrc(ms, 2 * kRep * ns);
  const float* ra = head + w * ns * kHD;
  const float* rb = head + (w + 4) * ns * kHD;
  float mc0 = ldr(rm, 4 * (jw * kRep + rh)), mc1 = ldr(rm, 4 * ((32 + jw) * kRep + rh));
  float sc0 = ldr(rm, 4 * (kRep * ns + jw * kRep + rh)), sc1 = ldr(rm, 4 * (kRep * ns + (32 + jw) * kRep + rh));
  float va[32], vb[32];
  {
    const auto r0 = rsrc(ra, ns * kHD), r1 = rsrc(rb, ns * kHD);
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      va[j] = ldr(r0, 4 * (kHD * j + lane));
      vb[j] = ldr(r1, 4 * (kHD * j + lane));
    }
  }
  mc0 = jw < ns ? mc0 : kNegInf;
  mc1 = 32 + jw < ns ? mc1 : kNegInf;
  sc0 = jw < ns ? sc0 : 0.f;
  sc1 = 32 + jw < ns ? sc1 : 0.f;
  const float mx = row16_max(fmaxf(mc0, mc1));
  const float m = fmaxf(sink, fmaxf(mx, lane_xor16(mx)));          // the half's row maximum
  const float s0 = expf(sink - m);
  const int wl[2] = {__builtin_bit_cast(int, mc0 == kNegInf ? 0.f : expf(mc0 - m)),
                     __builtin_bit_cast(int, mc1 == kNegInf ? 0.f : expf(mc1 - m))};
  const int sl[2] = {__builtin_bit_cast(int, sc0), __builtin_bit_cast(int, sc1)};
  auto lanef = [](int v, int l) { return __builtin_bit_cast(float, __builtin_amdgcn_readlane(v, l)); };
  float Sa = lanef(__builtin_bit_cast(int, s0), 0), Sb = lanef(__builtin_bit_cast(int, s0), 32), oa = 0.f, ob = 0.f;
#pragma nounroll
  for (int rd = 0; rd < 2 && 32 * rd < ns; ++rd) {     // uniform; ns <= 64
    if (rd > 0) {
      const auto r0 = rsrc(ra + 32 * kHD, (ns - 32) * kHD), r1 = rsrc(rb + 32 * kHD, (ns - 32) * kHD);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        va[j] = ldr(r0, 4 * (kHD * j + lane));
        vb[j] = ldr(r1, 4 * (kHD * j + lane));
      }
    }
    const int wr = rd ? wl[1] : wl[0], sr = rd ? sl[1] : sl[0];
#pragma unroll
    for (int j = 0; j < 32; ++j) {                     // the live chunks, in chunk order
      if (32 * rd + j < ns) {                          // uniform
        const float wa = lanef(wr, j), wb = lanef(wr, 32 + j);
        Sa = fmaf(lanef(sr, j), wa, Sa);
        Sb = fmaf(lanef(sr, 32 + j), wb, Sb);
        oa = fmaf(va[j], wa, oa);
        ob = fmaf(vb[j], wb, ob);
      }
    }
  }
  // bf16 pairs (d, d + 1): even lanes write row w's, odd lanes row w + 4's (word 32 row + d / 2 of the tagged output)
  const uint16_t ba = f32_to_bf16(oa * (1.f / Sa)), bb = f32_to_bf16(ob * (1.f / Sb));
  const uint32_t na = __builtin_bit_cast(uint32_t, dpp<0xB1>(__builtin_bit_cast(float, (uint32_t)ba)));
  const uint32_t nb = __builtin_bit_cast(uint32_t, dpp<0xB1>(__builtin_bit_cast(float, (uint32_t)bb)));
  const bool odd = lane & 1;
  const int r = odd ? w + 4 : w, d = lane & ~1;
  const uint32_t o = odd ? (nb | ((uint32_t)bb << 16)) : ((uint32_t)ba | (na << 16));
  *reinterpret_cast<uint32_t*>(orow + r * kHD + d) = o;
  if (att) tag_store(att + r * (kHD / 2) + d / 2, o, tag);
}

template <bool FUSED>
NA_DEVICE void decode_attn_body(AttnLds& L, int blk, const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc,
                                const uint16_t* __restrict__ vc, long long cache_rows, const uint16_t* __restrict__ sinks,
                                const int64_t* __restrict__ pos_p, uint16_t* __restrict__ out, float scaling,
                                int window, int ring, int ns, float* __restrict__ work,
                                uint32_t* __restrict__ counters, const AttnHandoff& hs) {
  constexpr int kCounterStride = FUSED ? kLine : 1;   // fused: each head's split counter on its own line
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, n = lane & 15;          // row group (D rows 4g..4g+3) and column of this lane
  const int c = blk % ns;
  const int bh = blk / ns;                         // b * 8 + h
  const int b = bh / kNKV, h = bh - b * kNKV;
  const long long pos = pos_p[b];
  const int hi = (int)pos;
  const int lo = window > 0 ? max(hi - window + 1, 0) : 0;
  int c0, c1;
  chunk_range(lo, hi, c, ns, c0, c1);
  const uint16_t* kbase = kc + ((long long)b * kNKV + h) * cache_rows * kHD;
  const uint16_t* vbase = vc + ((long long)b * kNKV + h) * cache_rows * kHD;

  // A operand: query rows (row n of the head for lanes n < 8, zero rows otherwise), d = 8g.. and 32 + 8g..
  const uint16_t* qrow = q + ((long long)b * kNQ + h * kRep + min(n, kRep - 1)) * kHD;
  uint4 qa0 = make_uint4(0, 0, 0, 0), qa1 = make_uint4(0, 0, 0, 0);
  // the sinks of the rows this thread finishes (constant weights), read now so that no dependent load waits at the
  // end.  FUSED (a kernel at its register limit): threads 0..7 hold one each until the first pass puts them in LDS,
  // where the finish and the combine read them (held in registers until the end, one was spilled and its reload
  // waited for every outstanding load); otherwise each thread holds its rows' sinks.
  const uint16_t* sk = sinks + h * kRep;
  uint16_t sk_own = 0;
  float sink_r[2] = {0.f, 0.f}, sink_c = 0.f;      // single chunk: rows 4 (g & 1) + 2 (g >> 1) + k; the combine's row
  if constexpr (FUSED) {
    sk_own = sk[min(tid, kRep - 1)];
  } else {
#pragma unroll
    for (int k = 0; k < 2; ++k) sink_r[k] = bf16_to_f32(sk[4 * (g & 1) + 2 * (g >> 1) + k]);
    sink_c = bf16_to_f32(sk[wave + 4 * (lane >> 5)]);
  }
  if constexpr (!FUSED) {
    qa0 = *reinterpret_cast<const uint4*>(qrow + 8 * g);
    qa1 = *reinterpret_cast<const uint4*>(qrow + 32 + 8 * g);
    if (n >= kRep) qa0 = qa1 = make_uint4(0, 0, 0, 0);
  }
  bool waited = !FUSED;

  float m_run[4], s_run[4];                        // rows 4g + r (meaningful for g < 2)
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};              // P V: D[rows 4g + r][d = 16 wave + n]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    m_run[r] = kNegInf;
    s_run[r] = 0.f;
  }

  for (int k0 = c0; k0 < c1; k0 += kSub) {
    // ---- loads: K and V rows of this wave's 64 keys (4 blocks of 16), all issued before any use
    const int kw = k0 + 64 * wave;
    uint4 kr[4][2], vr[4][2];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int key = min(kw + 16 * kb + n, hi);   // clamped: masked below, always a valid row
      long long row = ring > 0 ? key % ring : key;
      row = min(row, cache_rows - 1);
      const uint16_t* kp = kbase + row * kHD + 8 * g;
      const uint16_t* vp = vbase + row * kHD + 8 * g;
      kr[kb][0] = *reinterpret_cast<const uint4*>(kp);
      kr[kb][1] = *reinterpret_cast<const uint4*>(kp + 32);
      vr[kb][0] = *reinterpret_cast<const uint4*>(vp);
      vr[kb][1] = *reinterpret_cast<const uint4*>(vp + 32);
    }
    if (FUSED && !waited) {
      // every load above reads keys older than the step (or is replaced below); now the step's own q, K and V
      // (staged in the P rows' LDS, which the sub-chunk writes only after its next barrier)
      uint16_t* rows = reinterpret_cast<uint16_t*>(L.p);
      const uint32_t tg = launch_tag(hs.gen);
      if (tid == 0) tag_wait1(hs.qkv + (kNQ + kNKV + h) * 32 + 31, tg, hs.err);
      __syncthreads();
      tagged_group_rows(hs.qkv, h, tg, hs.err, rows);
      __syncthreads();
      waited = true;
      if (n < kRep) {
        qa0 = *reinterpret_cast<const uint4*>(rows + n * kHD + 8 * g);
        qa1 = *reinterpret_cast<const uint4*>(rows + n * kHD + 32 + 8 * g);
      }
      // the step's row, where the QKV phase stored it in the cache (a position outside a linear cache is stored
      // nowhere: the clamped row loaded above is what the cache holds)
      if (ring > 0 || hi < cache_rows) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
          if (kw + 16 * kb + n >= hi) {   // every lane clamped to hi takes the step's row, as the cache read would
            kr[kb][0] = *reinterpret_cast<const uint4*>(rows + kRep * kHD + 8 * g);
            kr[kb][1] = *reinterpret_cast<const uint4*>(rows + kRep * kHD + 32 + 8 * g);
            vr[kb][0] = *reinterpret_cast<const uint4*>(rows + (kRep + 1) * kHD + 8 * g);
            vr[kb][1] = *reinterpret_cast<const uint4*>(rows + (kRep + 1) * kHD + 32 + 8 * g);
          }
        }
      }
    }
    if (FUSED && k0 == c0 && tid < kRep) L.sink[tid] = bf16_to_f32(sk_own);   // read after the pass's first barrier
    // ---- V rows to LDS as they are (the P V step reads them transposed; stored before the scores, so that their
    // registers are free by then): lane (g, n) holds d = 8g..8g+7 and 32+8g.. of key 16 kb + n of this wave's 64
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      uint8_t* vrow = L.v + (64 * wave + 16 * kb + n) * kVPitch;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        *reinterpret_cast<uint2*>(vrow + 2 * (32 * hf + 8 * g)) = make_uint2(vr[kb][hf].x, vr[kb][hf].y);
        *reinterpret_cast<uint2*>(vrow + 2 * (32 * hf + 8 * g) + 8) = make_uint2(vr[kb][hf].z, vr[kb][hf].w);
      }
    }
    // ---- scores s = bf16(bf16(q . k) * scaling), -inf outside [k0, c1)
    float s[4][4];                                 // [block][r]
    float wmax[4] = {kNegInf, kNegInf, kNegInf, kNegInf};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      f32x4_t d = {0.f, 0.f, 0.f, 0.f};
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa0), as_bf16x8(kr[kb][0]), d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(qa1), as_bf16x8(kr[kb][1]), d, 0, 0, 0);
      const int key = kw + 16 * kb + n;
      const bool ok = key < c1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[kb][r] = ok ? rb(rb(d[r]) * scaling) : kNegInf;
        wmax[r] = fmaxf(wmax[r], s[kb][r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) wmax[r] = row16_max(wmax[r]);
    if (n == 0 && g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) L.mx[wave][4 * g + r] = wmax[r];
    }
    __syncthreads();
    // ---- sub-chunk max (exact, any order), new running max, P = bf16(exp(s - m_new)), row sums.  The scores of
    // query rows 0..7 sit in lanes g < 2; lanes g >= 2 hold the zero query rows 8..15.  Blocks 2 and 3 of the valid
    // rows move to the upper half (lane 32 + l takes lane l's, v_permlane32_swap), so that lane (g, n) exponentiates
    // blocks 2 (g >> 1) and 2 (g >> 1) + 1 of rows 4 (g & 1) + r: every lane eight valid scores.
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const auto p = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, s[kb][r]),
                                                        __builtin_bit_cast(uint32_t, s[kb + 2][r]), false, false);
        s[kb][r] = __builtin_bit_cast(float, (uint32_t)p[0]);
      }
    }
    const int hb = 2 * (g >> 1);                   // this lane's first key block
    float m_new[4], alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * (g & 1) + r;
      float mx = fmaxf(fmaxf(L.mx[0][row], L.mx[1][row]), fmaxf(L.mx[2][row], L.mx[3][row]));
      m_new[r] = fmaxf(m_run[r], mx);
      alpha[r] = m_new[r] == kNegInf ? 1.f : expf(m_run[r] - m_new[r]);
    }
    float psum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int kcol = 64 * wave + 16 * (hb + kb) + n;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = s[kb][r] == kNegInf ? 0.f : expf(s[kb][r] - m_new[r]);
        const uint16_t pb = f32_to_bf16(e);
        psum[r] += bf16_to_f32(pb);
        *reinterpret_cast<uint16_t*>(L.p + (4 * (g & 1) + r) * kPPitch + 2 * kcol) = pb;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) psum[r] = row16_sum(psum[r] + lane_xor32(psum[r]));   // exact in lane n = 0, g < 2
    if (n == 0 && g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) L.sm[wave][4 * g + r] = psum[r];
    }
    __syncthreads();
    // ---- running state: S = S alpha + sum of the 4 waves (fixed order); acc = acc alpha + P V
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * (g & 1) + r;
      const float sub = ((L.sm[0][row] + L.sm[1][row]) + L.sm[2][row]) + L.sm[3][row];
      s_run[r] = s_run[r] * alpha[r] + sub;
      m_run[r] = m_new[r];
      acc[r] *= alpha[r];
    }
    // every 32-key step of the sub-chunk, with no branch, so that all the LDS reads are in flight together: P is
    // +0 past c1 (and V holds finite cache rows there), so those steps add exact zeros to acc (never -0).  V's B
    // operand (lane (g, n): keys 32 ks + 8 g .. + 7 of dim 16 wave + n) comes from two transposing LDS reads
    // (ds_read_b64_tr_b16): in each 16-lane group, lane 4 j + q points at key k0 + j, dims 16 wave + 4 q .. + 3, and
    // lane n receives element n % 4 of lanes n / 4, 4 + n / 4, 8 + n / 4, 12 + n / 4, i.e. keys k0 .. k0 + 3 of dim
    // 16 wave + n.
    // (one LDS base per lane, the steps at constant offsets from it)
    typedef __attribute__((address_space(3))) v4i16_t lds_v4i16_t;
    lds_v4i16_t* const vt0 = reinterpret_cast<lds_v4i16_t*>(
        (__attribute__((address_space(3))) uint8_t*)(L.v) + (8 * g + ((lane & 15) >> 2)) * kVPitch +
        2 * (16 * wave + 4 * (lane & 3)));
    uint4 pa[kSub / 32], vb[kSub / 32];
#pragma unroll
    for (int ks = 0; ks < kSub / 32; ++ks) {
      pa[ks] = *reinterpret_cast<const uint4*>(L.p + (n & (kRep - 1)) * kPPitch + 2 * (32 * ks + 8 * g));
      const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt0 + 32 * ks * kVPitch / 8);
      const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(vt0 + (32 * ks + 4) * kVPitch / 8);
      vb[ks] = __builtin_bit_cast(uint4, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    }
#pragma unroll
    for (int ks = 0; ks < kSub / 32; ++ks)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pa[ks]), as_bf16x8(vb[ks]), acc, 0, 0, 0);
    __syncthreads();                               // LDS is rewritten by the next sub-chunk
  }

  // ---- finish: a single chunk writes the output; otherwise publish the partial, the last arriver combines.  FUSED:
  // the lane's indices are formed again (in this scope) from an opaque copy of the thread id, since the ones from
  // before the loop would be held across it (one was spilled, and its reload waited for every outstanding load).
  int tidf = tid;
  if constexpr (FUSED) asm volatile("" : "+v"(tidf));
  {
  const int lane = tidf & 63, wave = tidf >> 6, g = lane >> 4, n = lane & 15;
  uint16_t* orow = out + ((long long)b * kNQ + h * kRep) * kHD;
  if (ns == 1) {
    // rows 4 (g & 1) + r: lanes g < 2 finish r = 0, 1, lanes g >= 2 r = 2, 3.  The upper lanes already hold those
    // rows: their D rows 8..15 are rows 0..7 (P's rows 8..15 re-read rows 0..7), scaled by the same rows' alpha, and
    // their running maxima and sums are those rows'.
    const bool up = g >= 2;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const float av = up ? acc[2 + k] : acc[k];
      const int r = up ? 2 + k : k, row = 4 * (g & 1) + r;
      const float sink = FUSED ? L.sink[row] : sink_r[k];
      const float mr = up ? m_run[2 + k] : m_run[k], sr = up ? s_run[2 + k] : s_run[k];
      const float m = fmaxf(sink, mr);
      const float a = mr == kNegInf ? 0.f : expf(mr - m);
      const float S = expf(sink - m) + sr * a;     // the combine's formula, so one chunk == split at pos < 64
      const uint16_t o = f32_to_bf16((0.f + av * a) * (1.f / S));
      orow[row * kHD + 16 * wave + n] = o;
      if constexpr (FUSED) {                       // even lanes: (own, lane n + 1) = dims d, d + 1 of the row
        const uint32_t nb = __builtin_bit_cast(uint32_t, dpp<0xB1>(__builtin_bit_cast(float, (uint32_t)o)));
        if (!(n & 1))
          tag_store(hs.att + bh * (kRep * kHD / 2) + (row * kHD + 16 * wave + n) / 2, (uint32_t)o | (nb << 16),
                    launch_tag(hs.gen));
      }
    }
    return;
  }
  float* head = work + (long long)bh * ns * kPartFloats;
  if (g < 2) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
      __hip_atomic_store(head + (row * ns + c) * kHD + 16 * wave + n, acc[r], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (wave == 0 && n == 0) {
        float* ms = head + kRep * kHD * ns;
        __hip_atomic_store(ms + c * kRep + row, m_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(ms + kRep * ns + c * kRep + row, s_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // Publication: every wave waits until its own device-coherent stores are acknowledged, the workgroup barrier
  // orders the four waves, then one count per workgroup.  The counter's last incrementer reads the partials with
  // device-coherent loads (an acknowledged agent-scope store is visible to every agent-scope load).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t& last = L.last;
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counters + bh * kCounterStride, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (uint32_t)ns - 1;
    if (last) __hip_atomic_store(counters + bh * kCounterStride, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  // FUSED: an empty chunk ran no pass, so its LDS holds no sinks (then the sink is read here: rare, an empty chunk
  // arriving last)
  const int crow = wave + 4 * (lane >> 5);                     // the combine's row (attn_combine)
  const float sink_row = !FUSED ? sink_c : c0 < c1 ? L.sink[crow] : bf16_to_f32(sk[crow]);
  attn_combine(head, ns, sink_row, orow, FUSED ? hs.att + bh * (kRep * kHD / 2) : nullptr, FUSED ? launch_tag(hs.gen) : 0u);
  }
}

}  // namespace na
