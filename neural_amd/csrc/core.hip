// Dense decode core of GPT-OSS-120B on gfx950 (one token per step): per layer the fused residual + input RMSNorm +
// QKV GEMV + bias + RoPE + K/V cache write (reference fused_core.py:72-142, k_qkv), o_proj + bias + residual
// (:401-414, k_oproj), post-attention RMSNorm + router GEMV + top-4 + softmax (:417-502, k_router / k_topk), and the
// tail: residual + final RMSNorm, lm_head GEMV and argmax (server.py:521-525, t_body); plus the embedding lookup.
//
// Rounding points (the reference's): the residual x = bf16(mid + g) (g = the previous layer's expert output); the
// RMSNorm factor r = rsqrt(sum x^2 / H + eps) in fp32; the normed activation hc = bf16(w * (x * r)); GEMV rows
// bf16(fp32 dot + bias); RoPE cos/sin = bf16(cos(inv_freq[d] pos) * att_scale), o1 = bf16(bf16(ya cs) - bf16(yb sn)),
// o2 = bf16(bf16(yb cs) + bf16(ya sn)); o_proj mid = bf16(x + bf16(dot + bo)); router logits bf16(dot + br), top-4 by
// repeated argmax (lowest index on ties), weights bf16(exp(v_j - v_0) / sum); logits of the tail bf16(dot), argmax
// = the first index of the maximum.
//
// GEMV layout: a workgroup of 256 threads computes 16 weight rows; thread (r = tid / 16, j = tid % 16) streams row
// r's 16-byte chunks j, j + 16, ... (all issued before the first use) against the normed activation staged in LDS,
// and the 16 lanes of a row group sum with xor shuffles.
#include "attention_dev.h"
#include "common.h"
#include "handoff.h"
#include "topk.h"

#include <hip/hip_ext.h>

namespace na {

constexpr int kHq = 64 * 64;             // query width (NQ x HD)
constexpr int kQkvRows = (64 + 2 * 8) * 64;   // 5120
constexpr int kNE = 128;

// Sum over the TPR lanes of a row group (TPR = 16, 32 or 64, groups aligned to TPR lanes), exact in the group's first
// lane (the xor butterfly over offsets 1, 2, 4, .., TPR / 2; common.h): the only lane whose result is used.
template <int TPR>
NA_DEVICE float sum_group(float v) {
  static_assert(TPR == 16 || TPR == 32 || TPR == 64, "row groups of 16, 32 or 64 lanes");
  v = row16_sum(v);
  if constexpr (TPR >= 32) v += lane_xor16(v);
  if constexpr (TPR >= 64) v += lane_xor32(v);
  return v;
}

// dot of 8 bf16 weights with 8 bf16 activations, fp32 accumulation
NA_DEVICE float dot8(uint4 w, uint4 x, float a) {
  a = dot2_bf16(w.x, x.x, a);
  a = dot2_bf16(w.y, x.y, a);
  a = dot2_bf16(w.z, x.z, a);
  return dot2_bf16(w.w, x.w, a);
}

// One weight row's 16-byte chunks j, j + TPR, ... (thread j of the row's TPR threads) held in registers: issued before
// the activation is ready so that the weight stream overlaps the normalisation; dot() then sums them against the
// LDS-staged activation hc and every lane of the row group returns the row's total.
template <int K, int TPR>
struct RowChunks {
  static constexpr int NCH = K / 8, IT = (NCH + TPR - 1) / TPR;
  uint4 w[IT];
  NA_DEVICE void load(const uint16_t* __restrict__ wrow, int j) {
#pragma unroll
    for (int i = 0; i < IT; ++i) w[i] = load16<true>(wrow + 8 * min(j + TPR * i, NCH - 1));
  }
  // the row's dot product, in the row group's first lane (j == 0; the other lanes hold partial sums)
  NA_DEVICE float dot(const uint16_t* hc, int j) const {
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = j + TPR * i;
      if (c < NCH) a = dot8(w[i], *reinterpret_cast<const uint4*>(hc + 8 * c), a);
    }
    return sum_group<TPR>(a);
  }
};

// Threads per weight row of each GEMV (256 / TPR rows per workgroup).
#ifndef NA_QKV_TPR
#define NA_QKV_TPR 32
#endif
#ifndef NA_OPROJ_TPR
#define NA_OPROJ_TPR 32
#endif
#ifndef NA_ROUTER_TPR
#define NA_ROUTER_TPR 64
#endif
#ifndef NA_LM_TPR
#define NA_LM_TPR 16
#endif
constexpr int kQkvTpr = NA_QKV_TPR, kOprojTpr = NA_OPROJ_TPR, kRouterTpr = NA_ROUTER_TPR, kLmTpr = NA_LM_TPR;

// Inputs of the residual + RMSNorm stage, loaded first (before a kernel's weight stream, so that waiting for them
// does not wait for the weights): thread t holds chunks t and t + 256 (8 values each) of mid, of the expert outputs
// g (bf16) and c (fp32, optional: the experts computed elsewhere, reference fused_core.py:72-79) and of the norm
// weight.
struct NormIn {
  uint4 m[2], g[2], w[2], c[2][2];
  // HAS_C = false: c is absent (cp ignored), so its registers need not be held
  template <bool HAS_C = true>
  NA_DEVICE void load(const uint16_t* __restrict__ mid, const uint16_t* __restrict__ gp, const float* __restrict__ cp,
                      const uint16_t* __restrict__ wp) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int ch = min((int)threadIdx.x + 256 * i, kH / 8 - 1);
      m[i] = *reinterpret_cast<const uint4*>(mid + 8 * ch);
      w[i] = *reinterpret_cast<const uint4*>(wp + 8 * ch);
      // absent inputs are not read (uniform branches: every workgroup of a launch reads the same inputs, and these
      // requests queue in the L2 with the launch's weight stream); their values are unused
      g[i] = c[i][0] = c[i][1] = make_uint4(0, 0, 0, 0);
      if (gp) g[i] = *reinterpret_cast<const uint4*>(gp + 8 * ch);
      if (HAS_C && cp) {
        c[i][0] = *reinterpret_cast<const uint4*>(cp + 8 * ch);
        c[i][1] = *reinterpret_cast<const uint4*>(cp + 8 * ch + 4);
      }
    }
  }
};

NA_DEVICE float half_at(const uint4& v, int e) {
  const uint32_t wd = e < 2 ? v.x : e < 4 ? v.y : e < 6 ? v.z : v.w;
  return bf16_to_f32((uint16_t)(wd >> (16 * (e & 1))));
}

NA_DEVICE float float_at(const uint4 (&v)[2], int e) {
  const uint4& q = v[e >> 2];
  const int k = e & 3;
  return __uint_as_float(k == 0 ? q.x : k == 1 ? q.y : k == 2 ? q.z : q.w);
}

// x = mid, or bf16(mid + bf16(g + bf16(c))) when g is given; r = rsqrt(sum x^2 / H + eps); hc = bf16(w * (x * r)) into
// LDS (all H values); workgroup 0 also writes x to xbuf when given.  All 256 threads call it; ends with a barrier.
NA_DEVICE void norm_finish(const NormIn& in, bool has_g, bool has_c, float eps, uint16_t* hc,
                           uint16_t* __restrict__ xbuf) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  float xv[2][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float x = half_at(in.m[i], e);
      if (has_g) {
        const float c = has_c ? rb(float_at(in.c[i], e)) : 0.f;
        x = rb(x + rb(half_at(in.g[i], e) + c));
      }
      xv[i][e] = x;
      if (tid + 256 * i < kH / 8) ss += x * x;
    }
  }
  ss = wave_sum_lane0(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float var = ((red[0] + red[1]) + (red[2] + red[3])) * (1.0f / kH);
  const float r = rsqrtf(var + eps);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ch = tid + 256 * i;
    if (ch < kH / 8) {
      uint32_t o[4], xo[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        o[e >> 1] = pack_bf16x2(half_at(in.w[i], e) * (xv[i][e] * r), half_at(in.w[i], e + 1) * (xv[i][e + 1] * r));
        xo[e >> 1] = pack_bf16x2(xv[i][e], xv[i][e + 1]);
      }
      *reinterpret_cast<uint4*>(hc + 8 * ch) = make_uint4(o[0], o[1], o[2], o[3]);
      if (xbuf && blockIdx.x == 0) *reinterpret_cast<uint4*>(xbuf + 8 * ch) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
    }
  }
  __syncthreads();
}

// A bf16 vector of N values (N / 8 chunks, at most 512) copied to LDS: load() first, store() after the weights.
template <int N>
struct VecIn {
  static constexpr int NCH = N / 8;
  uint4 v[2];
  NA_DEVICE void load(const uint16_t* __restrict__ p) {
#pragma unroll
    for (int i = 0; i < 2; ++i) v[i] = *reinterpret_cast<const uint4*>(p + 8 * min((int)threadIdx.x + 256 * i, NCH - 1));
  }
  NA_DEVICE void store(uint16_t* lds) const {
#pragma unroll
    for (int i = 0; i < 2; ++i)
      if ((int)threadIdx.x + 256 * i < NCH) *reinterpret_cast<uint4*>(lds + 8 * (threadIdx.x + 256 * i)) = v[i];
    __syncthreads();
  }
};

// mid = embed[tok], tok = seq[*pos] (seq[0] without pos); the position is clamped into [0, seq_len) and the id into
// [0, vocab) so that bad device state cannot read out of bounds (one workgroup).
__global__ __launch_bounds__(256) void k_embed(const uint16_t* __restrict__ emb, long long vocab,
                                               const int64_t* __restrict__ seq, long long seq_len,
                                               const int64_t* __restrict__ pos, uint16_t* __restrict__ mid) {
  args_at_entry(emb, vocab, seq, seq_len, pos, mid);
  long long p = pos ? *pos : 0;
  p = p < 0 ? 0 : p >= seq_len ? seq_len - 1 : p;
  long long t = seq[p];
  t = t < 0 ? 0 : t >= vocab ? vocab - 1 : t;
  for (int ch = threadIdx.x; ch < kH / 8; ch += 256)
    *reinterpret_cast<uint4*>(mid + 8 * ch) = *reinterpret_cast<const uint4*>(emb + t * kH + 8 * ch);
}

// Lines (kLine words) of the fused attention block's sync buffer (handoff.h): each counter and flag on its own line.
// The attention block's sync buffer, in 256-byte lines: the error word; the generation number of the last completed
// launch (each launch reads it at entry and tags its words with it + 1; the router's last workgroup stores that
// number once every workgroup of the launch has read the old one); the split counters of the attention's chunks;
// the tagged words (handoff.h) of the phases' results: QKV rows (word 32 r + d: dims d and d + 32 of row r = head,
// 80 heads), the attention output (word i: elements 2i, 2i + 1), o_proj's mid (word i: rows 2i, 2i + 1) and the
// router's logits (word e: the fp32 logit of expert e); and, when the block leaves the top-4 selection to the expert
// body, the count of router workgroups that have read the generation word (the last one waits for it instead of for
// every logit before it advances the word, and returns it to zero).
constexpr int kSyncErr = 0, kSyncGen = 1;
constexpr int kSyncSplit = 2;                                   // 8 lines: the attention's split counters
constexpr int kTagQkv = 10;                                     // 2560 words, 80 lines
constexpr int kTagAtt = kTagQkv + kQkvRows / 2 / 32;            // 2048 words, 64 lines
constexpr int kTagMid = kTagAtt + kHq / 2 / 32;                 // 1440 words, 45 lines
constexpr int kTagLogit = kTagMid + kH / 2 / 32;                // 128 words, 4 lines
constexpr int kSyncEntered = kTagLogit + kNE / 32;              // router workgroups that have read the generation word
constexpr int kSyncLines = kSyncEntered + 1;                    // 204 lines, 52,224 bytes
constexpr int kSyncWords = kSyncLines * kLine;
NA_DEVICE uint64_t* sync_tags(uint32_t* sync, int line) { return reinterpret_cast<uint64_t*>(sync + line * kLine); }

// QKV: ROWS = 256 / TPR rows per workgroup, grid 5120 / ROWS; workgroup (head, c) computes the rows of dims
// d = c * ROWS/2 + (0 .. ROWS/2 - 1) (row groups 0 .. ROWS/2 - 1) and of their RoPE partners d + 32 (the other row
// groups) of head `head` (0..63 q, 64..71 k, 72..79 v).  FUSED (the first phase of k_attn_block): each (d, d + 32)
// pair is also written as tagged word 32 head + d (gen: the generation word as loaded at entry).  hc: kH bf16 of LDS, ys: ROWS floats of LDS.
template <int TPR, bool FUSED>
NA_DEVICE void qkv_body(int blk, uint16_t* hc, float* ys, const uint16_t* __restrict__ mid,
                        const uint16_t* __restrict__ g, const float* __restrict__ cext, uint16_t* __restrict__ xbuf,
                        const uint16_t* __restrict__ in_w, const uint16_t* __restrict__ W,
                        const uint16_t* __restrict__ bias, const int64_t* __restrict__ pos_p,
                        const float* __restrict__ inv_freq, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                        long long rows, int ring, uint16_t* __restrict__ qout, float eps, float att_scale,
                        uint64_t* tags, uint32_t gen) {
  constexpr int ROWS = 256 / TPR, HALF = ROWS / 2, PER_HEAD = 64 / ROWS;
  const int tid = threadIdx.x, r = tid / TPR, j = tid % TPR;
  const int head = blk / PER_HEAD, c = blk % PER_HEAD;
  const int d = HALF * c + (r % HALF);
  const int row = head * 64 + 32 * (r / HALF) + d;
  NormIn ni;
  ni.load(mid, g, cext, in_w);
  const uint16_t bv = bias[row];
  const long long pos = *pos_p;
  const float freq = inv_freq[HALF * c + (tid % HALF)];
  __builtin_amdgcn_sched_barrier(0);
  RowChunks<kH, TPR> rw;
  rw.load(W + (long long)row * kH, j);
  __builtin_amdgcn_sched_barrier(0);
  norm_finish(ni, g != nullptr, cext != nullptr, eps, hc, xbuf);
  const float s = rw.dot(hc, j);
  if (j == 0) ys[r] = rb(s + bf16_to_f32(bv));
  __syncthreads();
  if (tid < HALF) {                                  // thread t < HALF writes dims 32c' + t and its partner
    const int dd = HALF * c + tid;
    const float ya = ys[tid], yb = ys[tid + HALF];
    float o1 = ya, o2 = yb;
    if (head < 64 + 8) {                             // q and k heads: RoPE
      const float fr = freq * (float)pos;
      const float cs = rb(cosf(fr) * att_scale), sn = rb(sinf(fr) * att_scale);
      o1 = rb(rb(ya * cs) - rb(yb * sn));
      o2 = rb(rb(yb * cs) + rb(ya * sn));
    }
    uint16_t* dst = nullptr;
    if (head < 64) {
      dst = qout + head * 64;
    } else {
      const long long slot = ring > 0 ? pos % ring : pos;
      if (slot >= 0 && slot < rows)                  // a position outside the cache is stored nowhere
        dst = (head < 72 ? kc + (long long)(head - 64) * rows * 64 : vc + (long long)(head - 72) * rows * 64) +
              slot * 64;
    }
    const uint16_t b1 = f32_to_bf16(o1), b2 = f32_to_bf16(o2);
    if (dst) {
      dst[dd] = b1;
      dst[32 + dd] = b2;
    }
    if constexpr (FUSED) tag_store(tags + head * 32 + dd, (uint32_t)b1 | ((uint32_t)b2 << 16), launch_tag(gen));
  }
}

template <int TPR>
__global__ __launch_bounds__(256) void k_qkv(const uint16_t* __restrict__ mid, const uint16_t* __restrict__ g,
                                             const float* __restrict__ cext, uint16_t* __restrict__ xbuf,
                                             const uint16_t* __restrict__ in_w, const uint16_t* __restrict__ W,
                                             const uint16_t* __restrict__ bias, const int64_t* __restrict__ pos_p,
                                             const float* __restrict__ inv_freq, uint16_t* __restrict__ kc,
                                             uint16_t* __restrict__ vc, long long rows, int ring,
                                             uint16_t* __restrict__ qout, float eps, float att_scale) {
  __shared__ __align__(16) uint16_t hc[kH];
  __shared__ float ys[256 / TPR];
  qkv_body<TPR, false>(blockIdx.x, hc, ys, mid, g, cext, xbuf, in_w, W, bias, pos_p, inv_freq, kc, vc, rows, ring,
                       qout, eps, att_scale, nullptr, 0);
}

// o_proj + residual: 256 / TPR rows per workgroup: mid[n] = bf16(x[n] + bf16(att . Wo[n] + bo[n])), x = xbuf.
// FUSED (the third phase of k_attn_block): the weight rows are loaded first, then threads 0..7 poll a tagged word of
// each head's attention output (att_tags; gen: the generation word as loaded at entry), each thread reads its 8 words (16 of the 4096 elements), the
// workgroup recomputes its rows of x from mid, g and c (the residual the QKV phase normalised), and writes mid, also
// as tagged words (mid_tags: rows 2i, 2i + 1 in word i, from lanes 0 and 32 of each wave).
template <int TPR, bool FUSED>
NA_DEVICE void oproj_body(int blk, uint16_t* hc, const uint16_t* __restrict__ att, const uint16_t* __restrict__ Wo,
                          const uint16_t* __restrict__ bo, const uint16_t* __restrict__ xbuf,
                          const uint16_t* __restrict__ g, const float* __restrict__ cext, uint16_t* __restrict__ mid,
                          const uint64_t* att_tags, uint64_t* mid_tags, uint32_t gen, uint32_t* err) {
  constexpr int ROWS = 256 / TPR;
  static_assert(!FUSED || TPR == 32, "tagged mid words pair the rows of lanes 0 and 32");
  const int tid = threadIdx.x, r = tid / TPR, j = tid % TPR;
  const int row = ROWS * blk + r;
  VecIn<kHq> a;
  if constexpr (!FUSED) a.load(att);
  const uint16_t bv = bo[row];
  uint16_t xv;
  float gx = 0.f, cx = 0.f;
  if constexpr (FUSED) {
    xv = mid[row];
    if (g) gx = bf16_to_f32(g[row]);
    if (cext) cx = cext[row];
  } else {
    xv = xbuf[row];
  }
  __builtin_amdgcn_sched_barrier(0);
  RowChunks<kHq, TPR> rw;
  rw.load(Wo + (long long)row * kHq, j);
  __builtin_amdgcn_sched_barrier(0);
  float x = bf16_to_f32(xv);
  if constexpr (FUSED) {
    if (g) x = rb(x + rb(gx + (cext ? rb(cx) : 0.f)));
    gen = launch_tag(gen);
    // threads 0..7 poll the last word of each head's output, then every thread reads its 8 words (ordinary loads
    // first: the L2 of the XCD serves all but its first o_proj workgroup)
    if (tid < kNKV) tag_wait1(att_tags + (tid + 1) * (kHq / kNKV / 2) - 1, gen, err);
    __syncthreads();
    uint32_t w[8];
    tag_read<8, true>(att_tags + 8 * tid, gen, w, err);
    *reinterpret_cast<uint4*>(hc + 16 * tid) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint4*>(hc + 16 * tid + 8) = make_uint4(w[4], w[5], w[6], w[7]);
    __syncthreads();
  } else {
    a.store(hc);
  }
  const float s = rw.dot(hc, j);
  const uint16_t o = f32_to_bf16(x + rb(s + bf16_to_f32(bv)));
  if constexpr (FUSED) {
    if (j == 0) store_coherent(mid + row, o);
    const uint32_t o2 = (uint32_t)__builtin_amdgcn_readlane((int)o, 32);   // row 2 wave + 1
    if ((tid & 63) == 0) tag_store(mid_tags + ROWS / 2 * blk + (tid >> 6), (uint32_t)o | (o2 << 16), gen);
  } else {
    if (j == 0) mid[row] = o;
  }
}

template <int TPR>
__global__ __launch_bounds__(256) void k_oproj(const uint16_t* __restrict__ att, const uint16_t* __restrict__ Wo,
                                               const uint16_t* __restrict__ bo, const uint16_t* __restrict__ xbuf,
                                               uint16_t* __restrict__ mid) {
  __shared__ __align__(16) uint16_t hc[kHq];
  oproj_body<TPR, false>(blockIdx.x, hc, att, Wo, bo, xbuf, nullptr, nullptr, mid, nullptr, nullptr, 0, nullptr);
}

// post-attention RMSNorm + router + top-4: 256 / TPR experts per workgroup, grid 128 / (256 / TPR).  Workgroup 0 writes hn (the experts' input);
// every workgroup publishes its 16 logits (device-coherent stores, then a count); the last one selects the top 4,
// writes ids / weights and resets the count.
// Router phase: NR = 128 / (256 / TPR) workgroups; workgroup `blk` computes 256 / TPR logits.  FUSED (the last phase
// of k_attn_block): the weights and the norm weight are loaded first, then thread 0 polls one tagged word of mid
// (mid_tags; gen: the generation word as loaded at entry) and every thread reads its 8 words.  With ids (select):
// the logits are also written as tagged words (logit_tags), and the last workgroup (blk = NR - 1) reads all 128 of
// them, selects the top 4 and stores gen into *gen_word: every workgroup of the launch has read the old number by
// then (each one's result is an input of the router's logits, and each read the number before it produced
// anything).  Without ids the logits go to `logits` only, for the next launch (the expert body selects the top 4
// itself): each workgroup counts itself into *entered once its read of the generation word is complete, and the
// last workgroup, once its own logits are stored, waits for all NR counts (the other phases' workgroups have read
// the word, since their results fed its mid), returns the count to zero and advances the word.
template <int TPR, bool FUSED>
NA_DEVICE void router_body(int blk, int nr, uint16_t* hc, uint32_t& last, const uint16_t* __restrict__ mid,
                           const uint16_t* __restrict__ post_w, float eps, const uint16_t* __restrict__ Wr,
                           const uint16_t* __restrict__ br, uint16_t* __restrict__ hn, float* __restrict__ logits,
                           uint32_t* __restrict__ counter, int64_t* __restrict__ ids, uint16_t* __restrict__ wts,
                           const uint64_t* mid_tags, uint64_t* logit_tags, uint32_t* gen_word, uint32_t gen,
                           uint32_t* err, uint32_t* entered = nullptr) {
  constexpr int ROWS = 256 / TPR;
  const int tid = threadIdx.x, r = tid / TPR, j = tid % TPR;
  const int e = ROWS * blk + r;
  const bool select = ids != nullptr;
  if (FUSED && !select && tid == 0) {
    uint32_t one = 1u;
    asm volatile("; counted after the generation word %1 is read" : "+v"(one) : "v"(gen));
    __hip_atomic_fetch_add(entered, one, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  NormIn ni;
  if constexpr (FUSED) {
#pragma unroll
    for (int i = 0; i < 2; ++i) ni.w[i] = *reinterpret_cast<const uint4*>(post_w + 8 * min(tid + 256 * i, kH / 8 - 1));
  } else {
    ni.load(mid, nullptr, nullptr, post_w);
  }
  const uint16_t bv = br[e];
  __builtin_amdgcn_sched_barrier(0);
  RowChunks<kH, TPR> rw;
  rw.load(Wr + (long long)e * kH, j);
  __builtin_amdgcn_sched_barrier(0);
  if constexpr (FUSED) {
    gen = launch_tag(gen);
    if (tid == 0) tag_wait1(mid_tags + (kH / 2 - 1) - (kH / 2 / 32) * blk, gen, err);   // a word per workgroup
    __syncthreads();
    const uint64_t* src[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) src[k] = mid_tags + 4 * min(tid + 256 * (k >> 2), kH / 8 - 1) + (k & 3);
    uint32_t w[8];
    tag_read_at<8>(src, gen, w, err);
    ni.m[0] = make_uint4(w[0], w[1], w[2], w[3]);
    ni.m[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
  norm_finish(ni, false, false, eps, hc, nullptr);
  if (blk == 0)
    for (int i = tid; i < kH / 8; i += 256)
      *reinterpret_cast<uint4*>(hn + 8 * i) = *reinterpret_cast<const uint4*>(hc + 8 * i);
  const float s = rw.dot(hc, j);
  if constexpr (FUSED) {
    const float v = rb(s + bf16_to_f32(bv));
    if (!select) {
      if (j == 0) logits[e] = v;
      if (blk != nr - 1 || tid != 0) return;
      for (uint32_t n = 0; load_coherent(entered) < (uint32_t)nr; ++n) {
        if (n >= kSpinLimit) {
          __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      store_coherent(entered, 0u);
      store_coherent(gen_word, gen);
      return;
    }
    if (j == 0) {
      logits[e] = v;
      tag_store(logit_tags + e, __float_as_uint(v), gen);
    }
    if (blk != nr - 1 || tid >= 64) return;
    const uint64_t* src[2] = {logit_tags + tid, logit_tags + tid + 64};
    uint32_t l[2];
    tag_read_at<2>(src, gen, l, err);
    top4_softmax(__uint_as_float(l[0]), __uint_as_float(l[1]), tid, ids, wts);
    if (tid == 0) store_coherent(gen_word, gen);
    return;
  }
  if (j == 0) __hip_atomic_store(logits + e, rb(s + bf16_to_f32(bv)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (uint32_t)nr - 1;
    if (last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last || tid >= 64) return;
  top4_softmax(__hip_atomic_load(logits + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT),
               __hip_atomic_load(logits + tid + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), tid, ids, wts);
}

template <int TPR>
__global__ __launch_bounds__(256) void k_router_norm(const uint16_t* __restrict__ mid, const uint16_t* __restrict__ post_w,
                                                     float eps, const uint16_t* __restrict__ Wr,
                                                     const uint16_t* __restrict__ br, uint16_t* __restrict__ hn,
                                                     float* __restrict__ logits, uint32_t* __restrict__ counter,
                                                     int64_t* __restrict__ ids, uint16_t* __restrict__ wts) {
  __shared__ __align__(16) uint16_t hc[kH];
  __shared__ uint32_t last;
  router_body<TPR, false>(blockIdx.x, gridDim.x, hc, last, mid, post_w, eps, Wr, br, hn, logits, counter, ids, wts,
                          nullptr, nullptr, nullptr, 0, nullptr);
}

// Monotone map of bf16 bit patterns to unsigned order (-0 equal to +0; NaN patterns above +inf).
NA_DEVICE uint32_t bf16_order_key(uint16_t b) {
  if (b == 0x8000) b = 0;
  return (b & 0x8000) ? (uint32_t)(~b & 0xffff) : (uint32_t)(b | 0x8000);
}

// Monotone map of fp32 bit patterns to unsigned order (-0 equal to +0).
NA_DEVICE uint32_t f32_order_key(float f) {
  uint32_t b = __float_as_uint(f);
  if (b == 0x80000000u) b = 0;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// SplitMix64 (Steele, Lea and Flood, "Fast splittable pseudorandom number generators", OOPSLA 2014): the output
// function of its generator, used as a counter-based hash.
NA_DEVICE uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Uniform draw in [0, 1) on a 2^-24 grid for (seed, position, vocabulary index): the top 24 bits of
// splitmix64(splitmix64(seed ^ position) ^ index).
NA_DEVICE float uniform_draw(uint64_t seed, uint64_t p, uint32_t v) {
  return (float)(splitmix64(splitmix64(seed ^ p) ^ (uint64_t)v) >> 40) * 0x1p-24f;
}

// Sampling parameters of the tail (reference server.py:1576-1583, t_body_sample): token = argmax(logit / temp +
// g), g = -log(-log(clamp(u, 1e-12, 1 - 1e-7))), fp32, first index on ties; *temp <= 0 selects greedy argmax.  u
// from the array (the reference's u_dev, refreshed by the caller) or, without one, uniform_draw(*seed, *pos, v)
// (seed and pos read on the device, so a captured step draws new numbers at every position).
struct SampleArgs {
  const float* temp;
  const float* u;
  const int64_t* pos;
  const uint64_t* seed;
};

// ---- the decode tail in one launch (na_core_lm_tail; reference server.py:521-525): kTailWgs workgroups (fewer for
// a small vocabulary).  Each forms the final norm itself, x = bf16(mid + bf16(g + bf16(c))), hn = bf16(w * (x * r))
// (norm_finish: the same bits in every workgroup; workgroup 0 also writes hn), then streams the 16-row blocks
// blockIdx.x, blockIdx.x + gridDim.x, ... of lm_head, logit = bf16(hn . row) over TPR threads per row, keeping its
// best key (the logit's order key << 32 | ~index: a larger key is a larger logit, then a smaller index), and
// publishes it as two tagged words (handoff.h: the order key, and ~index).  The grid's last workgroup, once its own
// rows are done, reads every workgroup's two words, takes the largest key -> tok, and with pos (p = *pos, the
// position of this step's input token) sets pred[p + 1] = tok when pred is given, seq[p + 1] = tok unless position
// p + 1 is forced (p + 1 < *n_forced, a prompt token), pos = p + 1 when step_pos (writes stay below seq_len); then it
// advances the generation word (every workgroup has read the old one: its words carry the number formed from it).
// One launch instead of three (norm, lm_head, argmax): 175 -> 168 us per step at vocab 201,088.  The workgroups are
// persistent (3 per CU at this kernel's registers; c, when absent, holds none).  part: [line 0: error word][line 1:
// generation word][2 x grid tagged words] (uint32 lines of kLine), see na_core_lm_partials; any initial contents
// work, and a wait that gives up raises the error word.
constexpr int kTailWgs = 768;                              // 3 per CU (the kernel's occupancy) x 256 CUs
constexpr int kTailHead = 2 * kLine / 2;                    // uint64 entries of part before the tagged words

template <int TPR, bool SAMPLE, bool HAS_C>
__global__ __launch_bounds__(256) void k_tail(const uint16_t* __restrict__ mid, const uint16_t* __restrict__ g,
                                              const float* __restrict__ cext, const uint16_t* __restrict__ fw,
                                              float eps, const uint16_t* __restrict__ Wl, int vocab,
                                              uint16_t* __restrict__ hn, uint16_t* __restrict__ logits_out,
                                              uint32_t* __restrict__ part, int64_t* __restrict__ tok,
                                              int64_t* __restrict__ pos, int step_pos, int64_t* __restrict__ seq,
                                              const int64_t* __restrict__ n_forced, int64_t* __restrict__ pred,
                                              long long seq_len, SampleArgs sa) {
  __shared__ __align__(16) uint16_t hc[kH];
  constexpr int ROWS = 256 / TPR;
  __shared__ uint64_t best_lds[ROWS];
  const int tid = threadIdx.x, r = tid / TPR, j = tid % TPR;
  const int nblk = (vocab + ROWS - 1) / ROWS, nwg = gridDim.x;
  uint32_t* err = part;
  uint32_t* gen_word = part + kLine;
  uint64_t* words = reinterpret_cast<uint64_t*>(part) + kTailHead;
  const uint32_t gen = load_coherent(gen_word);             // raw: the tag is formed where it is first used
  float temp = 0.f;
  uint64_t p = 0, seed = 0;
  if constexpr (SAMPLE) {
    temp = *sa.temp;
    p = sa.pos ? (uint64_t)*sa.pos : 0;
    seed = sa.seed ? *sa.seed : 0;
  }
  NormIn ni;
  ni.load<HAS_C>(mid, g, cext, fw);
  int rb = blockIdx.x;
  int v = ROWS * rb + r;
  __builtin_amdgcn_sched_barrier(0);
  RowChunks<kH, TPR> rw;
  rw.load(Wl + (long long)min(v, vocab - 1) * kH, j);
  __builtin_amdgcn_sched_barrier(0);
  norm_finish(ni, g != nullptr, HAS_C && cext != nullptr, eps, hc, nullptr);
  if (blockIdx.x == 0)
    for (int i = tid; i < kH / 8; i += 256)
      *reinterpret_cast<uint4*>(hn + 8 * i) = *reinterpret_cast<const uint4*>(hc + 8 * i);
  uint64_t best = 0;                                        // this row group's best key (lane j == 0)
  for (;;) {
    const float s = rw.dot(hc, j);
    const int vr = v;
    rb += nwg;
    v = ROWS * rb + r;
    __builtin_amdgcn_sched_barrier(0);                  // one block's registers: the next loads after this dot
    if (rb < nblk) rw.load(Wl + (long long)min(v, vocab - 1) * kH, j);   // uniform
    __builtin_amdgcn_sched_barrier(0);
    if (j == 0 && vr < vocab) {
      const uint16_t lb = f32_to_bf16(s);
      if (logits_out) logits_out[vr] = lb;
      uint32_t key = bf16_order_key(lb);
      if constexpr (SAMPLE) {
        if (temp > 0.f) {
          float u = sa.u ? sa.u[vr] : uniform_draw(seed, p, (uint32_t)vr);
          u = fminf(fmaxf(u, 1e-12f), 1.0f - 1e-7f);
          const float gum = -logf(-logf(u));
          key = f32_order_key(bf16_to_f32(lb) / temp + gum);
        }
      }
      const uint64_t k = ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - (uint32_t)vr);
      best = k > best ? k : best;
    }
    if (rb >= nblk) break;
  }
  if (j == 0) best_lds[r] = best;
  __syncthreads();
  const uint32_t tag = launch_tag(gen);
  if (tid == 0) {
    uint64_t b = best_lds[0];
    for (int i = 1; i < ROWS; ++i) b = best_lds[i] > b ? best_lds[i] : b;
    tag_store(words + 2 * blockIdx.x, (uint32_t)(b >> 32), tag);
    tag_store(words + 2 * blockIdx.x + 1, (uint32_t)b, tag);
  }
  if ((int)blockIdx.x != nwg - 1) return;
  // the argmax over every workgroup's key: thread t reads the words of workgroups t, t + 256, t + 512, t + 768
  __shared__ uint64_t red[4];
  uint64_t b = 0;
  for (int w0 = 0; w0 < nwg; w0 += 4 * 256) {
    const uint64_t* src[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int w = min(w0 + tid + 256 * k, nwg - 1);
      src[2 * k] = words + 2 * w;
      src[2 * k + 1] = words + 2 * w + 1;
    }
    uint32_t kw[8];
    tag_read_at<8>(src, tag, kw, err);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint64_t c = ((uint64_t)kw[2 * k] << 32) | kw[2 * k + 1];
      b = c > b ? c : b;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint64_t ob = ((uint64_t)(uint32_t)__shfl_xor((int)(b >> 32), o) << 32) | (uint32_t)__shfl_xor((int)b, o);
    b = ob > b ? ob : b;
  }
  if ((tid & 63) == 0) red[tid >> 6] = b;
  __syncthreads();
  if (tid != 0) return;
  for (int i = 1; i < 4; ++i) b = red[i] > b ? red[i] : b;
  const int64_t t = (int64_t)(0xffffffffu - (uint32_t)(b & 0xffffffffu));
  *tok = t;
  if (pos) {
    const long long p0 = *pos, nx = p0 + 1;
    if (nx < seq_len && nx >= 0) {
      if (pred) pred[nx] = t;
      if (seq && !(n_forced && nx < *n_forced)) seq[nx] = t;
    }
    if (step_pos) *pos = nx;
  }
  store_coherent(gen_word, tag);
}

// ---- prompt rows (prefill of T tokens; reference server.py:2357-2403 _rope_tables / _attn_router and
//      _prefill_block :2406-2418): the same rounding points as the decode kernels above, one row per workgroup.

// x[t] = embed[ids[t]] (ids clamped into [0, vocab)).
__global__ __launch_bounds__(256) void k_rows_embed(const uint16_t* __restrict__ emb, long long vocab,
                                                    const int64_t* __restrict__ ids, uint16_t* __restrict__ x) {
  const long long t = blockIdx.x;
  long long id = ids[t];
  id = id < 0 ? 0 : id >= vocab ? vocab - 1 : id;
  for (int ch = threadIdx.x; ch < kH / 8; ch += 256)
    *reinterpret_cast<uint4*>(x + t * kH + 8 * ch) = *reinterpret_cast<const uint4*>(emb + id * kH + 8 * ch);
}

// Residual + RMSNorm of row t: x[t] = bf16(x[t] + add[t]) in place when add is given; hn[t] = bf16(w * (x * r)),
// r = rsqrt(sum x^2 / H + eps) with the decode kernels' summation order.
__global__ __launch_bounds__(256) void k_rows_norm(uint16_t* __restrict__ x, const uint16_t* __restrict__ add,
                                                   const uint16_t* __restrict__ w, float eps,
                                                   uint16_t* __restrict__ hn) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const long long base = (long long)blockIdx.x * kH;
  uint4 xv4[2], av4[2], wv4[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ch = min(tid + 256 * i, kH / 8 - 1);
    xv4[i] = *reinterpret_cast<const uint4*>(x + base + 8 * ch);
    av4[i] = *reinterpret_cast<const uint4*>((add ? add : x) + base + 8 * ch);
    wv4[i] = *reinterpret_cast<const uint4*>(w + 8 * ch);
  }
  float xv[2][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float v = half_at(xv4[i], e);
      if (add) v = rb(v + half_at(av4[i], e));
      xv[i][e] = v;
      if (tid + 256 * i < kH / 8) ss += v * v;
    }
  }
  ss = wave_sum_lane0(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  const float r = rsqrtf(((red[0] + red[1]) + (red[2] + red[3])) * (1.0f / kH) + eps);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int ch = tid + 256 * i;
    if (ch < kH / 8) {
      uint32_t o[4], xo[4];
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        o[e >> 1] = pack_bf16x2(half_at(wv4[i], e) * (xv[i][e] * r), half_at(wv4[i], e + 1) * (xv[i][e + 1] * r));
        xo[e >> 1] = pack_bf16x2(xv[i][e], xv[i][e + 1]);
      }
      *reinterpret_cast<uint4*>(hn + base + 8 * ch) = make_uint4(o[0], o[1], o[2], o[3]);
      if (add) *reinterpret_cast<uint4*>(x + base + 8 * ch) = make_uint4(xo[0], xo[1], xo[2], xo[3]);
    }
  }
}

// RoPE of row t of qkv [T, 5120] (q heads 0..63, k heads 64..71, v heads 72..79) at position p0 + t:
// q -> q_out [T, 64, 64]; k -> k_dst + t kt + h kh; v (no rotation) -> v_dst + t vt + h vh.
__global__ __launch_bounds__(256) void k_rows_rope(const uint16_t* __restrict__ qkv, long long p0,
                                                   const float* __restrict__ inv_freq, float att_scale,
                                                   uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_dst,
                                                   long long kt, long long kh, uint16_t* __restrict__ v_dst,
                                                   long long vt, long long vh) {
  __shared__ float cs[32], sn[32];
  const int tid = threadIdx.x;
  const long long t = blockIdx.x;
  const uint16_t* row = qkv + t * kQkvRows;
  if (tid < 32) {
    const float fr = inv_freq[tid] * (float)(p0 + t);
    cs[tid] = rb(cosf(fr) * att_scale);
    sn[tid] = rb(sinf(fr) * att_scale);
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 9; ++i) {                      // pairs 0..2047: q heads; 2048..2303: k heads
    const int P = tid + 256 * i;
    const int head = P >> 5, d = P & 31;
    const float ya = bf16_to_f32(row[head * 64 + d]), yb = bf16_to_f32(row[head * 64 + 32 + d]);
    const uint16_t o1 = f32_to_bf16(rb(ya * cs[d]) - rb(yb * sn[d]));
    const uint16_t o2 = f32_to_bf16(rb(yb * cs[d]) + rb(ya * sn[d]));
    if (head < 64) {
      q_out[t * kHq + head * 64 + d] = o1;
      q_out[t * kHq + head * 64 + 32 + d] = o2;
    } else {
      uint16_t* kr = k_dst + t * kt + (long long)(head - 64) * kh;
      kr[d] = o1;
      kr[32 + d] = o2;
    }
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int e = tid + 256 * i;                     // v values 0..511
    v_dst[t * vt + (long long)(e >> 6) * vh + (e & 63)] = row[kHq + 512 + e];
  }
}

// Top 4 of each row of router logits [T, 128] (bf16), softmax over the four: one wave per row.
__global__ __launch_bounds__(256) void k_rows_topk(const uint16_t* __restrict__ logits, int T,
                                                   int64_t* __restrict__ ids, uint16_t* __restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const long long t = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const uint16_t* lr = logits + t * kNE;
  top4_softmax(bf16_to_f32(lr[lane]), bf16_to_f32(lr[lane + 64]), lane, ids + 4 * t, wts + 4 * t);
}


// The serving bookkeeping around a routing na_core_router computed (reference fused_core.py:417-502, the k_router /
// k_topk stores beyond the logits): bx <- hn; pack[0, H) <- hn widened to fp32; for rank j with expert i_j, weight
// w_j, global id g = base + i_j and slot s = slot_tab ? slot_tab[g] : g (resident iff s >= 0): bslots[j] = s or 0,
// bgids[j] = g, bw[j] = w_j or +0, pack[H + j] = w_j, pack[H + 4 + j] = i_j, pack[H + 8 + j] = 1 or 0; with
// near_miss, pack[H + 12 + r] = the expert of rank 5 + r (repeated argmax of the logits without the top 4, lowest
// index on ties).  One workgroup.
__global__ __launch_bounds__(256) void k_route_pack(const uint16_t* __restrict__ hn, const float* __restrict__ logits,
                                                    const int64_t* __restrict__ ids, const uint16_t* __restrict__ wts,
                                                    const int64_t* __restrict__ slot_tab, long long base,
                                                    uint16_t* __restrict__ bx, float* __restrict__ pack,
                                                    int64_t* __restrict__ bslots, int64_t* __restrict__ bgids,
                                                    uint16_t* __restrict__ bw, int near_miss) {
  const int tid = threadIdx.x;
  for (int i = tid; i < kH; i += 256) {
    const uint16_t h = hn[i];
    if (bx) bx[i] = h;
    if (pack) pack[i] = bf16_to_f32(h);
  }
  if (tid < 4) {
    const int64_t e = ids[tid];
    const long long g = base + e;
    const int64_t s = slot_tab ? slot_tab[g] : g;
    const bool hit = s >= 0;
    bslots[tid] = hit ? s : 0;
    bgids[tid] = g;
    bw[tid] = hit ? wts[tid] : (uint16_t)0;
    if (pack) {
      pack[kH + tid] = bf16_to_f32(wts[tid]);
      pack[kH + 4 + tid] = (float)e;
      pack[kH + 8 + tid] = hit ? 1.f : 0.f;
    }
  }
  if (!near_miss || tid >= 64) return;
  float v0 = logits[tid], v1 = logits[tid + 64];
  for (int j = 0; j < 4; ++j) {
    const int64_t e = ids[j];
    if (e == tid) v0 = -INFINITY;
    if (e == tid + 64) v1 = -INFINITY;
  }
  for (int r = 0; r < 4; ++r) {
    float v = v0;
    int i = tid;
    if (v1 > v) {                                   // ties keep the lower index
      v = v1;
      i = tid + 64;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float ov = __shfl_xor(v, o);
      const int oi = __shfl_xor(i, o);
      if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
      }
    }
    if (tid == 0) pack[kH + 12 + r] = (float)i;
    if (i == tid) v0 = -INFINITY;
    if (i == tid + 64) v1 = -INFINITY;
  }
}


// ---------------------------------------------------------------- the attention block of a decode layer, one launch
// Phases by workgroup id (see handoff.h): [QKV: 640][attention: 8 ns][o_proj: 360][router: 32].  Each phase issues
// its own loads first (weights, the older keys of the cache) and then waits for what it needs, reading the earlier
// phases' results as tagged words: the attention of KV head h the 80 QKV rows of its group (query heads 8h .. 8h + 7,
// K and V head h: q and the step's K / V row), o_proj the 8 attention heads' output, the router every o_proj row,
// the router's last workgroup every logit.  sync: kSyncWords uint32 (the layout above), zero before the first launch;
// a launch leaves the split counters zero, the generation word advanced by one and the error word (line kSyncErr)
// as it was unless a wait gave up, which raises it (nothing clears it).
constexpr int kBlkQkv = kQkvRows / (256 / kQkvTpr);
constexpr int kBlkOproj = kH / (256 / kOprojTpr);
constexpr int kBlkRouter = kNE / (256 / kRouterTpr);

union AttnBlockLds {
  AttnLds attn;
  struct {
    __align__(16) uint16_t hc[kHq];
    float ys[256];
    uint32_t last;
  } core;
};

struct AttnBlockArgs {
  uint16_t* mid;
  const uint16_t* g;
  const float* c;
  uint16_t* xbuf;
  const uint16_t* in_w;
  const uint16_t* Wqkv;
  const uint16_t* bqkv;
  const int64_t* pos;
  const float* inv_freq;
  uint16_t* kc;
  uint16_t* vc;
  long long cache_rows;
  int ring;
  int window;
  int ns;
  float eps;
  float att_scale;
  float scaling;
  uint16_t* q;
  const uint16_t* sinks;
  float* work;
  uint16_t* att;
  const uint16_t* Wo;
  const uint16_t* bo;
  const uint16_t* post_w;
  const uint16_t* Wr;
  const uint16_t* br;
  uint16_t* hn;
  float* logits;
  int64_t* ids;
  uint16_t* wts;
  uint32_t* sync;
};

__global__ __launch_bounds__(256, 4) void k_attn_block(AttnBlockArgs a) {
  __shared__ AttnBlockLds L;
  uint32_t* sync = a.sync;
  uint32_t* err = sync + kSyncErr * kLine;
  const uint32_t gen = load_coherent(sync + kSyncGen * kLine);   // raw: each phase forms its tag where it needs it
  int blk = blockIdx.x;
  if (blk < kBlkQkv) {                                  // QKV -> tagged q, K, V rows
    qkv_body<kQkvTpr, true>(blk, L.core.hc, L.core.ys, a.mid, a.g, a.c, a.xbuf, a.in_w, a.Wqkv, a.bqkv, a.pos,
                            a.inv_freq, a.kc, a.vc, a.cache_rows, a.ring, a.q, a.eps, a.att_scale,
                            sync_tags(sync, kTagQkv), gen);
    return;
  }
  blk -= kBlkQkv;
  const int natt = kNKV * a.ns;
  if (blk < natt) {                                     // attention (chunks counted per head) -> tagged att
    decode_attn_body<true>(L.attn, blk, a.q, a.kc, a.vc, a.cache_rows, a.sinks, a.pos, a.att, a.scaling, a.window,
                           a.ring, a.ns, a.work, sync + kSyncSplit * kLine,
                           AttnHandoff{sync_tags(sync, kTagQkv), sync_tags(sync, kTagAtt), gen, err});
    return;
  }
  blk -= natt;
  if (blk < kBlkOproj) {                                // o_proj -> tagged mid
    oproj_body<kOprojTpr, true>(blk, L.core.hc, a.att, a.Wo, a.bo, nullptr, a.g, a.c, a.mid, sync_tags(sync, kTagAtt),
                                sync_tags(sync, kTagMid), gen, err);
    return;
  }
  blk -= kBlkOproj;
  router_body<kRouterTpr, true>(blk, kBlkRouter, L.core.hc, L.core.last, a.mid, a.post_w, a.eps, a.Wr, a.br, a.hn,
                                a.logits, nullptr, a.ids, a.wts, sync_tags(sync, kTagMid), sync_tags(sync, kTagLogit),
                                sync + kSyncGen * kLine, gen, err, sync + kSyncEntered * kLine);
}
}  // namespace na

using namespace na;

extern "C" {

int na_core_embed(const void* emb, long long vocab, const int64_t* seq, long long seq_len, const int64_t* pos,
                  void* mid, hipStream_t stream) {
  if (!emb || vocab <= 0 || !seq || seq_len <= 0 || !mid) return kErrArgs;
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, stream, (const uint16_t*)emb, vocab, seq, seq_len, pos,
                     (uint16_t*)mid);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_qkv(const void* mid, const void* g, const float* c, void* xbuf, const void* in_w, const void* W,
                const void* bias, const int64_t* pos, const float* inv_freq, void* kc, void* vc, long long cache_rows,
                int ring, void* q, float eps, float att_scale, hipStream_t stream) {
  if (!mid || !xbuf || !in_w || !W || !bias || !pos || !inv_freq || !kc || !vc || !q || cache_rows <= 0 || ring < 0)
    return kErrArgs;
  if (c && !g) return kErrArgs;
  if (ring > 0 && cache_rows != ring) return kErrArgs;
  hipLaunchKernelGGL(k_qkv<kQkvTpr>, dim3(kQkvRows / (256 / kQkvTpr)), dim3(256), 0, stream, (const uint16_t*)mid, (const uint16_t*)g, c,
                     (uint16_t*)xbuf, (const uint16_t*)in_w, (const uint16_t*)W, (const uint16_t*)bias, pos, inv_freq,
                     (uint16_t*)kc, (uint16_t*)vc, cache_rows, ring, (uint16_t*)q, eps, att_scale);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_oproj(const void* att, const void* Wo, const void* bo, const void* xbuf, void* mid, hipStream_t stream) {
  if (!att || !Wo || !bo || !xbuf || !mid) return kErrArgs;
  hipLaunchKernelGGL(k_oproj<kOprojTpr>, dim3(kH / (256 / kOprojTpr)), dim3(256), 0, stream, (const uint16_t*)att, (const uint16_t*)Wo,
                     (const uint16_t*)bo, (const uint16_t*)xbuf, (uint16_t*)mid);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_router(const void* mid, const void* post_w, float eps, const void* Wr, const void* br, void* hn,
                   float* logits, unsigned int* counter, int64_t* ids, void* wts, hipStream_t stream) {
  if (!mid || !post_w || !Wr || !br || !hn || !logits || !counter || !ids || !wts) return kErrArgs;
  hipLaunchKernelGGL(k_router_norm<kRouterTpr>, dim3(kNE / (256 / kRouterTpr)), dim3(256), 0, stream, (const uint16_t*)mid,
                     (const uint16_t*)post_w, eps, (const uint16_t*)Wr, (const uint16_t*)br, (uint16_t*)hn, logits,
                     (uint32_t*)counter, ids, (uint16_t*)wts);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_route_pack(const void* hn, const float* logits, const int64_t* ids, const void* wts,
                       const int64_t* slot_tab, long long base, void* bx, float* pack, int near_miss, int64_t* bslots,
                       int64_t* bgids, void* bw, hipStream_t stream) {
  if (!ids || !wts || !bslots || !bgids || !bw || base < 0) return kErrArgs;
  if ((bx || pack) && !hn) return kErrArgs;
  if (near_miss && (!pack || !logits)) return kErrArgs;
  hipLaunchKernelGGL(k_route_pack, dim3(1), dim3(256), 0, stream, (const uint16_t*)hn, logits, ids,
                     (const uint16_t*)wts, slot_tab, base, (uint16_t*)bx, pack, bslots, bgids, (uint16_t*)bw,
                     near_miss ? 1 : 0);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_attn_block(void* mid, const void* g, const float* c, void* xbuf, const void* in_w, const void* Wqkv,
                       const void* bqkv, const int64_t* pos, const float* inv_freq, void* kc, void* vc,
                       long long cache_rows, int ring, void* q, float eps, float att_scale, const void* sinks,
                       float scaling, int window, int n_split, float* attn_work, void* att, const void* Wo,
                       const void* bo, const void* post_w, const void* Wr, const void* br, void* hn, float* logits,
                       int64_t* ids, void* wts, unsigned int* sync, void* const* events, hipStream_t stream) {
  if (!mid || !xbuf || !in_w || !Wqkv || !bqkv || !pos || !inv_freq || !kc || !vc || !q || !sinks || !att || !Wo ||
      !bo || !post_w || !Wr || !br || !hn || !logits || !ids != !wts || !sync || cache_rows <= 0 || ring < 0)
    return kErrArgs;
  if (c && !g) return kErrArgs;
  if (ring > 0 && (window <= 0 || ring < window || cache_rows != ring)) return kErrArgs;
  if (n_split <= 0 || n_split > kAttnMaxSplit || window < 0 || (n_split > 1 && !attn_work)) return kErrArgs;
  // 16-byte rows for the vector accesses; the handoff words in sync are 64-bit device-coherent atomics
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc) |
       reinterpret_cast<uintptr_t>(att) | reinterpret_cast<uintptr_t>(sync)) & 15)
    return kErrArgs;
  AttnBlockArgs a{(uint16_t*)mid, (const uint16_t*)g, c, (uint16_t*)xbuf, (const uint16_t*)in_w,
                  (const uint16_t*)Wqkv, (const uint16_t*)bqkv, pos, inv_freq, (uint16_t*)kc, (uint16_t*)vc,
                  cache_rows, ring, window, n_split, eps, att_scale, scaling, (uint16_t*)q, (const uint16_t*)sinks,
                  attn_work, (uint16_t*)att, (const uint16_t*)Wo, (const uint16_t*)bo, (const uint16_t*)post_w,
                  (const uint16_t*)Wr, (const uint16_t*)br, (uint16_t*)hn, logits, ids, (uint16_t*)wts,
                  (uint32_t*)sync};
  const dim3 grid((unsigned)(kBlkQkv + kNKV * n_split + kBlkOproj + kBlkRouter)), block(256);
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  if (e0 || e1)
    hipExtLaunchKernelGGL(k_attn_block, grid, block, 0, stream, e0, e1, 0, a);
  else
    hipLaunchKernelGGL(k_attn_block, grid, block, 0, stream, a);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

long long na_core_attn_block_sync_words(void) { return kSyncWords; }

// Workgroups of the tail's launch: kTailWgs, or one per 16-row block of a smaller vocabulary.
static int tail_wgs(int vocab) { return min(kTailWgs, (vocab + 256 / kLmTpr - 1) / (256 / kLmTpr)); }

long long na_core_lm_partials(int vocab) { return vocab > 0 ? kTailHead + 2LL * tail_wgs(vocab) : -1; }

int na_core_lm_tail(const void* mid, const void* g, const float* c, const void* final_w, float eps, const void* Wl,
                    int vocab, void* hn, void* logits_out, unsigned long long* part, int64_t* tok, int64_t* pos,
                    int step_pos, int64_t* seq, const int64_t* n_forced, int64_t* pred, long long seq_len,
                    hipStream_t stream) {
  if (!mid || !final_w || !Wl || vocab <= 0 || !hn || !part || !tok) return kErrArgs;
  if ((step_pos || seq || pred) && !pos) return kErrArgs;
  if ((seq || pred) && seq_len <= 0) return kErrArgs;
  if (c && !g) return kErrArgs;
  if (reinterpret_cast<uintptr_t>(part) & 7) return kErrArgs;
  hipLaunchKernelGGL((c ? k_tail<kLmTpr, false, true> : k_tail<kLmTpr, false, false>), dim3(tail_wgs(vocab)), dim3(256), 0,
                     stream, (const uint16_t*)mid,
                     (const uint16_t*)g, c, (const uint16_t*)final_w, eps, (const uint16_t*)Wl, vocab, (uint16_t*)hn,
                     (uint16_t*)logits_out, (uint32_t*)part, tok, pos, step_pos, seq, n_forced, pred, seq_len,
                     SampleArgs{});
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_core_lm_tail_sample(const void* mid, const void* g, const float* c, const void* final_w, float eps,
                           const void* Wl, int vocab, void* hn, void* logits_out, unsigned long long* part,
                           int64_t* tok, int64_t* pos, int step_pos, int64_t* seq, const int64_t* n_forced,
                           int64_t* pred, long long seq_len, const float* temp, const float* u,
                           const unsigned long long* seed, hipStream_t stream) {
  if (!mid || !final_w || !Wl || vocab <= 0 || !hn || !part || !tok || !temp) return kErrArgs;
  if ((step_pos || seq || pred) && !pos) return kErrArgs;
  if ((seq || pred) && seq_len <= 0) return kErrArgs;
  if (c && !g) return kErrArgs;
  if (reinterpret_cast<uintptr_t>(part) & 7) return kErrArgs;
  hipLaunchKernelGGL((c ? k_tail<kLmTpr, true, true> : k_tail<kLmTpr, true, false>), dim3(tail_wgs(vocab)), dim3(256), 0,
                     stream, (const uint16_t*)mid,
                     (const uint16_t*)g, c, (const uint16_t*)final_w, eps, (const uint16_t*)Wl, vocab, (uint16_t*)hn,
                     (uint16_t*)logits_out, (uint32_t*)part, tok, pos, step_pos, seq, n_forced, pred, seq_len,
                     SampleArgs{temp, u, pos, (const uint64_t*)seed});
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_rows_embed(const void* emb, long long vocab, const int64_t* ids, int T, void* x, hipStream_t stream) {
  if (T < 0 || vocab <= 0) return kErrArgs;
  if (T == 0) return kOk;
  if (!emb || !ids || !x) return kErrArgs;
  hipLaunchKernelGGL(k_rows_embed, dim3(T), dim3(256), 0, stream, (const uint16_t*)emb, vocab, ids, (uint16_t*)x);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_rows_norm(void* x, const void* add, int T, const void* w, float eps, void* hn, hipStream_t stream) {
  if (T < 0) return kErrArgs;
  if (T == 0) return kOk;
  if (!x || !w || !hn) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(add) | reinterpret_cast<uintptr_t>(w) |
       reinterpret_cast<uintptr_t>(hn)) & 15)
    return kErrArgs;
  hipLaunchKernelGGL(k_rows_norm, dim3(T), dim3(256), 0, stream, (uint16_t*)x, (const uint16_t*)add,
                     (const uint16_t*)w, eps, (uint16_t*)hn);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_rows_rope(const void* qkv, int T, long long p0, const float* inv_freq, float att_scale, void* q, void* k_dst,
                 long long kt, long long kh, void* v_dst, long long vt, long long vh, hipStream_t stream) {
  if (T < 0 || p0 < 0) return kErrArgs;
  if (T == 0) return kOk;
  if (!qkv || !inv_freq || !q || !k_dst || !v_dst || kt < 0 || kh < 0 || vt < 0 || vh < 0) return kErrArgs;
  hipLaunchKernelGGL(k_rows_rope, dim3(T), dim3(256), 0, stream, (const uint16_t*)qkv, p0, inv_freq, att_scale,
                     (uint16_t*)q, (uint16_t*)k_dst, kt, kh, (uint16_t*)v_dst, vt, vh);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

int na_rows_topk(const void* logits, int T, int64_t* ids, void* wts, hipStream_t stream) {
  if (T < 0) return kErrArgs;
  if (T == 0) return kOk;
  if (!logits || !ids || !wts) return kErrArgs;
  hipLaunchKernelGGL(k_rows_topk, dim3((T + 3) / 4), dim3(256), 0, stream, (const uint16_t*)logits, T, ids,
                     (uint16_t*)wts);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
