// GQA decode attention with learned sinks (64 query heads, 8 KV heads, head_dim 64) on gfx950, for B sequences.
//
// Per (sequence b, KV head h): the 8 query rows of the head attend keys [lo, pos] (lo = max(pos - window + 1, 0) on
// sliding layers, 0 on full layers); key j lives in cache row j (linear cache) or j % ring (rolling cache).  Scores
// use the reference's rounding points, s = bf16(bf16(q . k) * scaling) with q . k accumulated in fp32 (reference
// fused_core.py:172-173), so every score is the reference's bf16 value.  The softmax with the sink then runs as
// flash decoding: the keys are split into NS chunks (the reference's split rule, fused_core.py:222-228), a
// workgroup computes for its chunk the row maximum m_c, the row sums S_c = sum bf16(exp(s - m_c)) and the
// unnormalised P V (P = bf16(exp(s - m_c)), fp32 accumulation, MFMA), and the last workgroup of the (b, h) to finish
// combines the NS partials in chunk order:
//   m = max(sink, max_c m_c);  S = exp(sink - m) + sum_c S_c exp(m_c - m);  out = bf16(sum_c acc_c exp(m_c - m) / S).
// The result is the reference's sink attention up to fp32/bf16 rounding (the reference instead rounds exp
// arguments and P / S to bf16 against the global maximum, in three dependent passes); one launch per layer.
//
// Work layout of a workgroup (4 waves): the chunk is walked in sub-chunks of 256 keys, wave w taking keys
// [64 w, 64 w + 64) of each; scores = v_mfma_f32_16x16x32_bf16 with A = the 8 query rows (rows 8..15 zero) and
// B = K^T (lane l = 16 q + n loads 16 bytes of key n's row: exactly its B operand); P and V^T are staged in LDS and
// P V = v_mfma_f32_16x16x32_bf16 with wave w producing output columns [16 w, 16 w + 16).  Sub-chunks after the first
// rescale the running state (online softmax).
#include "common.h"

#include <hip/hip_ext.h>

namespace na {

constexpr int kNQ = 64, kNKV = 8, kHD = 64, kRep = 8;
constexpr int kSub = 256;                          // keys per sub-chunk (4 waves x 64)
constexpr int kAttnMaxSplit = 64;
constexpr int kPartFloats = kRep + kRep + kRep * kHD;   // m[8], S[8], acc[8][64] per chunk
constexpr int kVtPitch = kSub * 2 + 16;            // LDS bytes per V^T row (d), padded against bank conflicts
constexpr int kPPitch = kSub * 2 + 16;             // LDS bytes per P row
constexpr float kNegInf = -__builtin_huge_valf();

struct AttnLds {
  __align__(16) uint8_t vt[kHD * kVtPitch];        // V^T of the sub-chunk, bf16 [d][key]
  __align__(16) uint8_t p[16 * kPPitch];           // P of the sub-chunk, bf16 [row][key] (rows 8..15 unused)
  float mx[4][kRep];                               // per-wave row maxima
  float sm[4][kRep];                               // per-wave row sums
  float fin[kRep][2];                              // combine: 1 / S per row (index 1)
  float cm[kAttnMaxSplit][kRep];                   // combine: chunk maxima, sums and weights
  float cs[kAttnMaxSplit][kRep];
  float cw[kAttnMaxSplit][kRep];
};

// Wave-wide max / sum over the 16 lanes of a row group (lanes 16 q .. 16 q + 15).
NA_DEVICE float group16_max(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
NA_DEVICE float group16_sum(float v) {
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) v += __shfl_xor(v, o);
  return v;
}

NA_DEVICE bf16x8_t as_bf16x8(uint4 v) { return __builtin_bit_cast(bf16x8_t, v); }

// Key range [c0, c1) of chunk c (empty when c0 >= c1): the reference's split rule over 64-key blocks of [lo, hi].
NA_DEVICE void chunk_range(int lo, int hi, int c, int ns, int& c0, int& c1) {
  const int n = hi - lo + 1;
  const int nb = (n + 63) / 64;
  const int bps = (nb + ns - 1) / ns;
  c0 = lo + c * bps * 64;
  c1 = min(c0 + bps * 64, hi + 1);
}

__global__ __launch_bounds__(256) void k_decode_attn(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    long long cache_rows, const uint16_t* __restrict__ sinks, const int64_t* __restrict__ pos_p,
    uint16_t* __restrict__ out, float scaling, int window, int ring, int ns, float* __restrict__ work,
    uint32_t* __restrict__ counters) {
  __shared__ AttnLds L;
  args_at_entry(q, kc, vc, cache_rows, sinks, pos_p, out, scaling, window, ring, ns, work, counters);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, n = lane & 15;          // row group (D rows 4g..4g+3) and column of this lane
  const int c = blockIdx.x % ns;
  const int bh = blockIdx.x / ns;                  // b * 8 + h
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
  uint4 qa0 = *reinterpret_cast<const uint4*>(qrow + 8 * g);
  uint4 qa1 = *reinterpret_cast<const uint4*>(qrow + 32 + 8 * g);
  if (n >= kRep) qa0 = qa1 = make_uint4(0, 0, 0, 0);

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
    for (int r = 0; r < 4; ++r) wmax[r] = group16_max(wmax[r]);
    if (n == 0 && g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) L.mx[wave][4 * g + r] = wmax[r];
    }
    // ---- V^T to LDS: lane (g, n) holds d = 8g..8g+7 and 32+8g.. of key 16 kb + n of this wave's 64
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int kcol = 64 * wave + 16 * kb + n;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const uint32_t w4[4] = {vr[kb][hf].x, vr[kb][hf].y, vr[kb][hf].z, vr[kb][hf].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int dd = 32 * hf + 8 * g + i;
          *reinterpret_cast<uint16_t*>(L.vt + dd * kVtPitch + 2 * kcol) =
              (uint16_t)((i & 1) ? (w4[i >> 1] >> 16) : (w4[i >> 1] & 0xffff));
        }
      }
    }
    __syncthreads();
    // ---- sub-chunk max (exact, any order), new running max, P = bf16(exp(s - m_new)), row sums
    float m_new[4], alpha[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * min(g, 1) + r;
      float mx = fmaxf(fmaxf(L.mx[0][row], L.mx[1][row]), fmaxf(L.mx[2][row], L.mx[3][row]));
      m_new[r] = fmaxf(m_run[r], mx);
      alpha[r] = m_new[r] == kNegInf ? 1.f : expf(m_run[r] - m_new[r]);
    }
    float psum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int kcol = 64 * wave + 16 * kb + n;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float e = s[kb][r] == kNegInf ? 0.f : expf(s[kb][r] - m_new[r]);
        const uint16_t pb = f32_to_bf16(e);
        psum[r] += bf16_to_f32(pb);
        if (g < 2) *reinterpret_cast<uint16_t*>(L.p + (4 * g + r) * kPPitch + 2 * kcol) = pb;
      }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) psum[r] = group16_sum(psum[r]);
    if (n == 0 && g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) L.sm[wave][4 * g + r] = psum[r];
    }
    __syncthreads();
    // ---- running state: S = S alpha + sum of the 4 waves (fixed order); acc = acc alpha + P V
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * min(g, 1) + r;
      const float sub = ((L.sm[0][row] + L.sm[1][row]) + L.sm[2][row]) + L.sm[3][row];
      s_run[r] = s_run[r] * alpha[r] + sub;
      m_run[r] = m_new[r];
      acc[r] *= alpha[r];
    }
    const int nks = (min(kSub, c1 - k0) + 31) / 32;     // 32-key steps holding live keys (P is 0 past c1)
#pragma unroll
    for (int ks = 0; ks < kSub / 32; ++ks) {
      if (ks < nks) {                                  // uniform
        const uint4 pa = *reinterpret_cast<const uint4*>(L.p + n * kPPitch + 2 * (32 * ks + 8 * g));
        const uint4 vb = *reinterpret_cast<const uint4*>(L.vt + (16 * wave + n) * kVtPitch + 2 * (32 * ks + 8 * g));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(pa), as_bf16x8(vb), acc, 0, 0, 0);
      }
    }
    __syncthreads();                               // LDS is rewritten by the next sub-chunk
  }

  // ---- finish: a single chunk writes the output; otherwise publish the partial, the last arriver combines
  const uint16_t* sk = sinks + h * kRep;
  uint16_t* orow = out + ((long long)b * kNQ + h * kRep) * kHD;
  if (ns == 1) {
    if (g < 2) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float sink = bf16_to_f32(sk[4 * g + r]);
        const float m = fmaxf(sink, m_run[r]);
        const float a = m_run[r] == kNegInf ? 0.f : expf(m_run[r] - m);
        const float S = expf(sink - m) + s_run[r] * a;   // the combine's formula, so one chunk == split at pos < 64
        orow[(4 * g + r) * kHD + 16 * wave + n] = f32_to_bf16((0.f + acc[r] * a) * (1.f / S));
      }
    }
    return;
  }
  float* part = work + ((long long)bh * ns + c) * kPartFloats;
  if (g < 2) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 4 * g + r;
      __hip_atomic_store(part + 2 * kRep + row * kHD + 16 * wave + n, acc[r], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
      if (wave == 0 && n == 0) {
        __hip_atomic_store(part + row, m_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(part + kRep + row, s_run[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  // Publication: every wave waits until its own device-coherent stores are acknowledged, the workgroup barrier
  // orders the four waves, then one count per workgroup.  The counter's last incrementer reads the partials with
  // device-coherent loads (an acknowledged agent-scope store is visible to every agent-scope load).
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ uint32_t last;
  if (tid == 0) {
    const uint32_t old = __hip_atomic_fetch_add(counters + bh, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == (uint32_t)ns - 1;
    if (last) __hip_atomic_store(counters + bh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;
  // Combine.  One acquire fence (the partials were published with device-coherent stores before the count), then
  // plain loads, spread over the workgroup so that they are in flight together: chunk maxima and sums to LDS, the
  // chunk weights exp(m_c - m) and 1 / S per row, then out[row][d] = sum_c acc_c[row][d] w_c[row] in chunk order.
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  const float* pbase = work + (long long)bh * ns * kPartFloats;
  for (int i = tid; i < ns * kRep; i += 256) {
    const int cc = i / kRep, row = i - cc * kRep;
    L.cm[cc][row] = pbase[cc * kPartFloats + row];
    L.cs[cc][row] = pbase[cc * kPartFloats + kRep + row];
  }
  __syncthreads();
  if (tid < kRep) {
    const int row = tid;
    const float sink = bf16_to_f32(sk[row]);
    float m = sink;
    for (int cc = 0; cc < ns; ++cc) m = fmaxf(m, L.cm[cc][row]);
    float S = expf(sink - m);
    for (int cc = 0; cc < ns; ++cc) {
      const float mc = L.cm[cc][row];
      const float w = mc == kNegInf ? 0.f : expf(mc - m);
      L.cw[cc][row] = w;
      S += L.cs[cc][row] * w;
    }
    L.fin[row][1] = 1.f / S;
  }
  __syncthreads();
  // Thread tid: outputs 2 tid, 2 tid + 1 (row tid / 32); the partials are read 32 chunks at a time with every load
  // issued before the first use, so the combine costs one round trip per 32 chunks, not one per few chunks.
  {
    const int i = 2 * tid, row = i / kHD;
    float o0 = 0.f, o1 = 0.f;
    for (int cb = 0; cb < ns; cb += 32) {              // uniform; ns <= 64
      float2 v[32];
#pragma unroll
      for (int j = 0; j < 32; ++j)
        v[j] = cb + j < ns ? *reinterpret_cast<const float2*>(pbase + (cb + j) * kPartFloats + 2 * kRep + i)
                           : make_float2(0.f, 0.f);
#pragma unroll
      for (int j = 0; j < 32; ++j) {
        if (cb + j < ns) {
          const float w = L.cw[cb + j][row];
          o0 += v[j].x * w;
          o1 += v[j].y * w;
        }
      }
    }
    const float inv = L.fin[row][1];
    *reinterpret_cast<uint32_t*>(orow + i) = (uint32_t)f32_to_bf16(o0 * inv) | ((uint32_t)f32_to_bf16(o1 * inv) << 16);
  }
}

}  // namespace na

using namespace na;

extern "C" {

long long na_attn_workspace_floats(int B, int n_split) {
  if (B <= 0 || n_split <= 0 || n_split > kAttnMaxSplit) return -1;
  return (long long)B * kNKV * n_split * kPartFloats;
}

int na_decode_attention(const void* q, const void* kc, const void* vc, long long cache_rows, const void* sinks,
                        const int64_t* pos, void* out, int B, float scaling, int window, int ring, int n_split,
                        float* work, unsigned int* counters, void* const* events, hipStream_t stream) {
  if (!q || !kc || !vc || !sinks || !pos || !out || B <= 0 || cache_rows <= 0) return kErrArgs;
  if (n_split <= 0 || n_split > kAttnMaxSplit || window < 0 || ring < 0) return kErrArgs;
  if (ring > 0 && (window <= 0 || ring < window || cache_rows != ring)) return kErrArgs;
  if (n_split > 1 && (!work || !counters)) return kErrArgs;
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(kc) | reinterpret_cast<uintptr_t>(vc)) & 15)
    return kErrArgs;
  const dim3 grid((unsigned)(B * kNKV * n_split)), block(256);
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  if (e0 || e1)
    hipExtLaunchKernelGGL(k_decode_attn, grid, block, 0, stream, e0, e1, 0, (const uint16_t*)q, (const uint16_t*)kc,
                          (const uint16_t*)vc, cache_rows, (const uint16_t*)sinks, pos, (uint16_t*)out, scaling,
                          window, ring, n_split, work, (uint32_t*)counters);
  else
    hipLaunchKernelGGL(k_decode_attn, grid, block, 0, stream, (const uint16_t*)q, (const uint16_t*)kc,
                       (const uint16_t*)vc, cache_rows, (const uint16_t*)sinks, pos, (uint16_t*)out, scaling, window,
                       ring, n_split, work, (uint32_t*)counters);
  return hipGetLastError() == hipSuccess ? kOk : kErrLaunch;
}

}  // extern "C"
