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
#include "attention_dev.h"

#include <hip/hip_ext.h>

namespace na {

__global__ __launch_bounds__(256) void k_decode_attn(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
    long long cache_rows, const uint16_t* __restrict__ sinks, const int64_t* __restrict__ pos_p,
    uint16_t* __restrict__ out, float scaling, int window, int ring, int ns, float* __restrict__ work,
    uint32_t* __restrict__ counters) {
  __shared__ AttnLds L;
  args_at_entry(q, kc, vc, cache_rows, sinks, pos_p, out, scaling, window, ring, ns, work, counters);
  decode_attn_body<false>(L, blockIdx.x, q, kc, vc, cache_rows, sinks, pos_p, out, scaling, window, ring, ns, work,
                          counters, AttnHandoff{nullptr, nullptr, 0, nullptr});
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
