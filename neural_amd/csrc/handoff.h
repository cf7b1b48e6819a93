// Handoffs between the phases of one launch on gfx950: producer workgroups and the consumer workgroups that read
// their results run in the same grid, every consumer at a higher workgroup id than every producer it waits for.
//
// * Data crosses workgroups (and XCDs, whose L2 caches are not coherent with each other for ordinary device
//   memory) through agent-scope relaxed atomic stores, which gfx950 issues with the sc1 bit (written through to the
//   coherent point).  A consumer reads with agent-scope atomic loads (sc1) what the launch read before the handoff
//   (an L2 could hold the old bytes), and with ordinary loads what nothing in the launch read before: a kernel
//   boundary leaves no stale line in any L2, so an XCD's first read fetches the final bytes and the L2 serves the
//   rest.
// * Completion: after its stores are acknowledged (s_waitcnt 0) and the workgroup's waves meet at a barrier, one
//   thread counts the workgroup (two-level counters, publish_done); the workgroup that completes the count raises
//   the phase's release flags, kGo words on separate 256-byte lines; a consumer polls the flag of its group (thread
//   0, a short sleep between reads), then the workgroup meets at a barrier.  Hundreds of consumers polling one word,
//   or hundreds of producers incrementing one, would queue every access to that line; spread over kGo lines they
//   do not.
// * Progress: the hardware dispatches a grid's workgroups in increasing id order on each XCD, so every producer
//   has been dispatched before any consumer that waits for it, and producers never wait for consumers: every wait
//   ends.  The wait is bounded anyway: after kSpinLimit polls the workgroup raises an error flag the host can read
//   and goes on with whatever the buffers hold, so a broken assumption shows up as a flagged wrong result, never as
//   a hung GPU.
// * Counters return themselves to zero; the flags are returned to zero inside the launch by the phase that knows
//   every waiter has passed (see the kernels), so a launch starts from zeros and leaves zeros.
#pragma once
#include "common.h"

namespace na {

constexpr uint32_t kSpinLimit = 1u << 16;   // polls (about 1 us each) before a wait gives up
constexpr int kLine = 64;                    // uint32 words per 256-byte line
constexpr int kGo = 16;                      // release flags per phase

NA_DEVICE void store_coherent(uint16_t* p, uint16_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
NA_DEVICE void store_coherent(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
NA_DEVICE uint32_t load_coherent(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 8 bytes with one device-coherent load (p 8-byte aligned).
NA_DEVICE float2 load8_coherent(const float* p) {
  const uint64_t v = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)));
}
NA_DEVICE float loadf_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// 16 bytes as four coherent dword loads (p 4-byte aligned).
NA_DEVICE uint4 load16_coherent(const void* p) {
  const uint32_t* w = reinterpret_cast<const uint32_t*>(p);
  return make_uint4(load_coherent(w), load_coherent(w + 1), load_coherent(w + 2), load_coherent(w + 3));
}

// Every thread of the workgroup calls it after its last coherent store of the phase (workgroup `blk` of the phase's
// n).  Counting is two-level: workgroup blk counts in group counter cnt[(1 + blk % kGo) * kLine], and the workgroup
// that completes its group counts in the top counter cnt[0]; the one that completes the top (min(n, kGo) groups)
// raises the kGo release flags go[i * kLine].  Hundreds of increments of one word would queue behind each other for
// microseconds; each counter here takes at most ceil(n / kGo).  A counter's last arrival returns it to zero: nobody
// waits on a counter, consumers wait on the flags.
NA_DEVICE void publish_done(uint32_t* cnt, int blk, uint32_t n, uint32_t* go) {
  __shared__ uint32_t completes;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t gi = (uint32_t)blk % kGo;
    const uint32_t quota = (n - gi + kGo - 1) / kGo;
    const uint32_t groups = n < (uint32_t)kGo ? n : (uint32_t)kGo;
    uint32_t* gc = cnt + (1 + gi) * kLine;
    bool top = false;
    if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == quota - 1) {
      __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      top = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == groups - 1;
      if (top) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    completes = top;
  }
  __syncthreads();
  if (completes && threadIdx.x < kGo) store_coherent(go + threadIdx.x * kLine, 1u);
}

// A release by group: every thread of the workgroup calls it after its last coherent store; the workgroup that
// completes the group's n counts in *cnt returns the counter to zero and raises the one flag *go.
NA_DEVICE void publish_group(uint32_t* cnt, uint32_t n, uint32_t* go) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0 && __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == n - 1) {
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    store_coherent(go, 1u);
  }
}

// Every thread of the workgroup calls it; returns when the release flag *go is raised (or the poll limit raised
// *err).
NA_DEVICE void wait_go(const uint32_t* go, uint32_t* err) {
  if (threadIdx.x == 0) {
    uint32_t polls = 0;
    while (load_coherent(go) == 0) {
      if (++polls > kSpinLimit) {
        __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

}  // namespace na
