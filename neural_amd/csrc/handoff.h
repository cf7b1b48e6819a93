// Handoffs between the phases of one launch on gfx950: producer workgroups and the consumer workgroups that read
// their results run in the same grid, every consumer at a higher workgroup id than every producer it waits for.
//
// * Data crosses workgroups (and XCDs, whose L2 caches are not coherent with each other for ordinary device
//   memory) through agent-scope relaxed atomic stores, which gfx950 issues with the sc1 bit (written through to the
//   coherent point), and agent-scope loads (sc1).  A kernel boundary leaves no stale line in any L2, so what nothing
//   in the launch read before can also be read with ordinary loads once it is complete.
// * Tagged words (the attention block, core.hip; the single-launch expert body, tiles.hip): each 64-bit word holds
//   a 32-bit payload and the launch's generation number, written by one store; the consumer polls the words it
//   needs until they carry its number.  No acknowledgement, count or flag stands between the producer's store and
//   the consumer's read.  One thread per awaited producer polls a single word first (with a short sleep between
//   reads), so that waiting workgroups do not flood the memory system with reads of whole areas.
// * Last-arriver counts (the attention's chunks, attention_dev.h): after its stores are acknowledged (s_waitcnt 0)
//   a workgroup increments its group's counter; the one that completes it reads the others' results.
// * Progress: the hardware dispatches a grid's workgroups in increasing id order on each XCD, so every producer
//   has been dispatched before any consumer that waits for it, and producers never wait for consumers: every wait
//   ends.  The waits are bounded anyway: after kSpinLimit polls the workgroup raises an error flag the host can
//   read and goes on with whatever the buffers hold, so a broken assumption shows up as a flagged wrong result,
//   never as a hung GPU.
#pragma once
#include "common.h"

namespace na {

constexpr uint32_t kSpinLimit = 1u << 16;   // polls (about 1 us each) before a wait gives up
constexpr int kLine = 64;                    // uint32 words per 256-byte line

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
// Dword 3 of a gfx9 buffer resource for raw (stride 0) 32-bit loads: DATA_FORMAT = 32 bit.  Such a load checks its
// offset against the resource's byte count and reads 0 past it.  Cache policy 16 = sc1: a device-coherent load.
constexpr int kBufDword3 = 0x00020000;
constexpr int kBufSc1 = 16;
// ---- tagged words: a 64-bit word holds a 32-bit payload (low half) and the generation number of the launch that
// wrote it (high half), written by one 64-bit device-coherent store and read by one 64-bit device-coherent load, so
// a reader that sees its launch's number sees that launch's payload.  Every word of a tagged area is written once
// per launch; a launch's number differs from the previous launch's (it is advanced by one per launch), so the area
// needs no clearing and the producer no acknowledgement, count or flag: the consumer polls the data itself.
NA_DEVICE void tag_store(uint64_t* p, uint32_t payload, uint32_t gen) {
  __hip_atomic_store(p, ((uint64_t)gen << 32) | payload, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
NA_DEVICE uint64_t tag_load(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
NA_DEVICE bool tag_is(uint64_t w, uint32_t gen) { return (uint32_t)(w >> 32) == gen; }
// A launch's number from the generation word as loaded at entry (raw + 1).  Call it where the number is first needed:
// the empty asm keeps the compiler from moving the addition, and with it the wait for that load, to the kernel's
// start, ahead of the loads a phase issues first.
NA_DEVICE uint32_t launch_tag(uint32_t raw) {
  asm volatile("" : "+v"(raw));
  return raw + 1u;
}

// One thread: poll *p (a short sleep between reads) until it carries gen, or raise *err after kSpinLimit polls.
NA_DEVICE void tag_wait1(const uint64_t* p, uint32_t gen, uint32_t* err) {
  uint32_t polls = 0;
  while (!tag_is(tag_load(p), gen)) {
    if (++polls > kSpinLimit) {
      __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// The payloads of the N words *p[0] .. *p[N - 1]: all loaded at once, then the ones not yet carrying gen polled
// again with device-coherent loads (bounded as above).  CACHED: the first loads are ordinary ones (64-bit, so still
// single-copy atomic), which an XCD's L2 serves once one of its workgroups has fetched the line: for words that
// many workgroups read.  A line fetched before all its words were written holds older tags, so those words are
// polled again device-coherently: a stale copy costs a round trip, never a wrong payload.
template <int N, bool CACHED = false>
NA_DEVICE void tag_read_at(const uint64_t* const (&p)[N], uint32_t gen, uint32_t (&out)[N], uint32_t* err) {
  uint64_t w[N];
#pragma unroll
  for (int k = 0; k < N; ++k)
    w[k] = CACHED ? __hip_atomic_load(p[k], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) : tag_load(p[k]);
  uint32_t polls = 0;
  for (;;) {
    bool ok = true;
#pragma unroll
    for (int k = 0; k < N; ++k) ok = ok && tag_is(w[k], gen);
    if (ok) break;
    if (++polls > kSpinLimit) {
      __hip_atomic_fetch_or(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
#pragma unroll
    for (int k = 0; k < N; ++k)
      if (!tag_is(w[k], gen)) w[k] = tag_load(p[k]);
  }
#pragma unroll
  for (int k = 0; k < N; ++k) out[k] = (uint32_t)w[k];
}
// ... of the N consecutive words p[0 .. N - 1].
template <int N, bool CACHED = false>
NA_DEVICE void tag_read(const uint64_t* p, uint32_t gen, uint32_t (&out)[N], uint32_t* err) {
  const uint64_t* q[N];
#pragma unroll
  for (int k = 0; k < N; ++k) q[k] = p + k;
  tag_read_at<N, CACHED>(q, gen, out, err);
}

}  // namespace na
