// Library identity and device self-checks of the gfx950 conversion builtins the kernels rely on.
#include "common.h"

namespace na {

// out[2 * b + i] = bf16 bits of element i (0 = low nibble) of byte b, through the same helper the GEMV kernels use.
__global__ void k_selftest_fp4(uint16_t* out) {
  const int b = threadIdx.x;   // 256 threads, one byte value each
  const uint32_t word = (uint32_t)b * 0x01010101u;   // the byte in every position: check all four selectors
  const uint32_t p0 = fp4x2_to_bf16x2<0>(word), p1 = fp4x2_to_bf16x2<1>(word);
  const uint32_t p2 = fp4x2_to_bf16x2<2>(word), p3 = fp4x2_to_bf16x2<3>(word);
  const bool same = p0 == p1 && p1 == p2 && p2 == p3;
  out[2 * b] = (uint16_t)(p0 & 0xffff);
  out[2 * b + 1] = (uint16_t)(p0 >> 16);
  out[512 + b] = same ? 1 : 0;
}

}  // namespace na

extern "C" {

int na_version(void) { return 1; }

// Writes 768 uint16: [0, 512) the bf16 decode of every byte (low nibble first), [512, 768) 1 where all four byte
// selectors of the conversion builtin agree.
int na_selftest_fp4(void* out, hipStream_t stream) {
  if (!out) return na::kErrArgs;
  hipLaunchKernelGGL(na::k_selftest_fp4, dim3(1), dim3(256), 0, stream, (uint16_t*)out);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

}  // extern "C"
