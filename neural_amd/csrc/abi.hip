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

// One v_mfma_f32_16x16x32_bf16 with A[m][k] = a_in[m * 32 + k], B[k][n] = b_in[k * 16 + n] (bf16 bits) under the
// operand layout the tile kernels assume: lane l holds A[l % 16][8 (l / 16) + 0..7], B[8 (l / 16) + 0..7][l % 16] and
// receives D[4 (l / 16) + r][l % 16], r = 0..3.  d_out[m * 16 + n] = D[m][n].
__global__ void k_selftest_mfma(const uint16_t* a_in, const uint16_t* b_in, float* d_out) {
  const int l = threadIdx.x, m = l % 16, q = l / 16;
  bf16x8_t a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = __builtin_bit_cast(__bf16, a_in[m * 32 + 8 * q + i]);
    b[i] = __builtin_bit_cast(__bf16, b_in[(8 * q + i) * 16 + m]);
  }
  f32x4_t c = {0.f, 0.f, 0.f, 0.f};
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  for (int r = 0; r < 4; ++r) d_out[(4 * q + r) * 16 + m] = c[r];
}

// out_hw[i] = bf16 bits of in[i] through the kernels' conversion (f32_to_bf16, and pack_bf16x2 for the pair
// (in[i & ~1], in[i | 1])); out_int[i] = the integer round-to-nearest-even reference.
__global__ void k_selftest_bf16(const float* __restrict__ in, uint16_t* __restrict__ out_hw,
                                uint16_t* __restrict__ out_pk, uint16_t* __restrict__ out_int, long long n) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float f = in[i];
  out_hw[i] = f32_to_bf16(f);
  out_int[i] = f32_to_bf16_int(f);
  const long long p = i & ~1ll;
  if (p + 1 < n) {
    const uint32_t w = pack_bf16x2(in[p], in[p + 1]);
    out_pk[i] = (uint16_t)(i & 1 ? w >> 16 : w & 0xffff);
  } else {
    out_pk[i] = f32_to_bf16(f);
  }
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

// D = A x B for A [16, 32], B [32, 16] bf16 (row-major), D [16, 16] fp32, through the tile kernels' MFMA layout.
int na_selftest_mfma(const void* a, const void* b, float* d, hipStream_t stream) {
  if (!a || !b || !d) return na::kErrArgs;
  hipLaunchKernelGGL(na::k_selftest_mfma, dim3(1), dim3(64), 0, stream, (const uint16_t*)a, (const uint16_t*)b, d);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

// Conversion self-check: n floats -> three uint16 arrays (hardware single, hardware pair, integer reference).
int na_selftest_bf16(const float* in, void* out_hw, void* out_pk, void* out_int, long long n, hipStream_t stream) {
  if (!in || !out_hw || !out_pk || !out_int || n <= 0) return na::kErrArgs;
  const long long blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffll) return na::kErrTooLarge;
  hipLaunchKernelGGL(na::k_selftest_bf16, dim3((unsigned)blocks), dim3(256), 0, stream, in, (uint16_t*)out_hw,
                     (uint16_t*)out_pk, (uint16_t*)out_int, n);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

}  // extern "C"
