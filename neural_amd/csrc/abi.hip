// Library identity and device self-checks of the gfx950 conversion builtins and MFMA operand orders the kernels use.
#include "common.h"
#include "t950.h"

#include <hip/hip_ext.h>

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

// One row of 2880 bf16 per workgroup (384 threads: chunk c = thread, threads past 360 quantise zeros) through the
// decode kernels' activation quantiser: hi[r][i], lo[r][i] = the E4M3 codes of element i, sc[r][0][b], sc[r][1][b] =
// the E8M0 bytes of block b for hi and lo.
__global__ __launch_bounds__(384) void k_selftest_x8(const uint16_t* __restrict__ in, uint8_t* __restrict__ hi,
                                                     uint8_t* __restrict__ lo, uint8_t* __restrict__ sc) {
  const int r = blockIdx.x, c = threadIdx.x;
  const uint4 v =
      c < kChunks ? *reinterpret_cast<const uint4*>(in + (long long)r * kH + 8 * c) : make_uint4(0, 0, 0, 0);
  uint2 h, l;
  uint32_t sh, sl;
  x8_quant_chunk(v, h, l, sh, sl);
  if (c < kChunks) {
    *reinterpret_cast<uint2*>(hi + (long long)r * kH + 8 * c) = h;
    *reinterpret_cast<uint2*>(lo + (long long)r * kH + 8 * c) = l;
    if ((c & 3) == 0) {
      sc[(long long)r * 2 * kGK + (c >> 2)] = (uint8_t)sh;
      sc[(long long)r * 2 * kGK + kGK + (c >> 2)] = (uint8_t)sl;
    }
  }
}

// One v_mfma_scale_f32_16x16x128_f8f6f4 in the decode kernels' operand order: A = E4M3 codes a[m][k] (16 x 128 bytes)
// with E8M0 bytes sa[m][kb] (16 x 4); B = one full t950 k-tile (1024 bytes: lane 16 kb + n holds the 16 code bytes of
// group kb of row n), as loaded, with E8M0 bytes sb[n][kb] (16 x 4).  d[m * 16 + n] = D[m][n].
__global__ void k_selftest_mfma8(const uint8_t* __restrict__ a, const uint8_t* __restrict__ sa,
                                 const uint8_t* __restrict__ tile, const uint8_t* __restrict__ sb,
                                 float* __restrict__ d) {
  const int l = threadIdx.x, kb = l >> 4, m = l & 15;
  const uint4 a0 = *reinterpret_cast<const uint4*>(a + m * 128 + 16 * kb);
  const uint4 a1 = *reinterpret_cast<const uint4*>(a + m * 128 + 64 + 16 * kb);
  const uint4 c = *reinterpret_cast<const uint4*>(tile + 16 * l);
  const mfma_i32x8_t A = {(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
  const mfma_i32x8_t Bv = {(int)c.x, (int)c.y, (int)c.z, (int)c.w, 0, 0, 0, 0};
  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(A, Bv, acc, 0, 4, 0, (int)sa[m * 4 + kb], 0,
                                                        (int)sb[m * 4 + kb]);
  for (int r = 0; r < 4; ++r) d[(4 * kb + r) * 16 + m] = acc[r];
}


// Matrix-core rate probe: every wave runs `iters` rounds of 4 independent MFMAs on register operands, kind 0 the
// block-scaled v_mfma_scale_f32_16x16x128_f8f6f4 with E4M3 A and E2M1 B (the instruction of the decode and prefill
// expert kernels), kind 1 v_mfma_f32_16x16x32_bf16 (the prompt attention's).  Operands are constant ones (E4M3 0x38,
// E2M1 0x2, bf16 1.0, E8M0 127), so the accumulators stay finite; out[wave] = their sum keeps every MFMA live.
// Flops per MFMA: 2 x 16 x 16 x 128 (kind 0), 2 x 16 x 16 x 32 (kind 1).
template <int KIND>
__global__ __launch_bounds__(256) void k_mfma_rate(int iters, float* __restrict__ out) {
  f32x4_t acc[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  if constexpr (KIND == 0) {
    const int one8 = 0x38383838, one4 = 0x22222222;
    const mfma_i32x8_t a = {one8, one8, one8, one8, one8, one8, one8, one8};
    const mfma_i32x8_t b = {one4, one4, one4, one4, 0, 0, 0, 0};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        acc[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc[j], 0, 4, 0, 127, 0, 127);
    }
  } else {
    bf16x8_t a;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = (__bf16)1.0f;
    for (int i = 0; i < iters; ++i) {
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, a, acc[j], 0, 0, 0);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) s += acc[j][0] + acc[j][1] + acc[j][2] + acc[j][3];
  if ((threadIdx.x & 63) == 0) out[blockIdx.x * 4 + (threadIdx.x >> 6)] = s;
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

// Activation quantiser self-check: rows x 2880 bf16 -> hi, lo (rows x 2880 E4M3 codes), sc (rows x 2 x 90 E8M0).
int na_selftest_x8(const void* in, int rows, void* hi, void* lo, void* sc, hipStream_t stream) {
  if (!in || !hi || !lo || !sc || rows <= 0) return na::kErrArgs;
  hipLaunchKernelGGL(na::k_selftest_x8, dim3(rows), dim3(384), 0, stream, (const uint16_t*)in, (uint8_t*)hi,
                     (uint8_t*)lo, (uint8_t*)sc);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

// D = A x B through the decode kernels' block-scaled MFMA and t950 operand rearrangement (see k_selftest_mfma8).
int na_selftest_mfma8(const void* a, const void* sa, const void* tile, const void* sb, float* d, hipStream_t stream) {
  if (!a || !sa || !tile || !sb || !d) return na::kErrArgs;
  hipLaunchKernelGGL(na::k_selftest_mfma8, dim3(1), dim3(64), 0, stream, (const uint8_t*)a, (const uint8_t*)sa,
                     (const uint8_t*)tile, (const uint8_t*)sb, d);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

int na_bench_mfma_rate(int kind, int blocks, int iters, float* out, void* const* events, hipStream_t stream) {
  if ((kind != 0 && kind != 1) || blocks <= 0 || iters <= 0 || !out) return na::kErrArgs;
  hipEvent_t e0 = events ? (hipEvent_t)events[0] : nullptr, e1 = events ? (hipEvent_t)events[1] : nullptr;
  auto kern = kind == 0 ? na::k_mfma_rate<0> : na::k_mfma_rate<1>;
  if (e0 || e1)
    hipExtLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, stream, e0, e1, 0, iters, out);
  else
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), 0, stream, iters, out);
  return hipGetLastError() == hipSuccess ? na::kOk : na::kErrLaunch;
}

}  // extern "C"
