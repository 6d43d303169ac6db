// Register-only matrix-core rate probe for MI355X (gfx950), used by bench.py
// to report the sustained MFMA rate of the box it runs on beside the update
// kernel's.  It has no counterpart in the reference and is not part of the
// attention path: a measurement of the hardware, nothing more.
//
// Each workgroup has 8 wavefronts (two per SIMD, as the update kernel); each
// wave issues independent v_mfma_f32_16x16x32_bf16 on operands held in
// registers (seeded pseudo-random bf16 values, so the matrix cores switch as
// they do on real data), with no memory traffic and no other VALU work in the
// loop.  The only store is one float per thread, so the MFMAs are not
// removed; the output buffer holds exactly one float per launched thread.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "seqattn_probe.h"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 512;
constexpr int kBlocks = 256 * 8;  // 8 rounds of one workgroup per CU
constexpr int kIters = 2048;      // 24 MFMAs per wave per iteration

__device__ inline uint32_t mix(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

__device__ inline __bf16 unit(uint32_t x) { return (__bf16)((float)(mix(x) & 0xffffu) / 32768.f - 1.f); }

__global__ __launch_bounds__(kThreads) void mfma_rate_kernel(float* out, uint32_t seed) {
  const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
  bf16x8 a[4], b[3];
  for (int r = 0; r < 4; ++r)
    for (int i = 0; i < 8; ++i) a[r][i] = unit(seed ^ (t * 64u + r * 8u + i));
  for (int r = 0; r < 3; ++r)
    for (int i = 0; i < 8; ++i) b[r][i] = unit(~seed ^ (t * 64u + r * 8u + i));
  f32x4 c[8][3] = {};
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int x = 0; x < 8; ++x)
#pragma unroll
      for (int y = 0; y < 3; ++y) c[x][y] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[x & 3], b[y], c[x][y], 0, 0, 0);
  }
  float s = 0.f;
  for (int x = 0; x < 8; ++x)
    for (int y = 0; y < 3; ++y) s += c[x][y][0] + c[x][y][1] + c[x][y][2] + c[x][y][3];
  out[t] = s;
}

}  // namespace

extern "C" {

int64_t sa_probe_mfma_out_elems(void) { return (int64_t)kBlocks * kThreads; }

double sa_probe_mfma_flop_per_launch(void) {
  return (double)kBlocks * (kThreads / 64) * kIters * 24 * (16.0 * 16.0 * 32.0 * 2.0);
}

int32_t sa_probe_mfma(float* out, int64_t out_elems, int32_t launches, uint32_t seed, void* stream) {
  if (out == nullptr || out_elems < sa_probe_mfma_out_elems() || launches < 0) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int32_t i = 0; i < launches; ++i) {
    mfma_rate_kernel<<<kBlocks, kThreads, 0, s>>>(out, seed + (uint32_t)i);
    if (hipGetLastError() != hipSuccess) return -2;
  }
  return 0;
}

}  // extern "C"
