// r3c_probe.hip -- MFMA shape throughput probe (measurement only; no
// counterpart in the reference).  Every wave issues `iters` rounds of NACC
// independent MFMAs of one shape on register operands, so the matrix pipe
// never waits on a result: the achieved rate is the shape's issue rate.
//   shape 0: v_mfma_f32_32x32x16_bf16 (32768 flops), 4 accumulators
//   shape 1: v_mfma_f32_16x16x32_bf16 (16384 flops), 8 accumulators
// The accumulators' sum is written per lane so the work is not removed.
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

typedef __attribute__((ext_vector_type(4))) float f32x4v;

__global__ __launch_bounds__(256) void mfma_probe_32(int iters, float* out) {
  const uint32_t t = threadIdx.x + 1;
  const uint4 av = make_uint4(0x3F803F80u ^ t, 0x3F803F80u, 0x3F803F80u + t, 0x3F803F80u);
  const uint4 bv = make_uint4(0x3F803F80u, 0x3F803F80u ^ (t << 3), 0x3F803F80u, 0x3F803F80u);
  f32x16_t acc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[k][e] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) acc[k] = mfma32<bf16_tag>(av, bv, acc[k]);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += acc[k][e];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

__global__ __launch_bounds__(256) void mfma_probe_16(int iters, float* out) {
  const uint32_t t = threadIdx.x + 1;
  const uint4 av = make_uint4(0x3F803F80u ^ t, 0x3F803F80u, 0x3F803F80u + t, 0x3F803F80u);
  const uint4 bv = make_uint4(0x3F803F80u, 0x3F803F80u ^ (t << 3), 0x3F803F80u, 0x3F803F80u);
  f32x4v acc[8];
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[k][e] = 0.f;
  for (int i = 0; i < iters; ++i) {
#pragma unroll
    for (int k = 0; k < 8; ++k)
      acc[k] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, av), __builtin_bit_cast(bf16x8_t, bv),
                                                       acc[k], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) s += acc[k][e];
  out[(size_t)blockIdx.x * 256 + threadIdx.x] = s;
}

}  // namespace

void launch_mfma_probe(int shape, int blocks, int iters, float* out, hipStream_t s) {
  if (shape == 0) hipLaunchKernelGGL(mfma_probe_32, dim3(blocks), dim3(256), 0, s, iters, out);
  else hipLaunchKernelGGL(mfma_probe_16, dim3(blocks), dim3(256), 0, s, iters, out);
}

}  // namespace r3c
