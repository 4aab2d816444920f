// r3c_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Every matrix product here is v_mfma_f32_32x32x16_{bf16,f16} (wave64, fp32
// accumulate).  Operand layouts (measured on gfx950; lane l, g = l / 32,
// i = l % 32):
//   A (32 x 16): lane holds A[i][8g .. 8g+7]      (8 halves = 4 VGPRs)
//   B (16 x 32): lane holds B[8g .. 8g+7][i]
//   C (32 x 32): acc[4q + r] = C[8q + 4g + r][i]  (16 fp32)
// Any permutation of k applied to both A and B gives the same product, so the
// only contract is the row/column placement above.
//
// ds_read_tr16_b64 (gfx950 transposing LDS read) inside each 16-lane group:
//   out[4a + b][i] = lds16[addr[a + 4i] + b]   (a, b, i in 0..3)
// i.e. four source lanes each read 4 consecutive halves and the result is
// handed out transposed.  Two such reads produce one MFMA operand whose k runs
// over 8 tile rows (positions) while the lanes run over contiguous channels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r3c {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
typedef __attribute__((ext_vector_type(4))) short s16x4_t;
// Plain 128-bit vector: copies of it are register moves, never memcpy through
// private memory (which a copy of the uint4 struct can turn into).
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4_t;
typedef __attribute__((address_space(3))) s16x4_t lds_s16x4_t;

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };

// Element tags: raw 16-bit storage with the arithmetic type chosen at compile time.
struct bf16_tag {
  static constexpr int code = DT_BF16;
  static constexpr uint16_t one = 0x3F80;
};
struct f16_tag {
  static constexpr int code = DT_F16;
  static constexpr uint16_t one = 0x3C00;
};

template <typename T>
__device__ __forceinline__ f32x16_t mfma32(const uint4& a, const uint4& b, const f32x16_t& c);
template <>
__device__ __forceinline__ f32x16_t mfma32<bf16_tag>(const uint4& a, const uint4& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x16_t mfma32<f16_tag>(const uint4& a, const uint4& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b), c,
                                                0, 0, 0);
}

// Round-to-nearest-even conversions (IEEE definition; hardware cvt on gfx950).
template <typename T>
__device__ __forceinline__ uint16_t from_f32(float v);
template <>
__device__ __forceinline__ uint16_t from_f32<bf16_tag>(float v) {
  return __builtin_bit_cast(uint16_t, (__bf16)v);
}
template <>
__device__ __forceinline__ uint16_t from_f32<f16_tag>(float v) {
  return __builtin_bit_cast(uint16_t, (_Float16)v);
}
template <typename T>
__device__ __forceinline__ float to_f32(uint16_t v);
template <>
__device__ __forceinline__ float to_f32<bf16_tag>(uint16_t v) {
  return __builtin_bit_cast(float, ((uint32_t)v) << 16);
}
template <>
__device__ __forceinline__ float to_f32<f16_tag>(uint16_t v) {
  return (float)__builtin_bit_cast(_Float16, v);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// Two transposing LDS reads -> one 8-half MFMA operand.  `p0` / `p1` are this
// lane's source addresses (element index into the LDS tile, 4-element aligned).
__device__ __forceinline__ uint4 lds_tr_pair(const uint16_t* lds, int p0, int p1) {
  const lds_s16x4_t* a0 = (const lds_s16x4_t*)((const __attribute__((address_space(3))) uint16_t*)lds + p0);
  const lds_s16x4_t* a1 = (const lds_s16x4_t*)((const __attribute__((address_space(3))) uint16_t*)lds + p1);
  s16x4_t r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)a0);
  s16x4_t r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t*)a1);
  uint2 u0 = __builtin_bit_cast(uint2, r0);
  uint2 u1 = __builtin_bit_cast(uint2, r1);
  return make_uint4(u0.x, u0.y, u1.x, u1.y);
}

}  // namespace r3c
