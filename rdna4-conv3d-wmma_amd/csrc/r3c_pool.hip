// r3c_pool.hip -- MaxPool3d(kernel 2, stride 2) forward and backward for the
// UNet3D down path the reference accelerates (reference
// benches/unet_e2e.py:27-37, nn.MaxPool3d(2)), on NCDHW planes.
//
// Forward: y = max over each 2x2x2 window, and a one-byte index per output
// (kd * 4 + kh * 2 + kw of the maximum) instead of PyTorch's 64-bit flat
// index.  The maximum is that of PyTorch's CPU kernel: starting from -inf at
// the window's first element, each element in (kd, kh, kw) order that is
// greater than the running maximum, or NaN, replaces it (so the last NaN
// wins, and a window of -inf keeps index 0).
// Backward: every input element receives dy of its window where it is the
// window's maximum, else 0; optionally plus the element of a second gradient
// of x (the skip connection's), added in fp32 and rounded once -- what
// autograd's sum of the two gradients computes, without a pass of its own.
//
// One thread covers 4 consecutive outputs along w: 8 inputs of each of the 4
// (kd, kh) rows of their windows, as 16-byte vectors (two for fp32).
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

template <int DT>
struct PoolElem;
template <>
struct PoolElem<DT_BF16> {
  __device__ __forceinline__ static void load8(const void* p, int64_t i, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = to_f32<bf16_tag>((uint16_t)(w[e] & 0xffff));
      v[2 * e + 1] = to_f32<bf16_tag>((uint16_t)(w[e] >> 16));
    }
  }
  __device__ __forceinline__ static uint16_t cvt(float v) { return from_f32<bf16_tag>(v); }
};
template <>
struct PoolElem<DT_F16> {
  __device__ __forceinline__ static void load8(const void* p, int64_t i, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = to_f32<f16_tag>((uint16_t)(w[e] & 0xffff));
      v[2 * e + 1] = to_f32<f16_tag>((uint16_t)(w[e] >> 16));
    }
  }
  __device__ __forceinline__ static uint16_t cvt(float v) { return from_f32<f16_tag>(v); }
};
template <>
struct PoolElem<DT_F32> {
  __device__ __forceinline__ static void load8(const void* p, int64_t i, float* v) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
};

// Output coordinates of thread t: (n, c, od, oh, ow0) with ow0 a multiple of 4.
struct PoolPos {
  int n, c, od, oh, ow0;
};
__device__ __forceinline__ bool pool_pos(const PoolArgs& a, int64_t t, PoolPos& p) {
  const int ow4 = a.ow >> 2;
  const int64_t total = (int64_t)a.n * a.c * a.od * a.oh * ow4;
  if (t >= total) return false;
  p.ow0 = (int)(t % ow4) * 4;
  t /= ow4;
  p.oh = (int)(t % a.oh);
  t /= a.oh;
  p.od = (int)(t % a.od);
  t /= a.od;
  p.c = (int)(t % a.c);
  p.n = (int)(t / a.c);
  return true;
}

template <int DT>
__global__ __launch_bounds__(256) void maxpool2_fwd_kernel(const PoolArgs a) {
  PoolPos p;
  if (!pool_pos(a, (int64_t)blockIdx.x * 256 + threadIdx.x, p)) return;
  const int64_t xb = (int64_t)p.n * a.xs0 + (int64_t)p.c * a.xs1 + (int64_t)(2 * p.od) * a.h * a.w +
                     (int64_t)(2 * p.oh) * a.w + 2 * p.ow0;
  float m[4];
  int k[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m[j] = -__builtin_inff();
    k[j] = 0;
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {  // r = kd * 2 + kh
    float v[8];
    PoolElem<DT>::load8(a.x, xb + (int64_t)(r >> 1) * a.h * a.w + (int64_t)(r & 1) * a.w, v);
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int kw = 0; kw < 2; ++kw) {
        const float val = v[2 * j + kw];
        if (val > m[j] || __builtin_isnan(val)) {
          m[j] = val;
          k[j] = r * 2 + kw;
        }
      }
  }
  const int64_t yb = (int64_t)p.n * a.ys0 + (int64_t)p.c * a.ys1 + ((int64_t)p.od * a.oh + p.oh) * a.ow + p.ow0;
  if constexpr (DT == DT_F32) {
    *reinterpret_cast<float4*>(static_cast<float*>(a.y) + yb) = make_float4(m[0], m[1], m[2], m[3]);
  } else {
    typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
    const u32x2 o = {pack2(PoolElem<DT>::cvt(m[0]), PoolElem<DT>::cvt(m[1])),
                     pack2(PoolElem<DT>::cvt(m[2]), PoolElem<DT>::cvt(m[3]))};
    *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(a.y) + yb) = o;
  }
  const int64_t ib = ((((int64_t)p.n * a.c + p.c) * a.od + p.od) * a.oh + p.oh) * a.ow + p.ow0;
  *reinterpret_cast<uint32_t*>(a.idx + ib) =
      (uint32_t)k[0] | ((uint32_t)k[1] << 8) | ((uint32_t)k[2] << 16) | ((uint32_t)k[3] << 24);
}

template <int DT>
__global__ __launch_bounds__(256) void maxpool2_bwd_kernel(const PoolArgs a) {
  PoolPos p;
  if (!pool_pos(a, (int64_t)blockIdx.x * 256 + threadIdx.x, p)) return;
  const int64_t yb = (int64_t)p.n * a.ys0 + (int64_t)p.c * a.ys1 + ((int64_t)p.od * a.oh + p.oh) * a.ow + p.ow0;
  float g[4];
  if constexpr (DT == DT_F32) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(a.dy) + yb);
    g[0] = q.x; g[1] = q.y; g[2] = q.z; g[3] = q.w;
  } else {
    typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
    const u32x2 q = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(a.dy) + yb);
    const uint16_t h[4] = {(uint16_t)(q.x & 0xffff), (uint16_t)(q.x >> 16), (uint16_t)(q.y & 0xffff),
                           (uint16_t)(q.y >> 16)};
#pragma unroll
    for (int j = 0; j < 4; ++j) g[j] = DT == DT_BF16 ? to_f32<bf16_tag>(h[j]) : to_f32<f16_tag>(h[j]);
  }
  const int64_t ib = ((((int64_t)p.n * a.c + p.c) * a.od + p.od) * a.oh + p.oh) * a.ow + p.ow0;
  const uint32_t kk = *reinterpret_cast<const uint32_t*>(a.idx + ib);
  const int64_t xb = (int64_t)p.n * a.xs0 + (int64_t)p.c * a.xs1 + (int64_t)(2 * p.od) * a.h * a.w +
                     (int64_t)(2 * p.oh) * a.w + 2 * p.ow0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float v[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int k = (int)((kk >> (8 * j)) & 255);
#pragma unroll
      for (int kw = 0; kw < 2; ++kw) v[2 * j + kw] = k == r * 2 + kw ? g[j] : 0.f;
    }
    const int64_t o = xb + (int64_t)(r >> 1) * a.h * a.w + (int64_t)(r & 1) * a.w;
    if (a.add) {  // dx = routed gradient + add, one rounding (as an add of the two tensors)
      const int64_t ao = (int64_t)p.n * a.as0 + (int64_t)p.c * a.as1 + (o - ((int64_t)p.n * a.xs0 + (int64_t)p.c * a.xs1));
      if constexpr (DT == DT_F32) {
        const float* q = static_cast<const float*>(a.add) + ao;
        const float4 u0 = *reinterpret_cast<const float4*>(q), u1 = *reinterpret_cast<const float4*>(q + 4);
        v[0] += u0.x; v[1] += u0.y; v[2] += u0.z; v[3] += u0.w;
        v[4] += u1.x; v[5] += u1.y; v[6] += u1.z; v[7] += u1.w;
      } else {
        const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(a.add) + ao);
        const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t lo = (uint16_t)(qw[e] & 0xffff), hi = (uint16_t)(qw[e] >> 16);
          v[2 * e] += DT == DT_BF16 ? to_f32<bf16_tag>(lo) : to_f32<f16_tag>(lo);
          v[2 * e + 1] += DT == DT_BF16 ? to_f32<bf16_tag>(hi) : to_f32<f16_tag>(hi);
        }
      }
    }
    if constexpr (DT == DT_F32) {
      float* d = static_cast<float*>(a.dx) + o;
      *reinterpret_cast<float4*>(d) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(d + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = pack2(PoolElem<DT>::cvt(v[2 * e]), PoolElem<DT>::cvt(v[2 * e + 1]));
      *reinterpret_cast<uint4*>(static_cast<uint16_t*>(a.dx) + o) = make_uint4(w[0], w[1], w[2], w[3]);
    }
  }
}

int64_t pool_blocks(const PoolArgs& a) {
  const int64_t total = (int64_t)a.n * a.c * a.od * a.oh * (a.ow >> 2);
  return (total + 255) / 256;
}

}  // namespace

void launch_maxpool2_fwd(int dtype, const PoolArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)pool_blocks(a));
  if (dtype == DT_BF16) hipLaunchKernelGGL(maxpool2_fwd_kernel<DT_BF16>, grid, dim3(256), 0, s, a);
  else if (dtype == DT_F16) hipLaunchKernelGGL(maxpool2_fwd_kernel<DT_F16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(maxpool2_fwd_kernel<DT_F32>, grid, dim3(256), 0, s, a);
}

void launch_maxpool2_bwd(int dtype, const PoolArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)pool_blocks(a));
  if (dtype == DT_BF16) hipLaunchKernelGGL(maxpool2_bwd_kernel<DT_BF16>, grid, dim3(256), 0, s, a);
  else if (dtype == DT_F16) hipLaunchKernelGGL(maxpool2_bwd_kernel<DT_F16>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(maxpool2_bwd_kernel<DT_F32>, grid, dim3(256), 0, s, a);
}

}  // namespace r3c
