// r3c_bn.hip -- BatchNorm3d + ReLU for the conv -> BN -> ReLU blocks of the
// UNet3D the reference accelerates (benches/unet_e2e.py:13-21): training-mode
// batch statistics, the normalise + affine + ReLU pass, and the backward of
// both, on NCDHW tensors (each channel plane of a sample contiguous).
//
// Each pass streams its tensors once through 16-byte vector loads.  Work is
// split into fixed chunks of kBnChunk positions of one (sample, channel) plane;
// every chunk writes its partial result, and a per-channel kernel combines the
// partials in a fixed order, so every result is bitwise reproducible.
//
//   statistics:   chunk -> (mean, M2) of its values (Chan et al.'s pairwise
//                 combination of per-thread sums), channel -> mean, biased
//                 variance, invstd = 1 / sqrt(var + eps), scale = gamma *
//                 invstd, shift = beta - mean * scale, running-stat update
//                 with the unbiased variance (PyTorch's BatchNorm semantics).
//   forward:      z = max(y * scale + shift, 0)
//   backward:     g = dz where y * scale + shift > 0 (ReLU), else 0;
//                 chunk -> (sum g, sum g * xhat), xhat = (y - mean) * invstd;
//                 channel -> dbeta = sum g, dgamma = sum g * xhat and
//                 dy = a g + b y + c with a = scale, b = -scale invstd
//                 sum(g xhat) / M, c = -scale sum(g) / M - b mean (training;
//                 with running statistics b = c = 0).
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

struct f32_tag {
  static constexpr int code = DT_F32;
};

// Element access: VEC elements per 16-byte vector, converted to / from fp32.
template <typename T>
struct BnElem {
  static constexpr int VEC = 8;
  __device__ __forceinline__ static void load(const void* p, int64_t i, float* v) {
    const uint4 q = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p) + i);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[2 * e] = to_f32<T>((uint16_t)(w[e] & 0xffff));
      v[2 * e + 1] = to_f32<T>((uint16_t)(w[e] >> 16));
    }
  }
  __device__ __forceinline__ static void store(void* p, int64_t i, const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) w[e] = pack2(from_f32<T>(v[2 * e]), from_f32<T>(v[2 * e + 1]));
    *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p) + i) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <>
struct BnElem<f32_tag> {
  static constexpr int VEC = 4;
  __device__ __forceinline__ static void load(const void* p, int64_t i, float* v) {
    const float4 q = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    v[0] = q.x;
    v[1] = q.y;
    v[2] = q.z;
    v[3] = q.w;
  }
  __device__ __forceinline__ static void store(void* p, int64_t i, const float* v) {
    *reinterpret_cast<float4*>(static_cast<float*>(p) + i) = make_float4(v[0], v[1], v[2], v[3]);
  }
};

constexpr int kBnThreads = 256;

// (count, mean, M2) of a set of values, combined pairwise (Chan, Golub and
// LeVeque's update); empty sets carry count 0.
struct Moments {
  float n, mean, m2;
};
__device__ __forceinline__ Moments combine(const Moments& a, const Moments& b) {
  if (b.n == 0.f) return a;
  if (a.n == 0.f) return b;
  const float n = a.n + b.n;
  const float d = b.mean - a.mean;
  const float fb = b.n / n;
  return {n, a.mean + d * fb, a.m2 + b.m2 + d * d * a.n * fb};
}

// Fixed-order combination over the 256 threads of a workgroup: a butterfly
// inside each wave (lane shuffles), then the four wave results in wave
// order.  The result is valid in thread 0.
__device__ __forceinline__ Moments block_combine(Moments m, float* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const Moments o{__shfl_xor(m.n, off), __shfl_xor(m.mean, off), __shfl_xor(m.m2, off)};
    m = combine(m, o);
  }
  const int t = threadIdx.x;
  if ((t & 63) == 0) {
    sh[3 * (t >> 6)] = m.n;
    sh[3 * (t >> 6) + 1] = m.mean;
    sh[3 * (t >> 6) + 2] = m.m2;
  }
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int w = 1; w < kBnThreads / 64; ++w) m = combine(m, Moments{sh[3 * w], sh[3 * w + 1], sh[3 * w + 2]});
  }
  return m;
}

__device__ __forceinline__ float2 block_sum2(float2 v, float* sh) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    v.x += __shfl_xor(v.x, off);
    v.y += __shfl_xor(v.y, off);
  }
  const int t = threadIdx.x;
  if ((t & 63) == 0) {
    sh[2 * (t >> 6)] = v.x;
    sh[2 * (t >> 6) + 1] = v.y;
  }
  __syncthreads();
  if (t == 0) {
#pragma unroll
    for (int w = 1; w < kBnThreads / 64; ++w) {
      v.x += sh[2 * w];
      v.y += sh[2 * w + 1];
    }
  }
  return v;
}

// scale and shift of channel c from the saved mean / invstd (the forward's
// own values, so the backward's ReLU mask is the forward's).
__device__ __forceinline__ float2 saved_scale_shift(const BnArgs& a, int c) {
  const float gamma = a.gamma ? a.gamma[c] : 1.f;
  const float beta = a.beta ? a.beta[c] : 0.f;
  const float scale = gamma * a.save_invstd[c];
  return make_float2(scale, beta - a.save_mean[c] * scale);
}

// First element of plane (n, c) of y; thread t owns vectors t, t + 256, ... of a chunk.
template <typename T>
__device__ __forceinline__ int64_t plane_base(const BnArgs& a, int n, int c) {
  return (int64_t)n * a.sn + (int64_t)c * a.sc;
}

// Training statistics, per chunk: (mean, M2) of its values -> part[(n * nchunk + chunk) * C + c].
template <typename T>
__global__ __launch_bounds__(kBnThreads) void bn_stats_kernel(const BnArgs a) {
  __shared__ float sh[3 * (kBnThreads / 64)];
  constexpr int VEC = BnElem<T>::VEC;
  const int chunk = blockIdx.x, c = blockIdx.y, n = blockIdx.z;
  const int64_t s0 = (int64_t)chunk * kBnChunk;
  const int len = (int)min((int64_t)kBnChunk, a.S - s0);
  const int64_t base = plane_base<T>(a, n, c) + s0;
  float sum = 0.f, sq = 0.f, cnt = 0.f;
#pragma unroll 4
  for (int i = threadIdx.x * VEC; i < len; i += kBnThreads * VEC) {
    float v[VEC];
    BnElem<T>::load(a.y, base + i, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      sum += v[e];
      sq = fmaf(v[e], v[e], sq);
    }
    cnt += VEC;
  }
  Moments m{cnt, 0.f, 0.f};
  if (cnt > 0.f) {
    m.mean = sum / cnt;
    m.m2 = fmaxf(sq - sum * m.mean, 0.f);
  }
  m = block_combine(m, sh);
  if (threadIdx.x == 0) {
    float* p = a.part + ((int64_t)(n * a.nchunk + chunk) * a.C + c) * 2;
    p[0] = m.mean;
    p[1] = m.m2;
  }
}

// Per channel: combine the chunks in fixed order; scale / shift for the
// forward, saved mean / invstd for the backward, running statistics.
__global__ __launch_bounds__(kBnThreads) void bn_stats_final_kernel(const BnArgs a) {
  __shared__ float sh[3 * (kBnThreads / 64)];
  const int c = blockIdx.x;
  const int nparts = a.N * a.nchunk;
  Moments m{0.f, 0.f, 0.f};
  for (int i = threadIdx.x; i < nparts; i += kBnThreads) {
    const int chunk = i % a.nchunk;
    const float cnt = (float)min((int64_t)kBnChunk, a.S - (int64_t)chunk * kBnChunk);
    const float* p = a.part + ((int64_t)i * a.C + c) * 2;
    m = combine(m, Moments{cnt, p[0], p[1]});
  }
  m = block_combine(m, sh);
  if (threadIdx.x == 0) {
    const float var = m.m2 / m.n;
    const float invstd = 1.f / sqrtf(var + a.eps);
    const float gamma = a.gamma ? a.gamma[c] : 1.f;
    const float beta = a.beta ? a.beta[c] : 0.f;
    const float scale = gamma * invstd;
    a.coef[4 * c + 0] = scale;
    a.coef[4 * c + 1] = beta - m.mean * scale;
    a.save_mean[c] = m.mean;
    a.save_invstd[c] = invstd;
    if (a.running_mean) {
      const float unbiased = m.n > 1.f ? m.m2 / (m.n - 1.f) : var;
      a.running_mean[c] = (1.f - a.momentum) * a.running_mean[c] + a.momentum * m.mean;
      a.running_var[c] = (1.f - a.momentum) * a.running_var[c] + a.momentum * unbiased;
    }
  }
}

// Running statistics (evaluation): scale / shift and the saved mean / invstd.
__global__ __launch_bounds__(kBnThreads) void bn_eval_coef_kernel(const BnArgs a) {
  const int c = blockIdx.x * kBnThreads + threadIdx.x;
  if (c >= a.C) return;
  const float mean = a.running_mean[c];
  const float invstd = 1.f / sqrtf(a.running_var[c] + a.eps);
  const float gamma = a.gamma ? a.gamma[c] : 1.f;
  const float beta = a.beta ? a.beta[c] : 0.f;
  const float scale = gamma * invstd;
  a.coef[4 * c + 0] = scale;
  a.coef[4 * c + 1] = beta - mean * scale;
  a.save_mean[c] = mean;
  a.save_invstd[c] = invstd;
}

// z = max(y * scale + shift, 0).
template <typename T>
__global__ __launch_bounds__(kBnThreads) void bn_relu_apply_kernel(const BnArgs a) {
  constexpr int VEC = BnElem<T>::VEC;
  const int chunk = blockIdx.x, c = blockIdx.y, n = blockIdx.z;
  const int64_t s0 = (int64_t)chunk * kBnChunk;
  const int len = (int)min((int64_t)kBnChunk, a.S - s0);
  const int64_t base = plane_base<T>(a, n, c) + s0;
  const int64_t obase = (int64_t)n * a.on + (int64_t)c * a.oc + s0;
  const float scale = a.coef[4 * c], shift = a.coef[4 * c + 1];
#pragma unroll 4
  for (int i = threadIdx.x * VEC; i < len; i += kBnThreads * VEC) {
    float v[VEC];
    BnElem<T>::load(a.y, base + i, v);
#pragma unroll
    for (int e = 0; e < VEC; ++e) v[e] = fmaxf(fmaf(v[e], scale, shift), 0.f);
    BnElem<T>::store(a.out, obase + i, v);
  }
}

// Backward sums per chunk: (sum g, sum g * xhat) -> part.
template <typename T>
__global__ __launch_bounds__(kBnThreads) void bn_relu_bwd_sums_kernel(const BnArgs a) {
  __shared__ float sh[2 * (kBnThreads / 64)];
  constexpr int VEC = BnElem<T>::VEC;
  const int chunk = blockIdx.x, c = blockIdx.y, n = blockIdx.z;
  const int64_t s0 = (int64_t)chunk * kBnChunk;
  const int len = (int)min((int64_t)kBnChunk, a.S - s0);
  const int64_t base = plane_base<T>(a, n, c) + s0;
  const int64_t gbase = (int64_t)n * a.gn + (int64_t)c * a.gc + s0;
  const float2 ss = saved_scale_shift(a, c);
  const float scale = ss.x, shift = ss.y;
  const float mean = a.save_mean[c], invstd = a.save_invstd[c];
  float2 acc = make_float2(0.f, 0.f);
#pragma unroll 4
  for (int i = threadIdx.x * VEC; i < len; i += kBnThreads * VEC) {
    float y[VEC], dz[VEC];
    BnElem<T>::load(a.y, base + i, y);
    BnElem<T>::load(a.dz, gbase + i, dz);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float g = fmaf(y[e], scale, shift) > 0.f ? dz[e] : 0.f;
      acc.x += g;
      acc.y = fmaf(g, (y[e] - mean) * invstd, acc.y);
    }
  }
  acc = block_sum2(acc, sh);
  if (threadIdx.x == 0) {
    float* p = a.part + ((int64_t)(n * a.nchunk + chunk) * a.C + c) * 2;
    p[0] = acc.x;
    p[1] = acc.y;
  }
}

// Per channel: dbeta, dgamma and the coefficients of dy = a g + b y + c.
__global__ __launch_bounds__(kBnThreads) void bn_relu_bwd_final_kernel(const BnArgs a) {
  __shared__ float sh[2 * (kBnThreads / 64)];
  const int c = blockIdx.x;
  const int nparts = a.N * a.nchunk;
  float2 acc = make_float2(0.f, 0.f);
  for (int i = threadIdx.x; i < nparts; i += kBnThreads) {
    const float* p = a.part + ((int64_t)i * a.C + c) * 2;
    acc.x += p[0];
    acc.y += p[1];
  }
  acc = block_sum2(acc, sh);
  if (threadIdx.x == 0) {
    if (a.dbeta) a.dbeta[c] = acc.x;
    if (a.dgamma) a.dgamma[c] = acc.y;
    const float scale = saved_scale_shift(a, c).x;
    float b = 0.f, c0 = 0.f;
    if (a.training) {
      const float M = (float)a.N * (float)a.S;
      b = -scale * a.save_invstd[c] * acc.y / M;
      c0 = -scale * acc.x / M - b * a.save_mean[c];
    }
    a.coef[4 * c + 2] = b;
    a.coef[4 * c + 3] = c0;
  }
}

// dy = scale * g + b * y + c.
template <typename T>
__global__ __launch_bounds__(kBnThreads) void bn_relu_bwd_apply_kernel(const BnArgs a) {
  constexpr int VEC = BnElem<T>::VEC;
  const int chunk = blockIdx.x, c = blockIdx.y, n = blockIdx.z;
  const int64_t s0 = (int64_t)chunk * kBnChunk;
  const int len = (int)min((int64_t)kBnChunk, a.S - s0);
  const int64_t base = plane_base<T>(a, n, c) + s0;
  const int64_t gbase = (int64_t)n * a.gn + (int64_t)c * a.gc + s0;
  const int64_t obase = (int64_t)n * a.on + (int64_t)c * a.oc + s0;
  const float2 ss = saved_scale_shift(a, c);
  const float scale = ss.x, shift = ss.y;
  const float b = a.coef[4 * c + 2], c0 = a.coef[4 * c + 3];
#pragma unroll 4
  for (int i = threadIdx.x * VEC; i < len; i += kBnThreads * VEC) {
    float y[VEC], dz[VEC];
    BnElem<T>::load(a.y, base + i, y);
    BnElem<T>::load(a.dz, gbase + i, dz);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      const float g = fmaf(y[e], scale, shift) > 0.f ? dz[e] : 0.f;
      dz[e] = fmaf(scale, g, fmaf(b, y[e], c0));
    }
    BnElem<T>::store(a.out, obase + i, dz);
  }
}

template <typename T>
void launch_fwd_t(const BnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)a.nchunk, (unsigned)a.C, (unsigned)a.N);
  if (a.training) {
    hipLaunchKernelGGL(bn_stats_kernel<T>, grid, dim3(kBnThreads), 0, s, a);
    hipLaunchKernelGGL(bn_stats_final_kernel, dim3((unsigned)a.C), dim3(kBnThreads), 0, s, a);
  } else {
    hipLaunchKernelGGL(bn_eval_coef_kernel, dim3((unsigned)((a.C + kBnThreads - 1) / kBnThreads)), dim3(kBnThreads), 0,
                       s, a);
  }
  hipLaunchKernelGGL(bn_relu_apply_kernel<T>, grid, dim3(kBnThreads), 0, s, a);
}

template <typename T>
void launch_bwd_t(const BnArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)a.nchunk, (unsigned)a.C, (unsigned)a.N);
  hipLaunchKernelGGL(bn_relu_bwd_sums_kernel<T>, grid, dim3(kBnThreads), 0, s, a);
  hipLaunchKernelGGL(bn_relu_bwd_final_kernel, dim3((unsigned)a.C), dim3(kBnThreads), 0, s, a);
  hipLaunchKernelGGL(bn_relu_bwd_apply_kernel<T>, grid, dim3(kBnThreads), 0, s, a);
}

}  // namespace

void launch_bn_relu_fwd(int dtype, const BnArgs& a, hipStream_t s) {
  if (dtype == DT_BF16) launch_fwd_t<bf16_tag>(a, s);
  else if (dtype == DT_F16) launch_fwd_t<f16_tag>(a, s);
  else launch_fwd_t<f32_tag>(a, s);
}

void launch_bn_relu_bwd(int dtype, const BnArgs& a, hipStream_t s) {
  if (dtype == DT_BF16) launch_bwd_t<bf16_tag>(a, s);
  else if (dtype == DT_F16) launch_bwd_t<f16_tag>(a, s);
  else launch_bwd_t<f32_tag>(a, s);
}

}  // namespace r3c
