// r3c_skinny.hip -- k=1 Conv3d with at most 4 output channels (the UNet3D's
// 1x1x1 class head, reference benches/unet_e2e.py:32), on NCDHW tensors with
// dense (d, h, w) planes: forward, dX and dW + db as streaming kernels.
//
// With O <= 4 output channels the product has no MFMA-sized dimension on the
// output side (a 32-wide block would be 8x padding) and moves
//   fwd  |x| + |y|,   dX  |dy| + |dx|,   dW  |x| + |dy|
// bytes for 2 * O * C flops per position: HBM-bound.  One thread covers 8
// consecutive positions of a plane, i.e. one 16-byte vector per channel, so a
// wave's load of one channel is a contiguous 1 KiB run; arithmetic in fp32.
//   fwd: y[o][p] = b[o] + sum_c w[o][c] x[c][p]      (reference _conv1x1 path)
//   dX : dx[c][p] = sum_o w[o][c] dy[o][p]           (_dgrad_k1_scale_kernel,
//                                                     src/rdna4_conv3d/conv3d_wmma.py:761-785)
//   dW : dw[o][c] = sum_p dy[o][p] x[c][p], db[o] = sum_p dy[o][p]
// dW: workgroup (s, b) owns a fixed, contiguous range s of position groups
// and channel block b of 8; it sums in registers, then over its 256 threads
// in a fixed shape (a butterfly per wave, the 4 waves in order), and writes
// partials [s][O][1][C] (+ [s][O] for db, from block 0) that the
// weight-gradient reduce adds in split order: deterministic.
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

template <typename T>
__device__ __forceinline__ void unpack8(const uint4& q, float* v) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    v[2 * e] = to_f32<T>((uint16_t)(w[e] & 0xffff));
    v[2 * e + 1] = to_f32<T>((uint16_t)(w[e] >> 16));
  }
}
template <typename T>
__device__ __forceinline__ uint4 pack8(const float* v) {
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) w[e] = pack2(from_f32<T>(v[2 * e]), from_f32<T>(v[2 * e + 1]));
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Position group g (8 positions) -> (sample, element offset of its first position in a plane).
__device__ __forceinline__ void group_at(const SkinnyArgs& a, int64_t g, int& n, int64_t& p) {
  const int64_t gp = a.P >> 3;
  n = (int)(g / gp);
  p = (g - (int64_t)n * gp) * 8;
}

template <typename T, int O>
__global__ __launch_bounds__(256) void skinny_fwd_kernel(const SkinnyArgs a) {
  __shared__ float ws[4 * kSkinnyMaxC];
  __shared__ float bs[4];
  for (int i = threadIdx.x; i < O * a.C; i += 256) ws[i] = to_f32<T>(a.w[i]);  // w[o][c]
  if (threadIdx.x < O) bs[threadIdx.x] = a.b ? to_f32<T>(a.b[threadIdx.x]) : 0.f;
  __syncthreads();
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= a.ngroups) return;
  int n;
  int64_t p;
  group_at(a, g, n, p);
  const uint16_t* x = a.x + n * a.xs0 + p;
  float acc[O][8];
#pragma unroll
  for (int o = 0; o < O; ++o)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[o][e] = bs[o];
  for (int c = 0; c < a.C; ++c) {
    float v[8];
    unpack8<T>(*reinterpret_cast<const uint4*>(x + c * a.xs1), v);
#pragma unroll
    for (int o = 0; o < O; ++o) {
      const float wv = ws[o * a.C + c];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[o][e] = fmaf(wv, v[e], acc[o][e]);
    }
  }
  uint16_t* y = a.y + n * a.ys0 + p;
#pragma unroll
  for (int o = 0; o < O; ++o) *reinterpret_cast<uint4*>(y + o * a.ys1) = pack8<T>(acc[o]);
}

template <typename T, int O>
__global__ __launch_bounds__(256) void skinny_dx_kernel(const SkinnyArgs a) {
  __shared__ float ws[4 * kSkinnyMaxC];
  for (int i = threadIdx.x; i < O * a.C; i += 256) ws[i] = to_f32<T>(a.w[i]);
  __syncthreads();
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= a.ngroups) return;
  int n;
  int64_t p;
  group_at(a, g, n, p);
  const uint16_t* dy = a.y + n * a.ys0 + p;
  float gv[O][8];
#pragma unroll
  for (int o = 0; o < O; ++o) unpack8<T>(*reinterpret_cast<const uint4*>(dy + o * a.ys1), gv[o]);
  uint16_t* dx = a.x + n * a.xs0 + p;
  for (int c = 0; c < a.C; ++c) {
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.f;
#pragma unroll
    for (int o = 0; o < O; ++o) {
      const float wv = ws[o * a.C + c];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = fmaf(wv, gv[o][e], v[e]);
    }
    *reinterpret_cast<uint4*>(dx + c * a.xs1) = pack8<T>(v);
  }
}

template <typename T, int O>
__global__ __launch_bounds__(256) void skinny_dw_kernel(const SkinnyArgs a) {
  constexpr int NV = O * 8 + O;  // per thread: 8 channels x O, and db
  __shared__ float red[4 * NV];
  const int s = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t g0 = ((int64_t)s * a.ngroups) / a.nsplit;
  const int64_t g1 = ((int64_t)(s + 1) * a.ngroups) / a.nsplit;
  float* part = a.part + (size_t)s * O * a.C;
  {
    // One channel block per workgroup row: every block streams at once (a
    // loop over the blocks would drain the whole grid's loads once per block).
    const int cb = 8 * (int)blockIdx.y;
    float acc[NV];
#pragma unroll
    for (int v = 0; v < NV; ++v) acc[v] = 0.f;
    const int nc = a.C - cb < 8 ? a.C - cb : 8;
    // Two position groups per iteration, every load of both issued before
    // any arithmetic (a split holds few groups per thread, so the loads of
    // one iteration are most of what the thread ever has in flight).
    for (int64_t g = g0 + threadIdx.x; g < g1; g += 512) {
      uint4 dq[2][O], xq[2][8];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int64_t gu = g + 256 * u;
        const bool live = gu < g1;
        int n;
        int64_t p;
        group_at(a, live ? gu : g, n, p);
        const uint16_t* dy = a.y + n * a.ys0 + p;
        const uint16_t* x = a.x + n * a.xs0 + p + (int64_t)cb * a.xs1;
#pragma unroll
        for (int o = 0; o < O; ++o)
          dq[u][o] = live ? *reinterpret_cast<const uint4*>(dy + o * a.ys1) : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int k = 0; k < 8; ++k)
          xq[u][k] = (live && k < nc) ? *reinterpret_cast<const uint4*>(x + k * a.xs1) : make_uint4(0u, 0u, 0u, 0u);
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        float gv[O][8];
#pragma unroll
        for (int o = 0; o < O; ++o) {
          unpack8<T>(dq[u][o], gv[o]);
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[O * 8 + o] += gv[o][e];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          if (k >= nc) break;
          float v[8];
          unpack8<T>(xq[u][k], v);
#pragma unroll
          for (int o = 0; o < O; ++o)
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[o * 8 + k] = fmaf(gv[o][e], v[e], acc[o * 8 + k]);
        }
      }
    }
    // Fixed-shape reduction (deterministic): a butterfly over the wave's 64
    // lanes (both partners of a step form the same sum), then the 4 waves in
    // order.
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1)
#pragma unroll
      for (int v = 0; v < NV; ++v) acc[v] += __shfl_xor(acc[v], off);
    if (lane == 0)
#pragma unroll
      for (int v = 0; v < NV; ++v) red[wave * NV + v] = acc[v];
    __syncthreads();
    if (threadIdx.x < NV) {
      const int v = threadIdx.x;
      const float t = ((red[v] + red[NV + v]) + red[2 * NV + v]) + red[3 * NV + v];
      if (v < O * 8) {
        const int o = v / 8, k = v % 8;
        if (k < nc) part[o * a.C + cb + k] = t;
      } else if (cb == 0 && a.dbpart) {
        a.dbpart[(size_t)s * O + (v - O * 8)] = t;
      }
    }
    __syncthreads();
  }
}

}  // namespace

namespace {
template <typename T, int O>
void launch_o(int pass, const SkinnyArgs& a, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ngroups + 255) / 256);
  if (pass == 0) hipLaunchKernelGGL((skinny_fwd_kernel<T, O>), dim3(blocks), dim3(256), 0, s, a);
  else if (pass == 1) hipLaunchKernelGGL((skinny_dx_kernel<T, O>), dim3(blocks), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((skinny_dw_kernel<T, O>), dim3((unsigned)a.nsplit, (unsigned)((a.C + 7) / 8)), dim3(256), 0, s, a);
}
template <typename T>
bool launch_t(int pass, const SkinnyArgs& a, hipStream_t s) {
  switch (a.O) {
    case 1: launch_o<T, 1>(pass, a, s); return true;
    case 2: launch_o<T, 2>(pass, a, s); return true;
    case 3: launch_o<T, 3>(pass, a, s); return true;
    case 4: launch_o<T, 4>(pass, a, s); return true;
    default: return false;
  }
}
}  // namespace

bool launch_skinny(int dtype, int pass, const SkinnyArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_t<bf16_tag>(pass, a, s) : launch_t<f16_tag>(pass, a, s);
}

}  // namespace r3c
