// r3c_strided.hip -- Conv3d with stride > 1 (k = 1 or 3, any padding): the
// downsampling convolution the reference routes to MIOpen (its policy admits
// stride 1 only, src/rdna4_conv3d/conv3d_wmma.py:89-95; README.md:55).
//
// Forward and dX are one direct implicit-GEMM kernel on v_mfma_f32_32x32x16
// in the C^T form (A = packed weights, rows = destination channels; B =
// source values, columns = 32 destination positions of one row):
//
//   forward  y[o][co] = b[co] + sum_{t, ci} x[o*s - p + t][ci] w[co][ci][t]
//            tile = 32 consecutive output positions along w.
//   dX       dx[i][ci] = sum_{t, co : i = o*s - p + t} dy[o][co] w[co][ci][t]
//            tile = 32 input positions of one residue class along w
//            (iw = r + s*j), so the taps that reach the tile are the same for
//            every lane: the K loop visits exactly them (no zero products for
//            the positions a stride skips).
//
// K walks (source-channel block of 16, tap); lane half g holds channels
// 8g .. 8g+7 of the block, so one MFMA is one tap of 16 source channels.
// Source fragments are loaded straight from memory: one 16-byte load when the
// source is channel-contiguous (NDHWC), else eight 2-byte loads.  Weights are
// packed once per call into [block][tap][column block][lane][8].
//
// dW reuses the stride-1 weight-gradient kernels: dY is scattered into the
// stride-1 output grid (zeros between, dilate_kernel) and dW, db of the
// stride-1 convolution of x with it are exactly the strided ones.
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

// Packed weights: element (block c16, tap t, column block nb, lane (g, i), e)
// = w at K channel c16 * 16 + 8 g + e and destination channel nb * 32 + i.
// Forward: K channel = ci, column = co; dX: K channel = co, column = ci.
__global__ __launch_bounds__(256) void strided_pack_kernel(const StridedPackArgs a) {
  const int64_t v = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (v >= a.total) return;
  const int lane = (int)(v & 63);
  int64_t rest = v >> 6;
  const int nb = (int)(rest % a.nbt);
  rest /= a.nbt;
  const int t = (int)(rest % a.taps);
  const int c16 = (int)(rest / a.taps);
  const int col = nb * 32 + (lane & 31), g = lane >> 5;
  const int kc = a.dx ? a.cout : a.cin, nc = a.dx ? a.cin : a.cout;
  uint32_t wd[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int kch = c16 * 16 + 8 * g + e;
    uint32_t h = 0u;
    if (col < nc && kch < kc) {
      const int co = a.dx ? kch : col, ci = a.dx ? col : kch;
      h = a.w[((int64_t)co * a.cin + ci) * a.taps + t];
    }
    wd[e >> 1] |= h << (16 * (e & 1));
  }
  reinterpret_cast<uint4*>(a.out)[v] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
}

template <typename T, int NB>
__global__ __launch_bounds__(256) void strided_kernel(const StridedArgs a) {
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, li = lane & 31;
  const int64_t wt = (int64_t)blockIdx.x * 4 + wv;
  if (wt >= a.ntiles) return;  // no barrier in this kernel
  // Wave tile -> (column tile, w block, [residue], row, plane, sample).
  int64_t r = wt;
  const int ct = (int)(r % a.n_ctiles);
  r /= a.n_ctiles;
  const int wb = (int)(r % a.nwb);
  r /= a.nwb;
  int res = 0;
  if (a.dx) {
    res = (int)(r % a.sw);
    r /= a.sw;
  }
  const int rh = (int)(r % a.Rh);
  r /= a.Rh;
  const int rd = (int)(r % a.Rd);
  const int n = (int)(r / a.Rd);
  // This lane's destination w and whether it exists.
  const int j = wb * 32 + li;
  const int rw = a.dx ? res + a.sw * j : j;
  const bool pos_ok = rw < a.Rw;

  f32x16_t acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;

  const uint16_t* src = a.src + (int64_t)n * a.ss[0];
  const uint4* wpk = reinterpret_cast<const uint4*>(a.wpk);
  for (int c16 = 0; c16 < a.nc16; ++c16) {
    const int kch0 = c16 * 16 + 8 * g;  // this lane's 8 source channels
    const uint16_t* srcc = src + (int64_t)kch0 * a.ss[1];
    for (int t = 0; t < a.taps; ++t) {
      const int kd = a.k == 3 ? t / 9 : 0, kh = a.k == 3 ? (t / 3) % 3 : 0, kw = a.k == 3 ? t % 3 : 0;
      // Source position of this lane for tap t (forward: o*s - p + k; dX:
      // (i + p - k) / s, which must divide: uniform per tile in d and h, and
      // in w because the tile holds one residue class).
      int sd, sh, sw;
      if (!a.dx) {
        sd = rd * a.sd - a.pd + kd;
        sh = rh * a.sh - a.ph + kh;
        sw = rw * a.sw - a.pw + kw;
      } else {
        const int qd = rd + a.pd - kd, qh = rh + a.ph - kh, qw = res + a.pw - kw;
        if (qd < 0 || qh < 0 || qd % a.sd || qh % a.sh || (qw % a.sw + a.sw) % a.sw) continue;  // uniform
        sd = qd / a.sd;
        sh = qh / a.sh;
        // (res + s j + p - k) / s = j + (qw / s), qw possibly negative but divisible
        sw = j + (qw >= 0 ? qw / a.sw : -((-qw) / a.sw));
      }
      const bool ok = pos_ok && (unsigned)sd < (unsigned)a.Sd && (unsigned)sh < (unsigned)a.Sh &&
                      (unsigned)sw < (unsigned)a.Sw && kch0 < a.Cs;
      uint4 bfr = make_uint4(0u, 0u, 0u, 0u);
      const uint16_t* p = srcc + (int64_t)sd * a.ss[2] + (int64_t)sh * a.ss[3] + (int64_t)sw * a.ss[4];
      if (a.scl) {
        if (ok) bfr = *reinterpret_cast<const uint4*>(p);
      } else {
        uint32_t wd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint16_t lo = (ok && kch0 + 2 * q < a.Cs) ? p[(int64_t)(2 * q) * a.ss[1]] : (uint16_t)0;
          const uint16_t hi = (ok && kch0 + 2 * q + 1 < a.Cs) ? p[(int64_t)(2 * q + 1) * a.ss[1]] : (uint16_t)0;
          wd[q] = pack2(lo, hi);
        }
        bfr = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
      const uint4* wrow = wpk + (((int64_t)c16 * a.taps + t) * a.nbt + ct * NB) * 64 + lane;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32<T>(wrow[nb * 64], bfr, acc[nb]);
    }
  }

  // Epilogue: acc[nb][4q + r] = destination channel (ct NB + nb) 32 + 8 q + 4 g + r
  // at this lane's position.
  if (!pos_ok) return;
  uint16_t* dp = a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] + (int64_t)rw * a.sd5[4];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c0 = (ct * NB + nb) * 32 + 8 * q + 4 * g;
      if ((ct * NB + nb) * 32 + 8 * q >= a.Cd) break;  // uniform
      float v[4];
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        v[rr] = acc[nb][4 * q + rr] + ((a.b && c0 + rr < a.Cd) ? to_f32<T>(a.b[c0 + rr]) : 0.f);
      if (a.dvec4) {  // channels contiguous, Cd % 4 == 0: one 8-byte store
        if (c0 < a.Cd)
          *reinterpret_cast<uint2*>(dp + c0) =
              make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])), pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
      } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          if (c0 + rr < a.Cd) dp[(int64_t)(c0 + rr) * a.sd5[1]] = from_f32<T>(v[rr]);
      }
    }
}

// dY of the strided convolution scattered into the stride-1 output grid
// (dense NCDHW [n][c][D1][H1][W1]): element (d1, h1, w1) is dy at (d1/s, h1/s,
// w1/s) when all three divide, else zero.  8 consecutive elements per thread.
__global__ __launch_bounds__(256) void dilate_kernel(const DilateArgs a) {
  const int64_t i0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i0 >= a.total) return;
  uint16_t v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int64_t i = i0 + e;
    v[e] = 0;
    if (i < a.total) {
      int64_t r = i;
      const int w1 = (int)(r % a.W1);
      r /= a.W1;
      const int h1 = (int)(r % a.H1);
      r /= a.H1;
      const int d1 = (int)(r % a.D1);
      r /= a.D1;
      const int c = (int)(r % a.C);
      const int64_t n = r / a.C;
      if (d1 % a.sd == 0 && h1 % a.sh == 0 && w1 % a.sw == 0)
        v[e] = a.src[n * a.ys[0] + c * a.ys[1] + (int64_t)(d1 / a.sd) * a.ys[2] + (int64_t)(h1 / a.sh) * a.ys[3] +
                     (int64_t)(w1 / a.sw) * a.ys[4]];
    }
  }
  if (i0 + 8 <= a.total) {
    *reinterpret_cast<uint4*>(a.dst + i0) =
        make_uint4(pack2(v[0], v[1]), pack2(v[2], v[3]), pack2(v[4], v[5]), pack2(v[6], v[7]));
  } else {
    for (int e = 0; e < 8 && i0 + e < a.total; ++e) a.dst[i0 + e] = v[e];
  }
}

template <typename T>
bool launch_t(const StridedArgs& a, int nb, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ntiles + 3) / 4);
  switch (nb) {
    case 1: hipLaunchKernelGGL((strided_kernel<T, 1>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((strided_kernel<T, 2>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 3: hipLaunchKernelGGL((strided_kernel<T, 3>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((strided_kernel<T, 4>), dim3(blocks), dim3(256), 0, s, a); return true;
    default: return false;
  }
}

}  // namespace

void launch_strided_pack(const StridedPackArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(strided_pack_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, s, a);
}

bool launch_strided(int dtype, int nb, const StridedArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_t<bf16_tag>(a, nb, s) : launch_t<f16_tag>(a, nb, s);
}

void launch_dilate(const DilateArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(dilate_kernel, dim3((unsigned)((a.total / 8 + 256) / 256)), dim3(256), 0, s, a);
}

}  // namespace r3c
