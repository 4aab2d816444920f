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

// Tap range of one dimension for a destination coordinate q: taps k0, k0 +
// step, ... (n of them) with source coordinates c0, c0 + dc, ...  Forward:
// every tap, source q s - p + k.  dX: the taps with (q + p - k) divisible by
// s, source (q + p - k) / s.
struct TapRange {
  int k0, step, n, c0, dc;
};
__device__ __forceinline__ TapRange tap_range(bool dx, int q, int p, int s, int k) {
  TapRange r;
  if (!dx) {
    r.k0 = 0;
    r.step = 1;
    r.n = k;
    r.c0 = q * s - p;
    r.dc = 1;
  } else {
    r.k0 = (q + p) % s;  // q + p >= 0
    r.step = s;
    r.n = r.k0 < k ? (k - 1 - r.k0) / s + 1 : 0;
    r.c0 = (q + p - r.k0) / s;
    r.dc = -1;
  }
  return r;
}

template <typename T, int NB, int SCL>
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

  // Taps that reach the tile, per dimension (uniform; in w the tile's
  // residue class makes the dX range the same for every lane), and this
  // lane's source w for the first of them.
  const TapRange td = tap_range(a.dx, rd, a.pd, a.sd, a.k);
  const TapRange th = tap_range(a.dx, rh, a.ph, a.sh, a.k);
  const TapRange tw = tap_range(a.dx, a.dx ? res : rw, a.pw, a.sw, a.k);
  const int sw0 = a.dx ? j + tw.c0 : tw.c0;
  const int nc16 = a.nc16;
  const int total = td.n * th.n * tw.n * nc16;  // K iterations: (tap d, h, w, channel block)

  f32x16_t acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;

  const uint16_t* src = a.src + (int64_t)n * a.ss[0] + (int64_t)(8 * g) * a.ss[1];
  const uint4* wpk = reinterpret_cast<const uint4*>(a.wpk) + (int64_t)ct * NB * 64 + lane;
  // Fragments of K iteration (md, mh, mw, c16), c16 fastest.
  struct KIt {
    int c16, mw, mh, md;
  };
  // live false: the fragment of a padding iteration (zero source values, so
  // its MFMAs add nothing; the weight loads stay in range at ki).
  auto load = [&](const KIt& ki, bool live, uint4& bfr, uint4 (&afr)[NB]) __attribute__((always_inline)) {
    const int c16 = ki.c16, mw = ki.mw, mh = ki.mh, md = ki.md;
    const int kd = td.k0 + md * td.step, kh = th.k0 + mh * th.step, kw = tw.k0 + mw * tw.step;
    // A tile no tap reaches (dX with a large stride) has no live iteration and
    // taps past the kernel in ki: its weight loads use tap 0.
    const int t = (live && a.k == 3) ? (kd * 3 + kh) * 3 + kw : 0;
    const int cd = td.c0 + md * td.dc, ch = th.c0 + mh * th.dc, cw = sw0 + mw * tw.dc;
    const int kch0 = c16 * 16 + 8 * g;
    const bool ok = live && pos_ok && (unsigned)cd < (unsigned)a.Sd && (unsigned)ch < (unsigned)a.Sh &&
                    (unsigned)cw < (unsigned)a.Sw && kch0 < a.Cs;
    const uint16_t* p =
        src + (int64_t)(16 * c16) * a.ss[1] + (int64_t)cd * a.ss[2] + (int64_t)ch * a.ss[3] + (int64_t)cw * a.ss[4];
    if (SCL) {
      bfr = ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0u, 0u, 0u, 0u);
    } else {
      uint32_t wd[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t lo = (ok && kch0 + 2 * e < a.Cs) ? p[(int64_t)(2 * e) * a.ss[1]] : (uint16_t)0;
        const uint16_t hi = (ok && kch0 + 2 * e + 1 < a.Cs) ? p[(int64_t)(2 * e + 1) * a.ss[1]] : (uint16_t)0;
        wd[e] = pack2(lo, hi);
      }
      bfr = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
    const uint4* wrow = wpk + ((int64_t)c16 * a.taps + t) * a.nbt * 64;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) afr[nb] = wrow[nb * 64];
  };

  // Software pipeline, PF iterations deep: slot u holds the fragments of an
  // iteration it + u; after its MFMAs the slot loads iteration it + u + PF.
  // The iteration count is padded to a multiple of PF with zero fragments, so
  // every load is unconditional and each MFMA waits only for its own slot.
  // The iteration counters advance by carries, no divisions.
  constexpr int PF = 4;
  auto advance = [&](KIt& ki) __attribute__((always_inline)) {
    if (++ki.c16 < nc16) return;
    ki.c16 = 0;
    if (++ki.mw < tw.n) return;
    ki.mw = 0;
    if (++ki.mh < th.n) return;
    ki.mh = 0;
    ++ki.md;
  };
  KIt kn = {0, 0, 0, 0};  // next iteration to load (stays at the last one past the end)
  int loaded = 0;
  uint4 bq[PF], aq[PF][NB];
  auto fetch = [&](int u) __attribute__((always_inline)) {
    const bool live = loaded < total;
    load(kn, live, bq[u], aq[u]);
    ++loaded;
    if (loaded < total) advance(kn);
  };
#pragma unroll
  for (int u = 0; u < PF; ++u) fetch(u);
  for (int it = 0; it < total; it += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32<T>(aq[u][nb], bq[u], acc[nb]);
      fetch(u);
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
// w1/s) when all three divide, else zero.  Rows have a pitch of W1p (a
// multiple of 8, the tail past W1 unused); a thread writes 8 consecutive
// elements of one row as one 16-byte store; rows whose d1 or h1 is not a
// multiple of the stride are all zeros.
__global__ __launch_bounds__(256) void dilate_kernel(const DilateArgs a) {
  const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int gpr = a.W1p >> 3;  // 8-element groups per row
  const int64_t row = gi / gpr;
  if (row >= a.rows) return;
  const int w0 = (int)(gi - row * gpr) * 8;
  const int h1 = (int)(row % a.H1);
  const int64_t r2 = row / a.H1;
  const int d1 = (int)(r2 % a.D1);
  const int64_t nc = r2 / a.D1;  // n * C + c
  uint32_t wd[4] = {0u, 0u, 0u, 0u};
  if (d1 % a.sd == 0 && h1 % a.sh == 0) {
    const int c = (int)(nc % a.C);
    const int64_t n = nc / a.C;
    const uint16_t* s = a.src + n * a.ys[0] + (int64_t)c * a.ys[1] + (int64_t)(d1 / a.sd) * a.ys[2] +
                        (int64_t)(h1 / a.sh) * a.ys[3];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w1 = w0 + e;
      if (w1 < a.W1 && w1 % a.sw == 0) wd[e >> 1] |= (uint32_t)s[(int64_t)(w1 / a.sw) * a.ys[4]] << (16 * (e & 1));
    }
  }
  *reinterpret_cast<uint4*>(a.dst + row * a.W1p + w0) = make_uint4(wd[0], wd[1], wd[2], wd[3]);
}

template <typename T, int SCL>
bool launch_ts(const StridedArgs& a, int nb, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ntiles + 3) / 4);
  switch (nb) {
    case 1: hipLaunchKernelGGL((strided_kernel<T, 1, SCL>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((strided_kernel<T, 2, SCL>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 3: hipLaunchKernelGGL((strided_kernel<T, 3, SCL>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((strided_kernel<T, 4, SCL>), dim3(blocks), dim3(256), 0, s, a); return true;
    default: return false;
  }
}
template <typename T>
bool launch_t(const StridedArgs& a, int nb, hipStream_t s) {
  return a.scl ? launch_ts<T, 1>(a, nb, s) : launch_ts<T, 0>(a, nb, s);
}

}  // namespace

void launch_strided_pack(const StridedPackArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(strided_pack_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, s, a);
}

bool launch_strided(int dtype, int nb, const StridedArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_t<bf16_tag>(a, nb, s) : launch_t<f16_tag>(a, nb, s);
}

void launch_dilate(const DilateArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(dilate_kernel, dim3((unsigned)((a.rows * (a.W1p / 8) + 255) / 256)), dim3(256), 0, s, a);
}

}  // namespace r3c
