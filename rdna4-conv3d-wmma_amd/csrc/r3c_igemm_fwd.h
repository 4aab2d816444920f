// r3c_igemm_fwd.h -- implicit-GEMM "row" kernel for gfx950 (template body).
//
// One workgroup = 4 waves = a box of TD x TH x 16 rows of the row grid times
// NB column blocks of 16.  Wave w owns MB consecutive 16-row blocks (one 16-wide
// w-row each); every lane keeps MB x NB fp32 accumulator tiles.
//
// K loop (per source-channel chunk of CK channels):
//   1. the source box plus its halo is staged into LDS as [position][channel],
//      row pitch CP halves (CP / 8 odd, so the 16 rows an MFMA operand reads in
//      one ds_read_b128 fall in distinct bank groups).  Out-of-range positions
//      and channels are zero-filled, so the MFMA loop has no bounds checks.
//   2. k walks (tap, 8-channel group); lane group g takes group 4 * step + g.
//      A fragments are single ds_read_b128 reads at row + tap offset (a small
//      LDS table maps the group index to that offset); B fragments are 16-byte
//      loads of the pre-packed weight, already in lane order.
//
// Index math follows the reference kernels: K3 fwd (src/rdna4_conv3d/
// conv3d_wmma.py:372-444), K1 fwd (328-369), ConvTranspose fwd scatter
// (793-860) and ConvTranspose dX gather (863-931).
#pragma once
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

// n / d for n < 4096 and 1 <= d < 256, via a 20-bit reciprocal (exact in range).
struct FastDiv20 {
  uint32_t m;
  __device__ __forceinline__ explicit FastDiv20(uint32_t d) : m(((1u << 20) + d - 1) / d) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (n * m) >> 20; }
};

template <int MODE>
struct FwdGeom {
  static constexpr int TAPS = MODE == MODE_K3 ? 27 : (MODE == MODE_T2DX ? 8 : 1);
  static constexpr int HW = MODE == MODE_K3 ? 18 : (MODE == MODE_T2DX ? 32 : 16);
};

template <typename T, int MODE, int CK, int NB, int MB>
__global__ __launch_bounds__(256) void igemm_fwd_kernel(const FwdArgs a) {
  extern __shared__ __align__(16) uint16_t smem[];
  constexpr int G8 = CK / 8;
  constexpr int CP = (G8 & 1) ? CK : CK + 8;
  constexpr int TAPS = FwdGeom<MODE>::TAPS;
  constexpr int HW = FwdGeom<MODE>::HW;
  constexpr int NKG = TAPS * G8;
  constexpr int NSTEP = (NKG + 3) / 4;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 4;

  int bid = blockIdx.x;
  const int ct = bid % a.n_ctiles;
  bid /= a.n_ctiles;
  const int bw = bid % a.nbw;
  bid /= a.nbw;
  const int bh = bid % a.nbh;
  bid /= a.nbh;
  const int bd = bid % a.nbd;
  const int n = bid / a.nbd;
  const int r0d = bd * a.TD, r0h = bh * a.TH, r0w = bw * 16;

  int s0d, s0h, s0w;  // source coordinate of the LDS tile origin
  if (MODE == MODE_K3 || MODE == MODE_K1) {
    s0d = r0d - a.pd;
    s0h = r0h - a.ph;
    s0w = r0w - a.pw;
  } else if (MODE == MODE_T2DX) {
    s0d = 2 * r0d;
    s0h = 2 * r0h;
    s0w = 2 * r0w;
  } else {
    s0d = r0d;
    s0h = r0h;
    s0w = r0w;
  }

  const int HH = a.HH;
  const int HPOS = a.HD * HH * HW;
  uint16_t* tile = smem;
  // k-group -> LDS offset table.  Groups past the last real one (the K padding
  // of the final step) point at offset 0, the row's own tap-0 channels: an
  // in-bounds read of values inside the receptive field, multiplied by the
  // zero weights the packer wrote for those groups.
  int* ktab = reinterpret_cast<int*>(smem + HPOS * CP);

  for (int kg = tid; kg < NSTEP * 4; kg += 256) {
    int off = 0;
    if (kg < NKG) {
      const int tap = kg / G8, cg = kg % G8;
      int toff = 0;
      if (MODE == MODE_K3) toff = ((tap / 9) * HH + (tap / 3) % 3) * HW + tap % 3;
      else if (MODE == MODE_T2DX) toff = ((tap >> 2) * HH + ((tap >> 1) & 1)) * HW + (tap & 1);
      off = toff * CP + cg * 8;
    }
    ktab[kg] = off;
  }

  int rowbase[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = wv * MB + mb;
    const int td = r / a.TH, th = r - (r / a.TH) * a.TH, tw = lane & 15;
    int hp;
    if (MODE == MODE_T2DX) hp = ((2 * td) * HH + 2 * th) * HW + 2 * tw;
    else hp = (td * HH + th) * HW + tw;
    rowbase[mb] = hp * CP;
  }

  f32x4_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const FastDiv20 divHH((uint32_t)HH);
  const uint16_t* srcn = a.src + (int64_t)n * a.ss[0];
  const uint4* wfr = reinterpret_cast<const uint4*>(a.wpk) + (size_t)ct * NB * 64 + lane;
  const int nitems = HPOS * G8;

  for (int chunk = 0; chunk < a.nchunks; ++chunk) {
    if (chunk) __syncthreads();
    const int cbase = chunk * CK;
    for (int it = tid; it < nitems; it += 256) {
      int hp, cg;
      if (a.src_cl) {
        cg = it % G8;
        hp = it / G8;
      } else {
        cg = it / HPOS;
        hp = it - cg * HPOS;
      }
      const int t = hp / HW;
      const int hw = hp - t * HW;
      const int hd = (int)divHH.div((uint32_t)t);
      const int hh = t - hd * HH;
      const int gd = s0d + hd, gh = s0h + hh, gw = s0w + hw;
      const int c0 = cbase + cg * 8;
      uint4 v = make_uint4(0, 0, 0, 0);
      if ((unsigned)gd < (unsigned)a.Sd && (unsigned)gh < (unsigned)a.Sh &&
          (unsigned)gw < (unsigned)a.Sw && c0 < a.Cs) {
        const uint16_t* p = srcn + gd * a.ss[2] + gh * a.ss[3] + gw * a.ss[4] + (int64_t)c0 * a.ss[1];
        if (a.src_cl && c0 + 8 <= a.Cs) {
          v = *reinterpret_cast<const uint4*>(p);
        } else {
          uint16_t e[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) e[i] = (c0 + i < a.Cs) ? p[(int64_t)i * a.ss[1]] : (uint16_t)0;
          v = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
        }
      }
      *reinterpret_cast<uint4*>(tile + hp * CP + cg * 8) = v;
    }
    __syncthreads();

    const uint4* wc = wfr + (size_t)chunk * NSTEP * a.nbt_pad * 64;
#pragma unroll 2
    for (int s = 0; s < NSTEP; ++s) {
      const int koff = ktab[s * 4 + g];
      uint4 bfr[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bfr[nb] = wc[((size_t)s * a.nbt_pad + nb) * 64];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint4 afr = *reinterpret_cast<const uint4*>(tile + rowbase[mb] + koff);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma<T>(afr, bfr[nb], acc[mb][nb]);
      }
    }
  }

  // Epilogue: lane (g, j) holds rows 4g..4g+3 (consecutive w) of column j.
  const int j = lane & 15;
  const int64_t* sd = a.sd;
  uint16_t* dstn = a.dst + (int64_t)n * sd[0];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = wv * MB + mb;
    const int td = r / a.TH, th = r - (r / a.TH) * a.TH;
    const int rd = r0d + td, rh = r0h + th;
    if (rd >= a.Rd || rh >= a.Rh) continue;
    const int rw0 = r0w + 4 * g;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int col = (ct * NB + nb) * 16 + j;
      if (col >= a.ncols) continue;
      if (MODE == MODE_T2FWD) {
        const int tap = col / a.cout_t2;
        const int co = col - tap * a.cout_t2;
        const float bv = a.bias ? to_f32<T>(a.bias[co]) : 0.f;
        const int kd = tap >> 2, kh = (tap >> 1) & 1, kw = tap & 1;
        uint16_t* base = dstn + (int64_t)co * sd[1] + (int64_t)(2 * rd + kd) * sd[2] + (int64_t)(2 * rh + kh) * sd[3];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int rw = rw0 + q;
          if (rw < a.Rw) base[(int64_t)(2 * rw + kw) * sd[4]] = from_f32<T>(acc[mb][nb][q] + bv);
        }
      } else {
        const float bv = a.bias ? to_f32<T>(a.bias[col]) : 0.f;
        uint16_t* base = dstn + (int64_t)col * sd[1] + (int64_t)rd * sd[2] + (int64_t)rh * sd[3];
        uint16_t* p = base + (int64_t)rw0 * sd[4];
        if (sd[4] == 1 && rw0 + 3 < a.Rw && ((reinterpret_cast<uintptr_t>(p) & 7) == 0)) {
          uint2 v;
          v.x = pack2(from_f32<T>(acc[mb][nb][0] + bv), from_f32<T>(acc[mb][nb][1] + bv));
          v.y = pack2(from_f32<T>(acc[mb][nb][2] + bv), from_f32<T>(acc[mb][nb][3] + bv));
          *reinterpret_cast<uint2*>(p) = v;
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (rw0 + q < a.Rw) base[(int64_t)(rw0 + q) * sd[4]] = from_f32<T>(acc[mb][nb][q] + bv);
        }
      }
    }
  }
}

template <typename T, int MODE, int CK, int NB, int MB>
static void launch_fwd_inst(const FwdArgs& a, size_t lds, hipStream_t stream) {
  auto kern = igemm_fwd_kernel<T, MODE, CK, NB, MB>;
  if (lds > 65536) hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3(a.nblocks), dim3(256), lds, stream, a);
}

}  // namespace r3c
