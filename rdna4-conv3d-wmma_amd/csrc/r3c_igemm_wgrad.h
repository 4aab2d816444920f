// r3c_igemm_wgrad.h -- weight-gradient ("reduction") kernel for gfx950 (template body).
//
//   C[f][(tap, g)] = sum over positions p of  F[p][f] * G[p (+) tap][g]
//
//   Conv3d dW (K3 / K1): F = dY (row grid = output grid), G = x at p + tap - pad,
//                        dW[co = f][ci = g][tap]            (src/rdna4_conv3d/
//                        conv3d_wmma.py:544-634 maps the same GEMM)
//   ConvTranspose dW (T2): F = x (row grid = input grid), G = dY at 2p + tap,
//                        dW[ci = f][co = g][tap]            (conv3d_wmma.py:934-1012)
//
// Grid = nsplit x (tap tiles x G tiles x F tiles).  A split owns a contiguous,
// fixed range of TD x TH x 16 position boxes (deterministic); per box the F box
// and the G box plus halo are staged in LDS as [position][channel] and the K
// loop walks the box 32 positions at a time.  Both MFMA operands need k to run
// over positions while lanes run over channels, which is exactly what two
// ds_read_tr16_b64 reads deliver from a channel-contiguous tile: source lane s
// of a 16-lane group reads 4 channels (4*(s%4) .. +3) of position 8g + s/4
// (+4 for the second read), and the hardware hands lane j channel j of the
// eight positions.  A tap only moves the G row address, so alignment holds.
//
// Each wave owns CBW (tap, 16-channel G block) column blocks and all FB F
// blocks.  Bias gradients ride along as one extra MFMA against an all-ones
// operand: db = sum F (db_mode 1, Conv3d) or db = sum G (db_mode 2, ConvTranspose,
// summed over taps later).  Every split writes fp32 partials; the reduce kernel
// adds splits in a fixed order.
#pragma once
#include "r3c_device.h"
#include "r3c_kernels.h"
#include "r3c_igemm_fwd.h"

namespace r3c {

template <int MODE>
struct WgGeom {
  static constexpr int TAPS = MODE == MODE_K3 ? 27 : (MODE == MODE_T2DW ? 8 : 1);
};

template <typename T, int MODE, int FB, int CBW>
__global__ __launch_bounds__(256) void igemm_wgrad_kernel(const WgradArgs a) {
  extern __shared__ __align__(16) uint16_t smem[];
  constexpr int TAPS = WgGeom<MODE>::TAPS;
  constexpr int NDBG = MODE == MODE_T2DW ? CBW : 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 4;
  const int sl = lane & 15;

  int bid = blockIdx.x;
  const int ft = bid % a.n_ftiles;
  bid /= a.n_ftiles;
  const int gt = bid % a.n_gtiles;
  bid /= a.n_gtiles;
  const int tt = bid % a.n_ttiles;
  const int split = bid / a.n_ttiles;
  const int box_begin = (int)(((int64_t)split * a.nbox) / a.nsplit);
  const int box_end = (int)(((int64_t)(split + 1) * a.nbox) / a.nsplit);

  const int cpf = a.cpf, cpg = a.cpg;
  const int HH = a.HH, HW = a.HW;
  const int BOXPOS = a.TD * a.TH * 16;
  const int HPOS = a.HD * HH * HW;
  uint16_t* ftile = smem;
  uint16_t* gtile = smem + BOXPOS * cpf;

  // Column blocks of this wave.
  int cb_off[CBW];
  int cb_tap[CBW];
  int cb_g[CBW];
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    const int cbl = wv * CBW + q;
    const int tl = cbl / a.GCB, gl = cbl - (cbl / a.GCB) * a.GCB;
    const int tap = tt * a.TT + tl;
    const bool ok = (tl < a.TT) && (tap < TAPS);
    int toff = 0;
    if (ok) {
      if (MODE == MODE_K3) toff = ((tap / 9) * HH + (tap / 3) % 3) * HW + tap % 3;
      else if (MODE == MODE_T2DW) toff = ((tap >> 2) * HH + ((tap >> 1) & 1)) * HW + (tap & 1);
    }
    cb_tap[q] = ok ? tap : -1;
    cb_off[q] = toff * cpg + gl * 16 + 4 * (sl & 3);
    cb_g[q] = (gt * a.GCB + gl) * 16;
  }

  const bool do_dbf = a.db_mode == 1 && gt == 0 && tt == 0 && wv == 0;
  const bool do_dbg = MODE == MODE_T2DW && a.db_mode == 2 && ft == 0;
  uint4 ones;
  ones.x = ones.y = ones.z = ones.w = pack2(T::one, T::one);

  f32x4_t acc[FB][CBW];
  f32x4_t accf[FB];
  f32x4_t accg[NDBG];
#pragma unroll
  for (int fb = 0; fb < FB; ++fb) {
    accf[fb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < CBW; ++q) acc[fb][q] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int q = 0; q < NDBG; ++q) accg[q] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const int fc0 = ft * FB * 16;          // first F channel of this tile
  const int gc0 = gt * a.GCB * 16;       // first G channel of this tile
  const int fgroups = FB * 2;            // 8-channel groups per F row
  const int ggroups = a.GCB * 2;
  const int nf_items = BOXPOS * fgroups;
  const int ng_items = HPOS * ggroups;
  const FastDiv20 divHH((uint32_t)HH);
  const FastDiv20 divHW((uint32_t)HW);
  const FastDiv20 divGG((uint32_t)ggroups);
  const int th_mask = a.TH - 1;

  for (int box = box_begin; box < box_end; ++box) {
    int b = box;
    const int bw = b % a.nbw;
    b /= a.nbw;
    const int bh = b % a.nbh;
    b /= a.nbh;
    const int bd = b % a.nbd;
    const int n = b / a.nbd;
    const int r0d = bd * a.TD, r0h = bh * a.TH, r0w = bw * 16;
    int s0d, s0h, s0w;
    if (MODE == MODE_T2DW) {
      s0d = 2 * r0d;
      s0h = 2 * r0h;
      s0w = 2 * r0w;
    } else {
      s0d = r0d - a.pd;
      s0h = r0h - a.ph;
      s0w = r0w - a.pw;
    }

    __syncthreads();  // previous box fully consumed
    // ---- stage F box: [BOXPOS][cpf]
    {
      const uint16_t* fn = a.fsrc + (int64_t)n * a.fs[0];
      for (int it = tid; it < nf_items; it += 256) {
        int pos, cg;
        if (a.f_cl) {
          cg = it % fgroups;
          pos = it / fgroups;
        } else {
          cg = it / BOXPOS;
          pos = it - cg * BOXPOS;
        }
        const int tw = pos & 15;
        const int rr = pos >> 4;
        const int th = rr & th_mask;
        const int td = rr >> a.th_log2;
        const int gd = r0d + td, gh = r0h + th, gw = r0w + tw;
        const int c0 = fc0 + cg * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (gd < a.Rd && gh < a.Rh && gw < a.Rw && c0 < a.Fc) {
          const uint16_t* p = fn + gd * a.fs[2] + gh * a.fs[3] + gw * a.fs[4] + (int64_t)c0 * a.fs[1];
          if (a.f_cl && c0 + 8 <= a.Fc) {
            v = *reinterpret_cast<const uint4*>(p);
          } else {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (c0 + i < a.Fc) ? p[(int64_t)i * a.fs[1]] : (uint16_t)0;
            v = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
          }
        }
        *reinterpret_cast<uint4*>(ftile + pos * cpf + cg * 8) = v;
      }
    }
    // ---- stage G box (+ halo): [HPOS][cpg]
    {
      const uint16_t* gn = a.gsrc + (int64_t)n * a.gs[0];
      for (int it = tid; it < ng_items; it += 256) {
        int hp, cg;
        if (a.g_cl) {
          hp = (int)divGG.div((uint32_t)it);
          cg = it - hp * ggroups;
        } else {
          cg = it / HPOS;
          hp = it - cg * HPOS;
        }
        const int t = (int)divHW.div((uint32_t)hp);
        const int hw = hp - t * HW;
        const int hd = (int)divHH.div((uint32_t)t);
        const int hh = t - hd * HH;
        const int gd = s0d + hd, gh = s0h + hh, gw = s0w + hw;
        const int c0 = gc0 + cg * 8;
        uint4 v = make_uint4(0, 0, 0, 0);
        if ((unsigned)gd < (unsigned)a.Gd && (unsigned)gh < (unsigned)a.Gh && (unsigned)gw < (unsigned)a.Gw &&
            c0 < a.Gc) {
          const uint16_t* p = gn + gd * a.gs[2] + gh * a.gs[3] + gw * a.gs[4] + (int64_t)c0 * a.gs[1];
          if (a.g_cl && c0 + 8 <= a.Gc) {
            v = *reinterpret_cast<const uint4*>(p);
          } else {
            uint16_t e[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) e[i] = (c0 + i < a.Gc) ? p[(int64_t)i * a.gs[1]] : (uint16_t)0;
            v = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
          }
        }
        *reinterpret_cast<uint4*>(gtile + hp * cpg + cg * 8) = v;
      }
    }
    __syncthreads();

    // ---- K loop: 32 positions per step.
    const int nsteps = BOXPOS >> 5;
    for (int st = 0; st < nsteps; ++st) {
      // positions read by this lane (as a source lane of the transposing reads)
      const int L0 = st * 32 + 8 * g + (sl >> 2);
      const int L1 = L0 + 4;
      int grow0, grow1;
      {
        const int tw0 = L0 & 15, r0 = L0 >> 4;
        const int th0 = r0 & th_mask, td0 = r0 >> a.th_log2;
        const int tw1 = L1 & 15, r1 = L1 >> 4;
        const int th1 = r1 & th_mask, td1 = r1 >> a.th_log2;
        if (MODE == MODE_T2DW) {
          grow0 = ((2 * td0) * HH + 2 * th0) * HW + 2 * tw0;
          grow1 = ((2 * td1) * HH + 2 * th1) * HW + 2 * tw1;
        } else {
          grow0 = (td0 * HH + th0) * HW + tw0;
          grow1 = (td1 * HH + th1) * HW + tw1;
        }
      }
      grow0 *= cpg;
      grow1 *= cpg;
      uint4 ffr[FB];
      const int fa0 = L0 * cpf + 4 * (sl & 3);
      const int fa1 = L1 * cpf + 4 * (sl & 3);
#pragma unroll
      for (int fb = 0; fb < FB; ++fb) ffr[fb] = lds_tr_pair(ftile, fa0 + fb * 16, fa1 + fb * 16);
      if (do_dbf) {
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) accf[fb] = mfma<T>(ffr[fb], ones, accf[fb]);
      }
#pragma unroll
      for (int q = 0; q < CBW; ++q) {
        if (cb_tap[q] < 0) continue;
        const uint4 gfr = lds_tr_pair(gtile, grow0 + cb_off[q], grow1 + cb_off[q]);
#pragma unroll
        for (int fb = 0; fb < FB; ++fb) acc[fb][q] = mfma<T>(ffr[fb], gfr, acc[fb][q]);
        if (MODE == MODE_T2DW) {
          if (do_dbg) accg[q < NDBG ? q : 0] = mfma<T>(ones, gfr, accg[q < NDBG ? q : 0]);
        }
      }
    }
  }

  // ---- partial store: lane (g, j) holds rows 4g..4g+3 (F channels) of column j.
  const int j = lane & 15;
  const size_t split_stride = (size_t)a.Fpad * TAPS * a.Gpad;
  float* part = a.part + (size_t)split * split_stride;
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    const int tap = cb_tap[q];
    if (tap < 0) continue;
    const int gch = cb_g[q] + j;
#pragma unroll
    for (int fb = 0; fb < FB; ++fb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = fc0 + fb * 16 + 4 * g + r;
        part[((size_t)f * TAPS + tap) * a.Gpad + gch] = acc[fb][q][r];
      }
    }
  }
  if (do_dbf && j == 0) {
#pragma unroll
    for (int fb = 0; fb < FB; ++fb)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.dbpart[(size_t)split * a.Fpad + fc0 + fb * 16 + 4 * g + r] = accf[fb][r];
  }
  if (MODE == MODE_T2DW && do_dbg && g == 0) {
#pragma unroll
    for (int q = 0; q < NDBG; ++q) {
      const int tap = cb_tap[q];
      if (tap < 0) continue;
      a.dbpart[((size_t)split * TAPS + tap) * a.Gpad + cb_g[q] + j] = accg[q][0];
    }
  }
}

template <typename T, int MODE, int FB, int CBW>
static void launch_wgrad_inst(const WgradArgs& a, size_t lds, hipStream_t stream) {
  auto kern = igemm_wgrad_kernel<T, MODE, FB, CBW>;
  if (lds > 65536) hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3(a.nblocks), dim3(256), lds, stream, a);
}

}  // namespace r3c
