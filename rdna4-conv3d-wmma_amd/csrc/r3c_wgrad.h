// r3c_wgrad.h -- weight-gradient ("reduction") kernel for gfx950 on v_mfma_f32_32x32x16 (template body).
//
//   C[f][(tap, g)] = sum over positions p of  F[p][f] * G[p (+) tap][g]
//
//   Conv3d dW (K3 / K1): F = dY (row grid = output grid), G = x at p + tap - pad,
//                        dW[co = f][ci = g][tap]     (src/rdna4_conv3d/conv3d_wmma.py:544-634)
//   ConvTranspose dW (T2DW): F = x (row grid = input grid), G = dY at 2p + tap,
//                        dW[ci = f][co = g][tap]     (conv3d_wmma.py:934-1012)
//
// A workgroup owns one 32-channel F block (MFMA rows), one G channel range of
// GCW channels, all taps, and a fixed contiguous range of TD x TH x 16
// position boxes (its split of K; deterministic).  The MFMA columns are the
// (tap, 4-channel quad) pairs of the range, flattened and cut into blocks of 32
// columns, so a 24-channel layer wastes no columns on channel padding; each
// wave owns CBW column blocks.
//
// Both operands need k to run over positions while lanes run over channels.
// The tiles are [position][channel] in LDS and the operands come from
// ds_read_tr16_b64 (inside a 16-lane group: out[4a + b][i] = lds16[addr[a + 4i] + b]):
// source lane s supplies the address of position 8g + s/4 (+4 for the second
// read) and of channel quad s%4 of its group, so every group of four output
// lanes may take its quad from a different tap -- that is what lets columns
// mix taps.  A tap only moves the row address, so alignment always holds.
//
// The bias gradient is one extra MFMA per step against an all-ones operand:
// db = sum F (db_mode 1, Conv3d) or sum G (db_mode 2, ConvTranspose, summed
// over taps by the reduce kernel).  Each split writes fp32 partials
// [split][Fpad][TAPS][Gpad]; wgrad_reduce_kernel adds the splits in a fixed
// order.
#pragma once
#include "r3c_row.h"

namespace r3c {

template <int MODE>
struct WgGeom {
  static constexpr int TAPS = MODE == MODE_K3 ? 27 : (MODE == MODE_T2DW ? 8 : 1);
};

template <typename T, int MODE, int CBW>
__global__ __launch_bounds__(256) void wgrad_kernel(const WgArgs a) {
  extern __shared__ uint4 smem4[];
  constexpr int TAPS = WgGeom<MODE>::TAPS;
  constexpr int NDBG = MODE == MODE_T2DW ? CBW : 1;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 5;          // MFMA k half (positions 8g .. 8g+7 of a step)
  const int h = (lane >> 4) & 1;    // which 16-lane half of the 32 columns / rows
  const int s = lane & 15;          // lane inside its 16-lane group
  const int li = lane & 31;

  int bid = blockIdx.x;
  const int ft = bid % a.n_ftiles;
  bid /= a.n_ftiles;
  const int gt = bid % a.n_gtiles;
  const int split = bid / a.n_gtiles;
  const int box_begin = (int)(((int64_t)split * a.nbox) / a.nsplit);
  const int box_end = (int)(((int64_t)(split + 1) * a.nbox) / a.nsplit);

  constexpr int CPF = 32;  // F tile row pitch (halves)
  const int cpg = a.GCW;   // G tile row pitch (halves)
  const int HH = a.HH, HW = a.HW;
  const int BOXPOS = a.TD * a.TH * 16;
  const int HPOS = a.HD * HH * HW;
  uint16_t* ftile = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* gtile = ftile + BOXPOS * CPF;

  const int nq = a.GCW >> 2;          // channel quads per tap
  const int nquads = TAPS * nq;
  // Column blocks of this wave: this lane's quad, its tap offset and channel.
  int goff[CBW];
  bool cbok[CBW];
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    const int cb = wv * CBW + q;
    cbok[q] = cb * 8 < nquads;
    const int Q = cb * 8 + 4 * h + (s & 3);
    const int tap = Q < nquads ? Q / nq : 0;
    const int cq = Q < nquads ? Q - (Q / nq) * nq : 0;
    int toff = 0;
    if (MODE == MODE_K3) toff = ((tap / 9) * HH + (tap / 3) % 3) * HW + tap % 3;
    else if (MODE == MODE_T2DW) toff = ((tap >> 2) * HH + ((tap >> 1) & 1)) * HW + (tap & 1);
    goff[q] = toff * cpg + cq * 4;
  }

  const bool do_dbf = a.db_mode == 1 && gt == 0 && wv == 0;
  const bool do_dbg = MODE == MODE_T2DW && a.db_mode == 2 && ft == 0;
  uint4 ones;
  ones.x = ones.y = ones.z = ones.w = pack2(T::one, T::one);

  f32x16_t acc[CBW], accf;
  f32x16_t accg[NDBG];
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    accf[e] = 0.f;
#pragma unroll
    for (int q = 0; q < CBW; ++q) acc[q][e] = 0.f;
#pragma unroll
    for (int q = 0; q < NDBG; ++q) accg[q][e] = 0.f;
  }

  const int fc0 = ft * 32;
  const int gc0 = gt * a.GCW;
  const int ggroups = a.GCW >> 3;  // 8-channel groups per G row
  const int nf_items = BOXPOS * 4;
  const int ng_items = HPOS * ggroups;
  const FastDiv20 divHH((uint32_t)HH);
  const FastDiv20 divHW((uint32_t)HW);
  const FastDiv20 divGG((uint32_t)ggroups);
  const int th_mask = a.TH - 1;
  const int fs1 = (int)a.fs[1], fs2 = (int)a.fs[2], fs3 = (int)a.fs[3], fs4 = (int)a.fs[4];
  const int gs1 = (int)a.gs[1], gs2 = (int)a.gs[2], gs3 = (int)a.gs[3], gs4 = (int)a.gs[4];
  const int fchan = s & 3;

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
    const __amdgpu_buffer_rsrc_t fsrc = make_rsrc(a.fsrc + (int64_t)n * a.fs[0], a.f_bytes);
    const __amdgpu_buffer_rsrc_t gsrc = make_rsrc(a.gsrc + (int64_t)n * a.gs[0], a.g_bytes);

    __syncthreads();  // the previous box is fully consumed
    // ---- stage F box: [BOXPOS][32]
    for (int it = tid; it < nf_items; it += 256) {
      int pos, cg;
      if (a.f_cl) {
        cg = it & 3;
        pos = it >> 2;
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
      const bool ok = gd < a.Rd && gh < a.Rh && gw < a.Rw && c0 < a.Fc;
      const int off = 2 * (gd * fs2 + gh * fs3 + gw * fs4 + c0 * fs1);
      uint4 v;
      if (a.f_cl) {
        v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(fsrc, ok ? off : kOob, 0, 0));
      } else {
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = __builtin_amdgcn_raw_buffer_load_b16(fsrc, (ok && c0 + q < a.Fc) ? off + 2 * q * fs1 : kOob, 0, 0);
        v = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
      }
      *reinterpret_cast<uint4*>(ftile + pos * CPF + cg * 8) = v;
    }
    // ---- stage G box (+ halo): [HPOS][GCW]
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
      const bool ok = (unsigned)gd < (unsigned)a.Gd && (unsigned)gh < (unsigned)a.Gh &&
                      (unsigned)gw < (unsigned)a.Gw && c0 < a.Gc;
      const int off = 2 * (gd * gs2 + gh * gs3 + gw * gs4 + c0 * gs1);
      uint4 v;
      if (a.g_cl) {
        v = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(gsrc, ok ? off : kOob, 0, 0));
      } else {
        uint16_t e[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
          e[q] = __builtin_amdgcn_raw_buffer_load_b16(gsrc, (ok && c0 + q < a.Gc) ? off + 2 * q * gs1 : kOob, 0, 0);
        v = make_uint4(pack2(e[0], e[1]), pack2(e[2], e[3]), pack2(e[4], e[5]), pack2(e[6], e[7]));
      }
      *reinterpret_cast<uint4*>(gtile + hp * cpg + cg * 8) = v;
    }
    __syncthreads();

    // ---- K loop: 16 positions (one 16-wide w line) per MFMA step.
    const int nsteps = BOXPOS >> 4;
    for (int st = 0; st < nsteps; ++st) {
      const int L0 = st * 16 + 8 * g + (s >> 2);
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
      const uint4 ffr = lds_tr_pair(ftile, L0 * CPF + 16 * h + 4 * fchan, L1 * CPF + 16 * h + 4 * fchan);
      if (do_dbf) accf = mfma32<T>(ffr, ones, accf);
#pragma unroll
      for (int q = 0; q < CBW; ++q) {
        if (!cbok[q]) continue;
        const uint4 gfr = lds_tr_pair(gtile, grow0 + goff[q], grow1 + goff[q]);
        acc[q] = mfma32<T>(ffr, gfr, acc[q]);
        if (MODE == MODE_T2DW) {
          if (do_dbg) accg[q < NDBG ? q : 0] = mfma32<T>(ones, gfr, accg[q < NDBG ? q : 0]);
        }
      }
    }
  }

  // ---- partial store: acc[q][4qq + r] = C[f = 8qq + 4g + r][column li of block]
  const size_t split_stride = (size_t)a.Fpad * TAPS * a.Gpad;
  float* part = a.part + (size_t)split * split_stride;
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    if (!cbok[q]) continue;
    const int Q = (wv * CBW + q) * 8 + (li >> 2);
    if (Q >= nquads) continue;
    const int tap = Q / nq;
    const int gch = gc0 + (Q - tap * nq) * 4 + (li & 3);
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = fc0 + 8 * qq + 4 * g + r;
        part[((size_t)f * TAPS + tap) * a.Gpad + gch] = acc[q][4 * qq + r];
      }
  }
  if (do_dbf && li == 0) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.dbpart[(size_t)split * a.Fpad + fc0 + 8 * qq + 4 * g + r] = accf[4 * qq + r];
  }
  if (MODE == MODE_T2DW && do_dbg && g == 0) {
#pragma unroll
    for (int q = 0; q < NDBG; ++q) {
      if (!cbok[q]) continue;
      const int Q = (wv * CBW + q) * 8 + (li >> 2);
      if (Q >= nquads) continue;
      const int tap = Q / nq;
      const int gch = gc0 + (Q - tap * nq) * 4 + (li & 3);
      a.dbpart[((size_t)split * TAPS + tap) * a.Gpad + gch] = accg[q][0];
    }
  }
}

template <typename T, int MODE, int CBW>
static void launch_wgrad_inst(const WgArgs& a, size_t lds, hipStream_t stream) {
  auto kern = wgrad_kernel<T, MODE, CBW>;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3(a.nblocks), dim3(256), lds, stream, a);
}

}  // namespace r3c
