// r3c_wgrow.h -- k=3 Conv3d weight gradient that walks output rows, for
// w-contiguous (NCDHW) operands with pad_w = 1 and W = 32, 64 or 128, on
// v_mfma_f32_32x32x16 (template body).
//
//   dW[f][g][kd][kh][kw] = sum over positions p of dY[p][f] * x[p + (kd, kh, kw) - pad][g]
//                          (src/rdna4_conv3d/conv3d_wmma.py:544-634)
//
// What limits a weight-gradient kernel here is the vector-memory path: small
// boxes use 32-40 bytes of every 128-byte line they fetch and need a tap halo
// around every box.  This kernel's unit of work is one whole output row
// (n, d, h, all W positions; WL MFMA k-steps of 16 positions), and a workgroup
// walks a column of rows h0 .. h1-1 at fixed (n, d):
//
//   * a step covers RS = min(16 / WL, 8) output rows; the x rows they
//     need are rows h - ph + kh (kh = 0..2) of the planes d - pd + kd, kept in
//     a ring of 2 RS + 2 LDS slots, so each step stages RS new x rows per kd
//     plane (whole 128-byte lines) and RS dY rows (32 channel rows);
//   * w padding needs no halo: every x row is W wide and padded in LDS by a
//     zero slot on its left; position -1 reads that slot and position W the
//     next row's (a trailing zero slot follows the last row).
//
// MFMA blocks: columns are (kd, kh, channel) in blocks of 32 (9 GCW columns,
// NTRIP blocks), one block per wave, each computed for kw = 0, 1, 2: the three
// kw taps of one (kd, kh) differ by one position along w, so one
// ds_read_b128 (positions 8g .. 8g+7 of the k-step) and two ds_read_b32 (the
// pairs at 8g-2 and 8g+8) feed three MFMAs, kw = 0 and 2 shifted in registers
// (v_alignbit).  The F operand (dY, 32 output channels) is one ds_read_b128
// per lane per k-step, shared by the three.
//
// LDS: ring [2 RS + 2 slots][3 kd][GCW channels] and two F buffers
// [RS rows][32 channels], each a row of W + 8 halves (8 zero halves, then the
// W positions).  The row pitch is an odd number of 16-byte slots and a slot
// holds 3 GCW rows, a multiple of 16 slots apart modulo 256 bytes, so the
// 16-byte reads of 16 lanes hit 16 distinct slots: conflict-free.
//
// Pipeline per step j of a column: barrier; K loop over the step's rows;
// after its second k-step the staged registers of step j+1 go to LDS (dY rows
// to the free F buffer, the new x rows to the ring slots step j-1 alone read)
// and step j+2's loads are issued.  A column starts with its first two x rows
// loaded and committed directly.
//
// Work: tile (32 output channels, GCW input channels) x job (n, d, h range);
// workgroup (tile, split) takes jobs split, split + nsplit, ... and keeps its
// sums across them; partials [split][Fpad][27][Gpad], the bias gradient on the
// first wave without a block, and the fixed-order reduce as in the general
// weight-gradient kernel.
#pragma once
#include "r3c_wgrad.h"

namespace r3c {

// One 16-bit position to the right across a register pair: (lo >> 16) | (hi << 16).
__device__ __forceinline__ uint32_t shift16(uint32_t lo, uint32_t hi) {
  return __builtin_amdgcn_alignbit(hi, lo, 16);
}

template <typename T, int GCW, int WL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 8))) void wgrow_kernel(const WgArgs a) {
  extern __shared__ uint4 smem4[];
  using Geo = WrGeom<GCW, WL>;
  constexpr int W = Geo::W, P = Geo::P, RS = Geo::RS, NSLOT = Geo::NSLOT;
  constexpr int NCOL = Geo::NCOL, NTRIP = Geo::NTRIP;
  constexpr int RING = Geo::RING_HALVES, FBUF = Geo::FBUF_HALVES;
  constexpr int NT = Geo::THREADS, NSEG = W / 8;
  constexpr int NFI = Geo::NFI, NGI = Geo::NGI, NFS = Geo::NFS, NGS = Geo::NGS;
  constexpr int SLOT = 3 * GCW * P;  // halves per ring slot
  constexpr int KSTEPS = RS * WL;    // MFMA k-steps per step (8 or 16)

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5;
  const int li = lane & 31;

  // Workgroup -> (F tile, G tile, split); each XCD takes a contiguous range of
  // splits, i.e. of neighbouring (n, d) columns, whose x planes meet in its L2.
  const int nwg = gridDim.x;
  int bid = (nwg & 7) == 0 ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int ft = bid % a.n_ftiles;
  bid /= a.n_ftiles;
  const int gt = bid % a.n_gtiles;
  const int split = bid / a.n_gtiles;

  uint16_t* const lds = reinterpret_cast<uint16_t*>(smem4);
  uint16_t* const ring = lds;
  uint16_t* const fbuf = lds + RING + 8;  // after the ring's trailing zero slot
  const int fc0 = ft * 32;
  const int gc0 = gt * GCW;
  // G of a channel concatenation: the tile's channels lie in one tensor.
  const bool gsec = a.gsplit > 0 && gc0 >= a.gsplit;  // uniform
  const uint16_t* const gptr = gsec ? a.gsrc2 : a.gsrc;
  const int64_t gsamp = gsec ? a.gs0_2 : a.gs[0];
  const uint32_t grange = gsec ? a.g2_bytes : a.g_bytes;
  const int gcl = gsec ? gc0 - a.gsplit : gc0;  // the tile's first channel in its tensor

  // Zero slots: the 8 leading halves of every ring row, and one after the ring
  // (dY rows are never read outside their W positions).
  for (int r = tid; r <= NSLOT * 3 * GCW; r += NT)
    *reinterpret_cast<u32x4_t*>(ring + r * P) = u32x4_t{0u, 0u, 0u, 0u};

  // This wave's block and this lane's column (kd, kh, channel).
  const bool has_trip = wv < NTRIP;
  const bool do_dbf = a.db_mode == 1 && gt == 0 && wv == NTRIP;
  int ncol = (has_trip ? wv : 0) * 32 + li;
  const bool col_ok = has_trip && ncol < NCOL;
  if (ncol >= NCOL) ncol -= 32;  // a dead column reads a live one's slot pattern
  const int khd = ncol / GCW, gch = ncol - (ncol / GCW) * GCW;
  const int kd = khd / 3, kh = khd % 3;

  // Staging items.  dY: it = k NT + tid -> (row it / (32 NSEG), channel, segment), segment fastest.
  const int fs1 = (int)a.fs[1], fs2 = (int)a.fs[2], fs3 = (int)a.fs[3];
  const int gs1 = (int)a.gs[1], gs2 = (int)a.gs[2], gs3 = (int)a.gs[3];
  int frel[NFI], fslot[NFI], frow[NFI];
  bool fval[NFI];
#pragma unroll
  for (int k = 0; k < NFI; ++k) {
    const int it = k * NT + tid;
    const int seg = it % NSEG, ch = (it / NSEG) % 32, r = it / (32 * NSEG);
    const bool ex = it < NFS;
    frow[k] = ex ? r : -1;
    fval[k] = ex && fc0 + ch < a.Fc;
    // A load that is switched off keeps channel 0 in its offset: the product
    // of a channel past Fc and a large channel stride could leave int32.
    frel[k] = 2 * ((fval[k] ? fc0 + ch : 0) * fs1 + r * fs3 + 8 * seg);
    fslot[k] = ((ex ? r : 0) * 32 + ch) * P + 8 + 8 * seg;
  }
  // x: it = k NT + tid -> (row r, plane kd, channel, segment), segment fastest.
  int grel[NGI], gslot[NGI], grow[NGI], gkd[NGI];
  bool gval[NGI];
#pragma unroll
  for (int k = 0; k < NGI; ++k) {
    const int it = k * NT + tid;
    const int seg = it % NSEG, rest = it / NSEG;
    const int ch = rest % GCW, pk = (rest / GCW) % 3, r = rest / (3 * GCW);
    const bool ex = it < NGS;
    grow[k] = ex ? r : -1;
    gkd[k] = pk;
    gval[k] = ex && gc0 + ch < a.Gc;
    grel[k] = 2 * ((gval[k] ? gcl + ch : 0) * gs1 + 8 * seg);  // as frel
    gslot[k] = (pk * GCW + ch) * P + 8 + 8 * seg;  // plus the ring slot of row r
  }

  // A disabled load gets bit 31 set in its offset: past any num_records.
  auto gate = [&](int off, bool on) { return (int)((uint32_t)off | ((uint32_t)!on << 31)); };
  u32x4_t pf[NFI], pg[NGI];
  // Loads of dY rows hf .. hf + nf - 1 and of x rows xr .. xr + nx - 1 (planes
  // d - pd + kd); rows outside [0, Gh) read as zero.
  auto issue = [&](int n, int d, int hf, int nf, int xr, int nx) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t fsrc = make_rsrc_u(a.fsrc + (int64_t)n * a.fs[0], a.f_bytes);
    const __amdgpu_buffer_rsrc_t gsrc = make_rsrc_u(gptr + (int64_t)n * gsamp, grange);
    const int fbase = 2 * (d * fs2 + hf * fs3);
#pragma unroll
    for (int k = 0; k < NFI; ++k) {
      const bool ok = fval[k] & (frow[k] < nf);
      pf[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(fsrc, gate(fbase + frel[k], ok), 0, 0));
    }
#pragma unroll
    for (int k = 0; k < NGI; ++k) {
      const int xd = d - a.pd + gkd[k], x_r = xr + grow[k];
      const bool ok = gval[k] & (grow[k] < nx) & ((unsigned)xd < (unsigned)a.Gd) & ((unsigned)x_r < (unsigned)a.Gh);
      const int off = 2 * (xd * gs2 + x_r * gs3) + grel[k];
      pg[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(gsrc, gate(off, ok), 0, 0));
    }
  };
  auto slot_of = [&](int xr) {  // ring slot of x row xr (xr >= -NSLOT)
    const int m = xr % NSLOT;
    return m < 0 ? m + NSLOT : m;
  };
  auto commit_f = [&](int buf) {
#pragma unroll
    for (int k = 0; k < NFI; ++k)
      if (frow[k] >= 0) *reinterpret_cast<u32x4_t*>(fbuf + buf * FBUF + fslot[k]) = pf[k];
  };
  // x rows xr .. xr + nx - 1 to their ring slots.
  auto commit_g = [&](int xr, int nx) {
    const int s0 = slot_of(xr);
#pragma unroll
    for (int k = 0; k < NGI; ++k) {
      if (grow[k] < 0 || grow[k] >= nx) continue;
      int sl = s0 + grow[k];
      sl = sl >= NSLOT ? sl - NSLOT : sl;
      *reinterpret_cast<u32x4_t*>(ring + sl * SLOT + gslot[k]) = pg[k];
    }
  };

  f32x16_t acc0, acc1, acc2, accf;
#pragma unroll
  for (int e = 0; e < 16; ++e) acc0[e] = acc1[e] = acc2[e] = accf[e] = 0.f;
  uint4 ones;
  ones.x = ones.y = ones.z = ones.w = pack2(T::one, T::one);

  // One step: RS output rows x WL k-steps.  ROLE 0 staging only, 1 three kw
  // MFMAs, 2 bias MFMA.  goff[r]: this lane's x row item for output row r.
  auto run_step = [&](int fb, const int (&goff)[RS], auto role_c, auto&& hook) __attribute__((always_inline)) {
    constexpr int ROLE = decltype(role_c)::value;
    const uint16_t* fr = fbuf + fb * FBUF + li * P + 8 + 8 * g;
    uint4 ffr[2];
    u32x4_t gq[2];
    uint32_t e0[2], e5[2];
    auto read_step = [&](auto s_c, int slot) __attribute__((always_inline)) {
      constexpr int S = decltype(s_c)::value;
      constexpr int R = S / WL, KS = S % WL;
      if constexpr (ROLE != 0) ffr[slot] = *reinterpret_cast<const uint4*>(fr + R * 32 * P + 16 * KS);
      if constexpr (ROLE == 1) {
        const uint16_t* gr = ring + goff[R] + 8 * g + 16 * KS;
        gq[slot] = *reinterpret_cast<const u32x4_t*>(gr);
        const uint32_t* pe = reinterpret_cast<const uint32_t*>(gr - 2);
        e0[slot] = pe[0];  // positions 8g - 2, 8g - 1 of the k-step
        e5[slot] = pe[5];  // positions 8g + 8, 8g + 9
      }
    };
    auto step = [&](auto s_c) __attribute__((always_inline)) {
      constexpr int S = decltype(s_c)::value;
      constexpr int CUR = S & 1;
      if constexpr (S + 1 < KSTEPS) read_step(std::integral_constant<int, S + 1>{}, CUR ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (ROLE == 1) {
        const u32x4_t q = gq[CUR];
        uint4 b0, b1, b2;
        b0.x = shift16(e0[CUR], q[0]);
        b0.y = shift16(q[0], q[1]);
        b0.z = shift16(q[1], q[2]);
        b0.w = shift16(q[2], q[3]);
        b1 = __builtin_bit_cast(uint4, q);
        b2.x = shift16(q[0], q[1]);
        b2.y = shift16(q[1], q[2]);
        b2.z = shift16(q[2], q[3]);
        b2.w = shift16(q[3], e5[CUR]);
        acc0 = mfma32<T>(ffr[CUR], b0, acc0);
        acc1 = mfma32<T>(ffr[CUR], b1, acc1);
        acc2 = mfma32<T>(ffr[CUR], b2, acc2);
      } else if constexpr (ROLE == 2) {
        accf = mfma32<T>(ffr[CUR], ones, accf);
      }
      if constexpr (S == 1) {
        __builtin_amdgcn_sched_barrier(0);
        hook();
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    read_step(std::integral_constant<int, 0>{}, 0);
    static_for(std::make_integer_sequence<int, KSTEPS>{}, step);
  };
  const int role = has_trip ? 1 : (do_dbf ? 2 : 0);

  // Jobs: (n, d, h range) = (job / (Rd * HS), (job / HS) % Rd, job % HS).
  const int HS = a.nbh;
  for (int job = split; job < a.nbox; job += a.nsplit) {
    const int hs = job % HS;
    const int d = (job / HS) % a.Rd;
    const int n = job / (HS * a.Rd);
    const int h0 = (int)(((int64_t)hs * a.Rh) / HS);
    const int h1 = (int)(((int64_t)(hs + 1) * a.Rh) / HS);
    const int nst = (h1 - h0 + RS - 1) / RS;  // steps; the last may cover fewer rows
    auto rows_at = [&](int j) { return j < nst ? min(RS, h1 - (h0 + j * RS)) : 0; };
    // Step j covers output rows h0 + j RS .. + RS - 1 and reads x rows
    // h0 + j RS - ph .. + RS + 1; its new x rows are the last RS of those.
    lds_barrier();  // the previous column's reads are done
    issue(n, d, h0, 0, h0 - a.ph, 2);
    commit_g(h0 - a.ph, 2);
    issue(n, d, h0, rows_at(0), h0 - a.ph + 2, RS);
    commit_f(0);
    commit_g(h0 - a.ph + 2, RS);
    issue(n, d, h0 + RS, rows_at(1), h0 + RS - a.ph + 2, nst > 1 ? RS : 0);
    for (int j = 0; j < nst; ++j) {
      const int h = h0 + j * RS;
      lds_barrier();  // step j's rows complete; the F buffer and ring slots of step j-1 free
      int goff[RS];
      {
        int sl = slot_of(h - a.ph) + kh;
#pragma unroll
        for (int r = 0; r < RS; ++r) {
          const int s_ = sl >= NSLOT ? sl - NSLOT : sl;
          goff[r] = s_ * SLOT + (kd * GCW + gch) * P + 8;
          sl = s_ + 1;
        }
      }
      auto hook = [&]() __attribute__((always_inline)) {
        if (j + 1 < nst) {
          commit_f((j + 1) & 1);
          commit_g(h + RS - a.ph + 2, RS);
        }
        issue(n, d, h + 2 * RS, rows_at(j + 2), h + 2 * RS - a.ph + 2, j + 2 < nst ? RS : 0);
      };
      if (role == 1) run_step(j & 1, goff, std::integral_constant<int, 1>{}, hook);
      else if (role == 2) run_step(j & 1, goff, std::integral_constant<int, 2>{}, hook);
      else run_step(j & 1, goff, std::integral_constant<int, 0>{}, hook);
    }
  }

  // ---- partial store: acc_kw[4q + r] = C[f = 8q + 4g + r][column li], tap = 3 khd + kw
  const size_t split_stride = (size_t)a.Fpad * 27 * a.Gpad;
  float* part = a.part + (size_t)split * split_stride;
  if (col_ok) {
    const int gcol = gc0 + gch;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int f = fc0 + 8 * q + 4 * g + r;
        float* o = part + ((size_t)f * 27 + 3 * khd) * a.Gpad + gcol;
        o[0] = acc0[4 * q + r];
        o[a.Gpad] = acc1[4 * q + r];
        o[2 * a.Gpad] = acc2[4 * q + r];
      }
  }
  if (do_dbf && li == 0) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) a.dbpart[(size_t)split * a.Fpad + fc0 + 8 * q + 4 * g + r] = accf[4 * q + r];
  }
}

template <typename T, int GCW, int WL>
static void launch_wgrow_inst(const WgArgs& a, hipStream_t stream) {
  auto kern = wgrow_kernel<T, GCW, WL>;
  constexpr int lds = WrGeom<GCW, WL>::LDS_BYTES;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  hipLaunchKernelGGL(kern, dim3(a.nblocks), dim3(WrGeom<GCW, WL>::THREADS), lds, stream, a);
}

}  // namespace r3c
