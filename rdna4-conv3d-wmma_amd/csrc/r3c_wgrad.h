// r3c_wgrad.h -- weight-gradient ("reduction") kernel for gfx950 on v_mfma_f32_32x32x16 (template body).
//
//   C[f][(tap, g)] = sum over positions p of  F[p][f] * G[p (+) tap][g]
//
//   Conv3d dW (K3 / K1): F = dY (row grid = output grid), G = x at p + tap - pad,
//                        dW[co = f][ci = g][tap]     (src/rdna4_conv3d/conv3d_wmma.py:544-634)
//   ConvTranspose dW (T2DW): F = x (row grid = input grid), G = dY at 2p + tap,
//                        dW[ci = f][co = g][tap]     (conv3d_wmma.py:934-1012)
//
// A workgroup (8 waves) owns one 32-channel F block (MFMA rows), one G channel
// range of GCW <= 32 channels, all taps, and a fixed contiguous range of
// position boxes (its split of K; deterministic).  The MFMA columns are the
// (tap, 4-channel quad) pairs of the range, flattened and cut into blocks of 32
// columns, so a 24-channel layer wastes no columns on channel padding; wave w
// owns column blocks w, w+8, w+16, ... (CBW of them at most).  The last wave,
// which has the fewest blocks, also accumulates the F-side bias gradient.
//
// Box geometry is fixed per mode: TD x TH lines of 16 positions along w, and
// the G tile is the box plus its tap halo.  Both LDS tiles are
// [position][32 channels] (64-byte rows), so every LDS offset the K loop uses
// is a compile-time immediate.
//
// Both MFMA operands need k to run over positions while lanes run over
// channels; they come from ds_read_tr16_b64 (inside a 16-lane group:
// out[4a + b][i] = lds16[addr[a + 4i] + b]).  Source lane s supplies the
// address of position 8g + s/4 (+4 for the second read) and of channel quad
// s%4 of its group, so every group of four output lanes may take its quad from
// a different tap -- that is what lets columns mix taps.  A tap only moves the
// row address, so alignment always holds.
//
// Pipeline: double-buffered LDS tiles, one barrier per box.  After the barrier
// the registers holding box b+1 are written to the free buffer, the loads of
// box b+2 are issued into those registers, and box b is computed.
//
// The bias gradient is one extra MFMA per step against an all-ones operand:
// db = sum F (db_mode 1, Conv3d) or sum G (db_mode 2, ConvTranspose, summed
// over taps by the reduce).  Each split writes fp32 partials
// [split][Fpad][TAPS][Gpad]; the reduce kernels add the splits in a fixed
// order.
#pragma once
#include "r3c_tap.h"

namespace r3c {


// CL: G staged by 16-byte channel vectors (else 8 two-byte loads per slot);
// with FL 0 the same holds for F, whose tile is [position][channel] and is read
// with ds_read_tr16_b64.  FL 1: F comes from a w-contiguous source (NCDHW) and
// is staged channel-major, [channel][FP positions], by 16-byte loads of 8
// positions; its A fragment (8 consecutive positions of one channel) is then a
// single ds_read_b128, and the padded pitch (FP = BOXPOS + 8) puts the 16
// lanes of a group on 16 distinct bank slots.  FL 2 (k=1 without padding,
// where G has no tap shift): G is staged and read the same way.  FL 3 (k=3, G
// w-contiguous as well): F as with FL 1; G keeps its [position][channel] halo
// tile but is staged from the w-contiguous source: an item (halo row,
// 8-channel group, 8-position segment) loads 8 positions of each of its 8
// channels with eight 16-byte loads and transposes them in registers into 8
// slots, so no NDHWC copy of G is needed.
template <typename T, int MODE, int CBW, int CL, int FL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 8))) void wgrad_kernel(const WgArgs a) {
  extern __shared__ uint4 smem4[];
  using Geo = WgGeom<MODE>;
  constexpr int TAPS = Geo::TAPS;
  constexpr int TH = Geo::TH;
  constexpr int HH = Geo::HH, HW = Geo::HW;
  constexpr int BOXPOS = Geo::BOXPOS, HPOS = Geo::HPOS;
  constexpr int NFI = Geo::NFI, NGI = Geo::NGI;
  constexpr int NT = Geo::THREADS;
  constexpr int FP = Geo::FP, FT = Geo::FT;
  constexpr int LINES = Geo::LINES;
  constexpr int TILE = FT + Geo::GT;  // halves per buffer
  constexpr int NDBG = MODE == MODE_T2DW ? CBW : 1;
  constexpr int WS = MODE == MODE_T2DW ? 2 : 1;  // G positions per F position along each axis
  // FL 3 G items per thread: HD * HH * 4 * GCW / 8 = 18 GCW items, one per
  // thread up to GCW = 24 (CBW <= 3); at GCW = 32 (CBW = 4) the 64 items past
  // the first 512 go to wave XW, which owns three of the 27 column blocks
  // (waves 0-2 own four, wave 7 adds the bias MFMA).
  constexpr int NGW = FL == 3 ? (CBW == 4 ? 2 : 1) : 1;
  constexpr int XW = 6;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int wvu = __builtin_amdgcn_readfirstlane(wv);  // the same, known wave-uniform
  const int g = lane >> 5;          // MFMA k half (positions 8g .. 8g+7 of a step)
  const int h = (lane >> 4) & 1;    // which 16-lane half of the 32 columns / rows
  const int s = lane & 15;          // lane inside its 16-lane group
  const int li = lane & 31;

  // Workgroups are dealt to the 8 XCDs round-robin; renumbering them so each
  // XCD owns a contiguous eighth keeps boxes whose halos overlap on one L2.
  const int nwg = gridDim.x;
  int bid = (nwg & 7) == 0 ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int ft = bid % a.n_ftiles;
  bid /= a.n_ftiles;
  const int gt = bid % a.n_gtiles;
  const int split = bid / a.n_gtiles;
  // Boxes of this split.  With a multiple of 8 splits, the splits of one XCD
  // (consecutive split indices) share a contiguous eighth of the boxes and take
  // them round-robin (box = first + si + k * s8): the workgroups running at the
  // same time then work on neighbouring boxes, whose halos meet in the XCD's
  // L2.  The assignment is fixed, so the sums stay deterministic.
  const bool sg8 = (a.nsplit & 7) == 0;
  const int s8 = sg8 ? a.nsplit >> 3 : 1;
  const int sgrp = sg8 ? split / s8 : split, si = sg8 ? split % s8 : 0;
  const int ngrp = sg8 ? 8 : a.nsplit;
  const int gb0 = (int)(((int64_t)sgrp * a.nbox) / ngrp);
  const int gb1 = (int)(((int64_t)(sgrp + 1) * a.nbox) / ngrp);
  const int box_begin = gb0 + si;

  uint16_t* const tiles = reinterpret_cast<uint16_t*>(smem4);  // [2][F tile, G tile]

  const int nq = a.GCW >> 2;  // channel quads per tap
  const int nquads = TAPS * nq;
  // This lane's column in each of the wave's blocks: its quad's tap offset and channel.
  int goff[CBW];
  bool cbok[CBW];
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    const int cb = q * 8 + wv;
    cbok[q] = cb * 8 < nquads;
    const int Q = cb * 8 + 4 * h + (s & 3);
    const int tap = Q < nquads ? Q / nq : 0;
    const int cq = Q < nquads ? Q - (Q / nq) * nq : 0;
    int toff = 0;
    if (MODE == MODE_K3) toff = ((tap / 9) * HH + (tap / 3) % 3) * HW + tap % 3;
    else if (MODE == MODE_T2DW) toff = ((tap >> 2) * HH + ((tap >> 1) & 1)) * HW + (tap & 1);
    goff[q] = toff * 32 + cq * 4;
  }

  const bool do_dbf = a.db_mode == 1 && gt == 0 && wv == 7;
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
  const int ng_items = HPOS * ggroups;

  // Staging items of this thread: item it = NT k + tid.  Code = (d, h, w, group)
  // of the item inside its tile, 8 bits each; -1 = no such item.
  //   F, CL: position it/4, group it%4    F, generic: group it/BOXPOS, position it%BOXPOS
  //   G, CL: position it/ggroups, group it%ggroups   G, generic: group it/HPOS, position it%HPOS
  int fcode[NFI], gcode[NGI];
#pragma unroll
  for (int k = 0; k < NFI; ++k) {
    const int it = k * NT + tid;
    if (FL >= 1) {  // (channel, line, half line): 8 positions of one channel
      const int half = it & 1, line = (it >> 1) % LINES, ch = (it >> 1) / LINES;
      fcode[k] = it < 32 * LINES * 2 ? ((line / TH) | ((line % TH) << 8) | ((8 * half) << 16) | (ch << 24)) : -1;
    } else {
      const int pos = CL ? it >> 2 : it % BOXPOS;
      const int cg = CL ? it & 3 : it / BOXPOS;
      const int line = pos >> 4;
      fcode[k] = it < BOXPOS * 4 ? ((line / TH) | ((line % TH) << 8) | ((pos & 15) << 16) | (cg << 24)) : -1;
    }
  }
#pragma unroll
  for (int k = 0; k < NGI; ++k) {
    const int it = k * NT + tid;
    if (FL == 2) {
      const int half = it & 1, line = (it >> 1) % LINES, ch = (it >> 1) / LINES;
      gcode[k] = it < 32 * LINES * 2 ? ((line / TH) | ((line % TH) << 8) | ((8 * half) << 16) | (ch << 24)) : -1;
      continue;
    }
    const int hp = CL ? it / ggroups : it % HPOS;
    const int cg = CL ? it - hp * ggroups : it / HPOS;
    const int t = hp / HW;
    gcode[k] = it < ng_items ? ((t / HH) | ((t % HH) << 8) | ((hp % HW) << 16) | (cg << 24)) : -1;
  }
  const int fs1 = (int)a.fs[1], fs2 = (int)a.fs[2], fs3 = (int)a.fs[3], fs4 = (int)a.fs[4];
  const int gs1 = (int)a.gs[1], gs2 = (int)a.gs[2], gs3 = (int)a.gs[3], gs4 = (int)a.gs[4];

  u32x4_t pf[NFI], pg[NGI];
  u32x4_t pgw[NGW][8];  // FL 3: eight channels x 8 positions per G item
  auto load8 = [&](const __amdgpu_buffer_rsrc_t& rs, bool ok, int off, int cvalid, int cs1) -> u32x4_t {
    if (CL) return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, ok ? off : kOob, 0, 0));
    u32x4_t v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(rs, (ok && 2 * q < cvalid) ? off + 4 * q * cs1 : kOob, 0, 0);
      const uint32_t hi =
          __builtin_amdgcn_raw_buffer_load_b16(rs, (ok && 2 * q + 1 < cvalid) ? off + (4 * q + 2) * cs1 : kOob, 0, 0);
      v[q] = lo | (hi << 16);
    }
    return v;
  };
  // Per-item relative byte offsets inside a box (F) or its halo tile (G),
  // whether the item exists with its channels in range (fixed per workgroup),
  // and the channel count left for the element-wise path.
  int frel[NFI], grel[NGI], fcv[NFI], gcv[NGI];
  bool fval[NFI], gval[NGI];
#pragma unroll
  for (int k = 0; k < NFI; ++k) {
    const int c = fcode[k];
    const int td = c & 255, th = (c >> 8) & 255, tw = (c >> 16) & 255, cg = c >> 24;
    if (FL >= 1) {
      const int ch = fc0 + cg;
      frel[k] = 2 * (td * fs2 + th * fs3 + tw + ch * fs1);
      fval[k] = c >= 0 && ch < a.Fc;
      fcv[k] = 8;
    } else {
      const int c0 = fc0 + cg * 8;
      frel[k] = 2 * (td * fs2 + th * fs3 + tw * fs4 + c0 * fs1);
      fval[k] = c >= 0 && c0 < a.Fc;
      fcv[k] = a.Fc - c0;
    }
  }
#pragma unroll
  for (int k = 0; k < NGI; ++k) {
    const int c = gcode[k];
    const int hd = c & 255, hh = (c >> 8) & 255, hw = (c >> 16) & 255, cg = c >> 24;
    if (FL == 2) {
      const int ch = gc0 + cg;
      grel[k] = 2 * (hd * gs2 + hh * gs3 + hw + ch * gs1);
      gval[k] = c >= 0 && ch < a.Gc;
      gcv[k] = 8;
    } else {
      const int c0 = gc0 + cg * 8;
      grel[k] = 2 * (hd * gs2 + hh * gs3 + hw * gs4 + c0 * gs1);
      gval[k] = c >= 0 && c0 < a.Gc;
      gcv[k] = a.Gc - c0;
    }
  }
  // FL 3 G items: item it = NT k + tid is (halo row, channel group cg,
  // segment j), j fastest so four neighbouring lanes load one 64-byte run.
  // Segment j covers w in [r0w - 8 + 8j, r0w + 8j) (r0w = the box's first w,
  // a multiple of 16; W % 8 == 0, so a segment is wholly inside or outside the
  // volume), i.e. tile columns hw0 = pw - 8 + 8j .. hw0 + 7, of which those in
  // [0, HW) are written (gwmask).  Code (hd, hh, j, cg), 8 bits each.
  static_assert(FL != 3 || (MODE == MODE_K3 && Geo::HD * HH * 4 * (CBW == 4 ? 4 : 3) <= NT + (NGW - 1) * 64),
                "FL 3: G items per thread");
  int gwcode[NGW], gwrel[NGW], gwmask[NGW], gwslot[NGW];
  if (FL == 3) {
    const int ncg = a.GCW >> 3;
#pragma unroll
    for (int k = 0; k < NGW; ++k) {
      const int it = k == 0 ? tid : (wv == XW ? NT + lane : 1 << 20);
      const int j = it & 3, rest = it >> 2;
      const int cg = rest % ncg, row = rest / ncg;
      const int hd = row / HH, hh = row - (row / HH) * HH;
      const bool ex = row < Geo::HD * HH;  // false for k = 1 outside wave XW
      const int hw0 = a.pw - 8 + 8 * j;
      int m = 0;
#pragma unroll
      for (int p = 0; p < 8; ++p) m |= ((unsigned)(hw0 + p) < (unsigned)HW) ? (1 << p) : 0;
      gwcode[k] = ex ? (hd | (hh << 8) | (j << 16) | (cg << 24)) : -1;
      gwmask[k] = ex ? m : 0;
      gwslot[k] = ((hd * HH + hh) * HW + hw0) * 32 + cg * 8;  // halves; only masked columns are written
      gwrel[k] = 2 * (hd * gs2 + hh * gs3 + 8 * j - 8 + (gc0 + cg * 8) * gs1);
    }
  }

  // Box cursor (w fastest), advanced by carries: the divisions happen once.
  struct BoxCur {
    int bw, bh, bd, n, box;
  };
  // The divisions run on the vector unit; readfirstlane puts the (uniform)
  // results back in scalar registers, so buffer resources built from them are
  // scalar too.  A resource in vector registers makes the compiler wrap every
  // buffer load in a readfirstlane / compare / exec-mask loop.
  auto box_at = [&](int box) {
    BoxCur c;
    box = __builtin_amdgcn_readfirstlane(box);
    c.box = box;
    c.bw = __builtin_amdgcn_readfirstlane(box % a.nbw);
    box = __builtin_amdgcn_readfirstlane(box / a.nbw);
    c.bh = __builtin_amdgcn_readfirstlane(box % a.nbh);
    box = __builtin_amdgcn_readfirstlane(box / a.nbh);
    c.bd = __builtin_amdgcn_readfirstlane(box % a.nbd);
    c.n = __builtin_amdgcn_readfirstlane(box / a.nbd);
    return c;
  };
  // Next box of this split: box + s8, as a digit-wise add of s8's digits
  // (w fastest) with carries -- each digit sum is below twice its radix, so
  // one conditional subtraction normalises it; no divisions per box.
  const BoxCur sdig = box_at(s8);
  auto box_advance = [&](BoxCur& c) {
    c.box += s8;
    int v = c.bw + sdig.bw;
    int cy = v >= a.nbw;
    c.bw = cy ? v - a.nbw : v;
    v = c.bh + sdig.bh + cy;
    cy = v >= a.nbh;
    c.bh = cy ? v - a.nbh : v;
    v = c.bd + sdig.bd + cy;
    cy = v >= a.nbd;
    c.bd = cy ? v - a.nbd : v;
    c.n += sdig.n + cy;
  };
  // Loads of one box into the staging registers.  A box whose tile lies
  // inside the volume (the common case) takes the precomputed validity; one
  // on an edge checks every item's position (branch-free).
  // The loads are issued whether or not box `cur` exists (`live`): a box past
  // the end reads with every offset out of range (zeros, no memory access)
  // from sample 0, which keeps the compiler's load counting exact (a commit
  // then waits only for its own box's loads).
  // A disabled load gets bit 31 set in its offset: past any num_records (every
  // valid offset is below 1 GiB; an edge item's offset may be negative, which
  // is past it too), by arithmetic rather than a select, which the compiler
  // would turn into branches around duplicated loads.
  auto gate = [&](int off, bool on) { return (int)((uint32_t)off | ((uint32_t)!on << 31)); };
  auto issue = [&](const BoxCur& cur, bool live) __attribute__((always_inline)) {
    const int r0d = cur.bd * Geo::TD, r0h = cur.bh * TH, r0w = cur.bw * 16;
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
    const __amdgpu_buffer_rsrc_t fsrc = make_rsrc_u(a.fsrc + (live ? (int64_t)cur.n * a.fs[0] : 0), a.f_bytes);
    const __amdgpu_buffer_rsrc_t gsrc = make_rsrc_u(a.gsrc + (live ? (int64_t)cur.n * a.gs[0] : 0), a.g_bytes);
    const int fbase = 2 * (r0d * fs2 + r0h * fs3 + r0w * fs4);
    const int gbase = 2 * (s0d * gs2 + s0h * gs3 + s0w * gs4);
    const bool f_in = r0d + Geo::TD <= a.Rd && r0h + TH <= a.Rh && r0w + 16 <= a.Rw;
    const bool g_in = s0d >= 0 && s0d + Geo::HD <= a.Gd && s0h >= 0 && s0h + HH <= a.Gh && s0w >= 0 &&
                      s0w + (FL == 2 ? 16 : HW) <= a.Gw;
#pragma unroll
    for (int k = 0; k < NFI; ++k) {
      const int c = fcode[k];
      const int gd = r0d + (c & 255), gh = r0h + ((c >> 8) & 255), gw = r0w + ((c >> 16) & 255);
      const bool ok = live & fval[k] & (f_in | ((gd < a.Rd) & (gh < a.Rh) & (gw < a.Rw)));
      const int off = fbase + frel[k];
      if (FL >= 1) pf[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(fsrc, gate(off, ok), 0, 0));
      else pf[k] = load8(fsrc, ok, off, fcv[k], fs1);
    }
    if constexpr (FL == 3) {
      // Tile rows start at (s0d, s0h); segments are addressed from the box's first w.
      const int gb3 = 2 * (s0d * gs2 + s0h * gs3 + r0w);
#pragma unroll
      for (int k = 0; k < NGW; ++k) {
        if (k > 0 && wvu != XW) break;  // wave-uniform: only wave XW holds second items
        const int c = gwcode[k];
        const int gd = s0d + (c & 255), gh = s0h + ((c >> 8) & 255), gw = r0w - 8 + 8 * ((c >> 16) & 255);
        const bool ok = live & (c >= 0) & ((unsigned)gd < (unsigned)a.Gd) & ((unsigned)gh < (unsigned)a.Gh) &
                        ((unsigned)gw < (unsigned)a.Gw);
        const int off = gb3 + gwrel[k];
        // G's buffer range ends at channel Gc (the host takes FL 3 only with
        // channel planes outermost), so channels past it need no gating; the
        // per-lane position gate is applied to each full offset (an edge
        // item's offset may be negative, and bit 31 must survive the channel
        // offset).
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pgw[k][e] = __builtin_bit_cast(
              u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(gsrc, gate(off + 2 * e * gs1, ok), 0, 0));
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < NGI; ++k) {
      const int c = gcode[k];
      const int gd = s0d + (c & 255), gh = s0h + ((c >> 8) & 255), gw = s0w + ((c >> 16) & 255);
      const bool ok = live & gval[k] &
                      (g_in | (((unsigned)gd < (unsigned)a.Gd) & ((unsigned)gh < (unsigned)a.Gh) & ((unsigned)gw < (unsigned)a.Gw)));
      const int off = gbase + grel[k];
      if (FL == 2) pg[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(gsrc, gate(off, ok), 0, 0));
      else pg[k] = load8(gsrc, ok, off, gcv[k], gs1);
    }
  };
  auto commit = [&](int buf) {
    uint16_t* ft = tiles + buf * TILE;
    uint16_t* gtl = ft + FT;
#pragma unroll
    for (int k = 0; k < NFI; ++k) {
      const int c = fcode[k];
      if (c >= 0) {
        const int pos = ((c & 255) * TH + ((c >> 8) & 255)) * 16 + ((c >> 16) & 255);
        if (FL >= 1) *reinterpret_cast<u32x4_t*>(ft + (c >> 24) * FP + pos) = pf[k];
        else *reinterpret_cast<u32x4_t*>(ft + pos * 32 + (c >> 24) * 8) = pf[k];
      }
    }
    if constexpr (FL == 3) {
      // Position p of channel e is half p of pgw[k][e]; slot p gathers the
      // eight channels of position p (v_perm picks the 16-bit halves).  A
      // position outside the tile row is written to this thread's trash slot
      // (past both buffers) instead of being branched around.
      // Offsets in halves from `tiles`, chosen by masking (a select of
      // pointers becomes a branch per position).
      const uint32_t toff = (uint32_t)(2 * TILE + tid * 8);
      const uint32_t gbase = (uint32_t)(gtl - tiles);
#pragma unroll
      for (int k = 0; k < NGW; ++k) {
        if (k > 0 && wvu != XW) break;
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const uint32_t sel = (p & 1) ? 0x07060302u : 0x05040100u;
          u32x4_t v;
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = __builtin_amdgcn_perm(pgw[k][2 * q + 1][p >> 1], pgw[k][2 * q][p >> 1], sel);
          const uint32_t keep = 0u - (uint32_t)((gwmask[k] >> p) & 1);
          const uint32_t o = toff ^ (((gbase + (uint32_t)(gwslot[k] + p * 32)) ^ toff) & keep);
          *reinterpret_cast<u32x4_t*>(tiles + o) = v;
        }
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < NGI; ++k) {
      const int c = gcode[k];
      if (FL == 2 && c >= 0) {
        const int pos = ((c & 255) * TH + ((c >> 8) & 255)) * 16 + ((c >> 16) & 255);
        *reinterpret_cast<u32x4_t*>(gtl + (c >> 24) * FP + pos) = pg[k];
      } else if (c >= 0) {
        const int hp = ((c & 255) * HH + ((c >> 8) & 255)) * HW + ((c >> 16) & 255);
        *reinterpret_cast<u32x4_t*>(gtl + hp * 32 + (c >> 24) * 8) = pg[k];
      }
    }
  };

  // Per-lane operand addresses (halves) for step 0; a step adds a line.
  const int tw0 = 8 * g + (s >> 2);
  const int fo = tw0 * 32 + 16 * h + 4 * (s & 3);
  int go[CBW];
#pragma unroll
  for (int q = 0; q < CBW; ++q) go[q] = WS * tw0 * 32 + goff[q];
  // Column blocks of this wave (blocks wv, wv + 8, ...): a prefix of q.
  int nv = 0;
#pragma unroll
  for (int q = 0; q < CBW; ++q) nv += cbok[q] ? 1 : 0;

  // Pipeline: box i computes from buffer i % 2.  After the barrier and the
  // first step, box i+1's registers go to the other buffer and box i+2's loads
  // are issued into them, inside the MFMA stream.  The barrier waits for LDS
  // traffic only, so those loads stay in flight across it.
  const int nbx = box_begin < gb1 ? (gb1 - box_begin + s8 - 1) / s8 : 0;
  BoxCur ca = box_at(box_begin < gb1 ? box_begin : 0);
  if (nbx > 0) {
    issue(ca, true);
    box_advance(ca);
    commit(0);
    issue(ca, nbx > 1);
    box_advance(ca);
  }
  constexpr int HOOK = 1;
  // K loop of one box with NV column blocks and, with DBF, the bias MFMA.
  auto run_box = [&](int i, auto buf_c, auto nv_c, auto dbf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    constexpr int NV = decltype(nv_c)::value;
    constexpr bool DBF = decltype(dbf_c)::value;
    const uint16_t* ftile = tiles + BUF * TILE;
    const uint16_t* gtile = ftile + FT;
    uint4 ffr[2], gfr[2][NV > 0 ? NV : 1];
    auto read_step = [&](auto st_c, int slot) __attribute__((always_inline)) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int TD_ = ST / TH, TH_ = ST % TH;
      constexpr int FROW = ST * 16 * 32;
      constexpr int GROW = ((WS * TD_) * HH + WS * TH_) * HW * 32;
      ffr[slot] = FL >= 1 ? *reinterpret_cast<const uint4*>(ftile + li * FP + ST * 16 + 8 * g)
                          : lds_tr_pair(ftile, fo + FROW, fo + FROW + 4 * 32);
#pragma unroll
      for (int q = 0; q < NV; ++q)
        gfr[slot][q] = FL == 2 ? *reinterpret_cast<const uint4*>(gtile + ((q * 8 + wv) * 32 + li) * FP + ST * 16 + 8 * g)
                               : lds_tr_pair(gtile, go[q] + GROW, go[q] + GROW + WS * 4 * 32);
    };
    auto step = [&](auto st_c) __attribute__((always_inline)) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int CUR = ST & 1;
      if constexpr (ST + 1 < LINES) read_step(std::integral_constant<int, ST + 1>{}, CUR ^ 1);
      __builtin_amdgcn_sched_barrier(0);
      if (DBF) accf = mfma32<T>(ffr[CUR], ones, accf);
#pragma unroll
      for (int q = 0; q < NV; ++q) acc[q] = mfma32<T>(ffr[CUR], gfr[CUR][q], acc[q]);
      if constexpr (ST == HOOK) {
        __builtin_amdgcn_sched_barrier(0);
        if (i + 1 < nbx) commit(BUF ^ 1);
        issue(ca, i + 2 < nbx);
        box_advance(ca);
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    read_step(std::integral_constant<int, 0>{}, 0);
    static_for(std::make_integer_sequence<int, LINES>{}, step);
  };
  // The generic box (ConvTranspose, or an uncommon block split) tests each
  // block per step.
  auto run_box_generic = [&](int i, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    const uint16_t* ftile = tiles + BUF * TILE;
    const uint16_t* gtile = ftile + FT;
#pragma unroll
    for (int st = 0; st < LINES; ++st) {
      const int td = st / TH, th = st % TH;
      const int frow = st * 16 * 32;
      const int grow = ((WS * td) * HH + WS * th) * HW * 32;
      const uint4 ffr = FL >= 1 ? *reinterpret_cast<const uint4*>(ftile + li * FP + st * 16 + 8 * g)
                                : lds_tr_pair(ftile, fo + frow, fo + frow + 4 * 32);
      if (do_dbf) accf = mfma32<T>(ffr, ones, accf);
#pragma unroll
      for (int q = 0; q < CBW; ++q) {
        if (!cbok[q]) continue;
        const uint4 gfr = FL == 2 ? *reinterpret_cast<const uint4*>(gtile + ((q * 8 + wv) * 32 + li) * FP + st * 16 + 8 * g)
                                  : lds_tr_pair(gtile, go[q] + grow, go[q] + grow + WS * 4 * 32);
        acc[q] = mfma32<T>(ffr, gfr, acc[q]);
        if (MODE == MODE_T2DW) {
          if (do_dbg) accg[q < NDBG ? q : 0] = mfma32<T>(ones, gfr, accg[q < NDBG ? q : 0]);
        }
      }
      if (st == HOOK) {
        if (i + 1 < nbx) commit(BUF ^ 1);
        issue(ca, i + 2 < nbx);
        box_advance(ca);
      }
    }
  };
  // 0: full blocks, 1: one block fewer, 2: full + bias, 3: one fewer + bias, 4: generic.
  const int kind = (MODE == MODE_T2DW || CBW < 2) ? 4
                   : nv == CBW                  ? (do_dbf ? 2 : 0)
                   : nv == CBW - 1              ? (do_dbf ? 3 : 1)
                                                : 4;
  auto run = [&](int i, auto buf_c) __attribute__((always_inline)) {
    lds_barrier();  // buffer i%2 complete; buffer (i+1)%2 no longer read
    using NF = std::integral_constant<int, (CBW >= 2 ? CBW : 1)>;
    using NL = std::integral_constant<int, (CBW >= 2 ? CBW - 1 : 1)>;
    if (MODE != MODE_T2DW && CBW >= 2 && kind == 0) run_box(i, buf_c, NF{}, std::false_type{});
    else if (MODE != MODE_T2DW && CBW >= 2 && kind == 1) run_box(i, buf_c, NL{}, std::false_type{});
    else if (MODE != MODE_T2DW && CBW >= 2 && kind == 2) run_box(i, buf_c, NF{}, std::true_type{});
    else if (MODE != MODE_T2DW && CBW >= 2 && kind == 3) run_box(i, buf_c, NL{}, std::true_type{});
    else run_box_generic(i, buf_c);
  };
  for (int i = 0; i < nbx; i += 2) {
    run(i, std::integral_constant<int, 0>{});
    if (i + 1 < nbx) run(i + 1, std::integral_constant<int, 1>{});
  }

  // ---- partial store: acc[q][4qq + r] = C[f = 8qq + 4g + r][column li of block]
  const size_t split_stride = (size_t)a.Fpad * TAPS * a.Gpad;
  float* part = a.part + (size_t)split * split_stride;
#pragma unroll
  for (int q = 0; q < CBW; ++q) {
    if (!cbok[q]) continue;
    const int Q = (q * 8 + wv) * 8 + (li >> 2);
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
      const int Q = (q * 8 + wv) * 8 + (li >> 2);
      if (Q >= nquads) continue;
      const int tap = Q / nq;
      const int gch = gc0 + (Q - tap * nq) * 4 + (li & 3);
      a.dbpart[((size_t)split * TAPS + tap) * a.Gpad + gch] = accg[q][0];
    }
  }
}

template <typename T, int MODE, int CBW, int CL, int FL>
static void launch_wgrad_inst(const WgArgs& a, size_t lds, hipStream_t stream) {
  auto kern = wgrad_kernel<T, MODE, CBW, CL, FL>;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3(a.nblocks), dim3(WgGeom<MODE>::THREADS), lds, stream, a);
}

}  // namespace r3c
