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
#include "r3c_row.h"

namespace r3c {


// CL: G staged by 16-byte channel vectors (else 8 two-byte loads per slot);
// with FL 0 the same holds for F, whose tile is [position][channel] and is read
// with ds_read_tr16_b64.  FL 1: F comes from a w-contiguous source (NCDHW) and
// is staged channel-major, [channel][FP positions], by 16-byte loads of 8
// positions; its A fragment (8 consecutive positions of one channel) is then a
// single ds_read_b128, and the padded pitch (FP = BOXPOS + 8) puts the 16
// lanes of a group on 16 distinct bank slots.  FL 2 (k=1 without padding,
// where G has no tap shift): G is staged and read the same way.
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

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
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
  const int box_begin = (int)(((int64_t)split * a.nbox) / a.nsplit);
  const int box_end = (int)(((int64_t)(split + 1) * a.nbox) / a.nsplit);

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
  auto issue = [&](int box) {
    int b = box;
    const int bw = b % a.nbw;
    b /= a.nbw;
    const int bh = b % a.nbh;
    b /= a.nbh;
    const int bd = b % a.nbd;
    const int n = b / a.nbd;
    const int r0d = bd * Geo::TD, r0h = bh * TH, r0w = bw * 16;
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
#pragma unroll
    for (int k = 0; k < NFI; ++k) {
      const int c = fcode[k];
      const int td = c & 255, th = (c >> 8) & 255, tw = (c >> 16) & 255, cg = c >> 24;
      const int gd = r0d + td, gh = r0h + th, gw = r0w + tw;
      if (FL >= 1) {  // 8 positions gw .. gw+7 of channel fc0 + cg (the planner keeps Rw % 8 == 0)
        const int ch = fc0 + cg;
        const bool ok = c >= 0 && gd < a.Rd && gh < a.Rh && gw < a.Rw && ch < a.Fc;
        const int off = 2 * (gd * fs2 + gh * fs3 + gw + ch * fs1);
        pf[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(fsrc, ok ? off : kOob, 0, 0));
      } else {
        const int c0 = fc0 + cg * 8;
        const bool ok = c >= 0 && gd < a.Rd && gh < a.Rh && gw < a.Rw && c0 < a.Fc;
        const int off = 2 * (gd * fs2 + gh * fs3 + gw * fs4 + c0 * fs1);
        pf[k] = load8(fsrc, ok, off, a.Fc - c0, fs1);
      }
    }
#pragma unroll
    for (int k = 0; k < NGI; ++k) {
      const int c = gcode[k];
      if (FL == 2) {  // 8 positions of channel gc0 + ch (k=1 without padding: G sits on the F grid)
        const int gd = s0d + (c & 255), gh = s0h + ((c >> 8) & 255), gw = s0w + ((c >> 16) & 255);
        const int ch = gc0 + (c >> 24);
        const bool ok = c >= 0 && gd < a.Gd && gh < a.Gh && gw < a.Gw && ch < a.Gc;
        const int off = 2 * (gd * gs2 + gh * gs3 + gw + ch * gs1);
        pg[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(gsrc, ok ? off : kOob, 0, 0));
        continue;
      }
      const int hd = c & 255, hh = (c >> 8) & 255, hw = (c >> 16) & 255, cg = c >> 24;
      const int gd = s0d + hd, gh = s0h + hh, gw = s0w + hw, c0 = gc0 + cg * 8;
      const bool ok = c >= 0 && (unsigned)gd < (unsigned)a.Gd && (unsigned)gh < (unsigned)a.Gh &&
                      (unsigned)gw < (unsigned)a.Gw && c0 < a.Gc;
      const int off = 2 * (gd * gs2 + gh * gs3 + gw * gs4 + c0 * gs1);
      pg[k] = load8(gsrc, ok, off, a.Gc - c0, gs1);
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

  if (box_begin < box_end) {
    issue(box_begin);
    commit(0);
    if (box_begin + 1 < box_end) issue(box_begin + 1);
  }
  for (int box = box_begin; box < box_end; ++box) {
    const int buf = (box - box_begin) & 1;
    __syncthreads();  // buffer buf is complete; buffer buf^1 is no longer read
    if (box + 1 < box_end) {
      commit(buf ^ 1);
      if (box + 2 < box_end) issue(box + 2);  // in flight during the K loop
    }
    const uint16_t* ftile = tiles + buf * TILE;
    const uint16_t* gtile = ftile + FT;

#pragma unroll
    for (int st = 0; st < Geo::LINES; ++st) {
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
    }
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
