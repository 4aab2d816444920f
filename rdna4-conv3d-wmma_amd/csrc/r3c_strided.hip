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

template <typename T, int NB, int SCL, int MB>
__global__ __launch_bounds__(256) void strided_kernel(const StridedArgs a) {
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, li = lane & 31;
  // Workgroups are dealt to the 8 XCDs in turn; renumber them so that each XCD
  // runs a contiguous run of tiles (neighbouring rows and planes, which read
  // the same input rows, share an L2).
  int64_t bid = blockIdx.x;
  const int64_t nblk = gridDim.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int64_t wt = bid * 4 + wv;
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
  // This lane's destination w in each of the MB blocks of 32 and whether it
  // exists.
  int rw[MB];
  bool pos_ok[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const int j = (wb * MB + m) * 32 + li;
    rw[m] = a.dx ? res + a.sw * j : j;
    pos_ok[m] = rw[m] < a.Rw;
  }

  // Taps that reach the tile, per dimension (uniform; in w the tile's
  // residue class makes the dX range the same for every lane), and this
  // lane's source w for the first of them.
  const TapRange td = tap_range(a.dx, rd, a.pd, a.sd, a.k);
  const TapRange th = tap_range(a.dx, rh, a.ph, a.sh, a.k);
  const TapRange tw = tap_range(a.dx, a.dx ? res : rw[0], a.pw, a.sw, a.k);  // k0, step, n, dc: lane-free
  int sw0[MB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
    sw0[m] = a.dx ? (wb * MB + m) * 32 + li + tw.c0 : rw[m] * a.sw - a.pw;
  const int nc16 = a.nc16;
  const int total = td.n * th.n * tw.n * nc16;  // K iterations: (tap d, h, w, channel block)

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[m][nb][e] = 0.f;

  const uint16_t* src = a.src + (int64_t)n * a.ss[0] + (int64_t)(8 * g) * a.ss[1];
  const uint4* wpk = reinterpret_cast<const uint4*>(a.wpk) + (int64_t)ct * NB * 64 + lane;
  // Fragments of K iteration (md, mh, mw, c16), c16 fastest.
  struct KIt {
    int c16, mw, mh, md;
  };
  // live false: the fragment of a padding iteration (zero source values, so
  // its MFMAs add nothing; the weight loads stay in range at ki).
  auto load = [&](const KIt& ki, bool live, uint4 (&bfr)[MB], uint4 (&afr)[NB]) __attribute__((always_inline)) {
    const int c16 = ki.c16, mw = ki.mw, mh = ki.mh, md = ki.md;
    const int kd = td.k0 + md * td.step, kh = th.k0 + mh * th.step, kw = tw.k0 + mw * tw.step;
    // A tile no tap reaches (dX with a large stride) has no live iteration and
    // taps past the kernel in ki: its weight loads use tap 0.
    const int t = (live && a.k == 3) ? (kd * 3 + kh) * 3 + kw : 0;
    const int cd = td.c0 + md * td.dc, ch = th.c0 + mh * th.dc;
    const int kch0 = c16 * 16 + 8 * g;
    const bool row_ok =
        live && (unsigned)cd < (unsigned)a.Sd && (unsigned)ch < (unsigned)a.Sh && kch0 < a.Cs;
    const uint16_t* prow = src + (int64_t)(16 * c16) * a.ss[1] + (int64_t)cd * a.ss[2] + (int64_t)ch * a.ss[3];
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const int cw = sw0[m] + mw * tw.dc;
      const bool ok = row_ok && pos_ok[m] && (unsigned)cw < (unsigned)a.Sw;
      const uint16_t* p = prow + (int64_t)cw * a.ss[4];
      if (SCL) {
        bfr[m] = ok ? *reinterpret_cast<const uint4*>(p) : make_uint4(0u, 0u, 0u, 0u);
      } else {
        uint32_t wd[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint16_t lo = (ok && kch0 + 2 * e < a.Cs) ? p[(int64_t)(2 * e) * a.ss[1]] : (uint16_t)0;
          const uint16_t hi = (ok && kch0 + 2 * e + 1 < a.Cs) ? p[(int64_t)(2 * e + 1) * a.ss[1]] : (uint16_t)0;
          wd[e] = pack2(lo, hi);
        }
        bfr[m] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
    }
    const uint4* wrow = wpk + ((int64_t)c16 * a.taps + t) * a.nbt * 64;
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) afr[nb] = wrow[nb * 64];
  };

  // Software pipeline, PF iterations deep: slot u holds the fragments of an
  // iteration it + u; after its MFMAs the slot loads iteration it + u + PF.
  // The iteration count is padded to a multiple of PF with zero fragments, so
  // every load is unconditional and each MFMA waits only for its own slot.
  // The iteration counters advance by carries, no divisions.  With MB = 2 a
  // weight fragment feeds two MFMAs (the vector-memory data path, not the
  // MFMAs, bounds this kernel).
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
  uint4 bq[PF][MB], aq[PF][NB];
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
      for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[m][nb] = mfma32<T>(aq[u][nb], bq[u][m], acc[m][nb]);
      fetch(u);
    }
  }

  // Epilogue: acc[m][nb][4q + r] = destination channel (ct NB + nb) 32 + 8 q + 4 g + r
  // at this lane's position of block m.
  if (a.dtile) {
    // Each block of 32 positions (all Cd channels) is one contiguous run of
    // the destination: through this wave's LDS block [32 positions][P] and out
    // as 16-byte chunks, consecutive lanes on consecutive chunks.  A wave's
    // LDS operations complete in order, so block m + 1's writes follow block
    // m's reads.
    constexpr int P = 32 * NB + 8;
    __shared__ __align__(16) uint16_t s_tile[4 * 32 * P];
    uint16_t* tb = s_tile + wv * (32 * P);
    const int cpp = a.Cd >> 3;  // 16-byte chunks per position
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const int w0 = (wb * MB + m) * 32;
      if (w0 >= a.Rw) break;  // uniform
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c0 = nb * 32 + 8 * q + 4 * g;
          float v[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            v[rr] = acc[m][nb][4 * q + rr] + ((a.b && c0 + rr < a.Cd) ? to_f32<T>(a.b[c0 + rr]) : 0.f);
          *reinterpret_cast<uint2*>(tb + li * P + c0) = make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])),
                                                                   pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
        }
      const int npos = min(32, a.Rw - w0);
      uint16_t* dp = a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] +
                     (int64_t)w0 * a.Cd;
      for (int k = lane; k < npos * cpp; k += 64) {
        const int pos = k / cpp, c8 = k - pos * cpp;
        *reinterpret_cast<uint4*>(dp + (int64_t)pos * a.Cd + 8 * c8) =
            *reinterpret_cast<const uint4*>(tb + pos * P + 8 * c8);
      }
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    if (!pos_ok[m]) continue;
    uint16_t* dp =
        a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] + (int64_t)rw[m] * a.sd5[4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = (ct * NB + nb) * 32 + 8 * q + 4 * g;
        if ((ct * NB + nb) * 32 + 8 * q >= a.Cd) break;  // uniform
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          v[rr] = acc[m][nb][4 * q + rr] + ((a.b && c0 + rr < a.Cd) ? to_f32<T>(a.b[c0 + rr]) : 0.f);
        if (a.dvec4) {  // channels contiguous, Cd % 4 == 0: one 8-byte store
          if (c0 < a.Cd)
            *reinterpret_cast<uint2*>(dp + c0) = make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])),
                                                            pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
        } else {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (c0 + rr < a.Cd) dp[(int64_t)(c0 + rr) * a.sd5[1]] = from_f32<T>(v[rr]);
        }
      }
  }
}

// Forward, k = 3, w stride SW (1 or 2), at most 32 source channels (NC
// 16-channel blocks): the x operand through the wave's LDS.  Per (kd, kh) the wave's input row segment (the SEGP positions its
// 32 MB outputs read for kw = 0 .. 2) is loaded with 16-byte loads of
// consecutive (position, 8-channel group) chunks -- whole row runs when
// positions are contiguous, instead of one 16-byte fragment at each of 32
// strided positions per tap -- and stored [position][channel group] with a
// pitch of 2 NC + 1 slots (conflict-free 16-byte reads at stride 1 or 2).
// The three kw taps then read their fragments from LDS.  The next row
// segment is in registers while the current one is multiplied; the segment
// block is private to the wave (in-order LDS).  The weight fragments of a
// stage (3 kw x NC x NB) are loaded once per workgroup into shared LDS
// between two barriers (all four waves step through the same nine stages;
// a wave past the last tile takes part without loading or storing), the
// next stage's in registers meanwhile.  Tile order and epilogue as in
// strided_kernel.  At least 3 waves per SIMD: the register cap that implies
// (168) holds every instantiation but NB 2, MB 2, CF 4 without spills (the
// host gives that case one position block).
// CF = 0: channel-contiguous source.  CF = 1 .. 4: an NCDHW source with CF
// 8-channel groups (Cs = 8 CF, W % 8 == 0), read in place: a lane item is
// (8 aligned positions, 8-channel group), eight 16-byte loads of one row run
// per channel, transposed in registers (v_perm) into 8 position slots, as
// the tap kernel stages NCDHW tiles.
// Workgroup barrier for LDS hand-off only: waits for this wave's LDS
// accesses (lgkmcnt 0) and not for its global loads, so register prefetches
// stay in flight across it.
__device__ __forceinline__ void lds_barrier_w() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

template <typename T, int NB, int MB, int SW, int NC, int CF>
__global__ __launch_bounds__(256, 3) void strided_fwd_rs_kernel(const StridedArgs a) {
  constexpr int SEGP = (32 * MB - 1) * SW + 3;  // positions of a row segment
  constexpr int PPS = 2 * NC + 1;                // slots (16 bytes) per position
  constexpr int SEGSLOTS = SEGP * PPS;
  constexpr int P = 32 * NB + 8;                 // epilogue pitch (halves)
  constexpr int WSLOTS = SEGSLOTS > 4 * P ? SEGSLOTS : 4 * P;
  constexpr int NQ = CF ? 1 : (SEGP * 2 * NC + 63) / 64;   // channel-last chunks per lane (upper bound)
  constexpr int NS8 = (SEGP + 14) / 8;                      // CF: 8-position runs covering a segment
  constexpr int NQC = CF ? (NS8 * CF + 63) / 64 : 1;        // CF: items per lane
  static_assert(!CF || (CF + 1) / 2 == NC, "CF channel groups fill NC 16-channel blocks");
  constexpr int WFR = 3 * NC * NB * 64;  // weight fragments of one (kd, kh) stage
  constexpr int WIT = (WFR + 255) / 256;  // per thread
  __shared__ uint4 s_seg[4 * WSLOTS];
  __shared__ uint4 s_w[WFR];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, li = lane & 31;
  int64_t bid = blockIdx.x;
  const int64_t nblk = gridDim.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int64_t wt = bid * 4 + wv;
  // Every wave stays for the workgroup barriers of the weight stages; a wave
  // past the last tile loads nothing and stores nothing.
  const bool tile_ok = wt < a.ntiles;
  int64_t r = tile_ok ? wt : 0;
  const int ct = (int)(r % a.n_ctiles);
  r /= a.n_ctiles;
  const int wb = (int)(r % a.nwb);
  r /= a.nwb;
  const int rh = (int)(r % a.Rh);
  r /= a.Rh;
  const int rd = (int)(r % a.Rd);
  const int n = (int)(r / a.Rd);
  const int ow0 = wb * MB * 32;
  const int iw0 = ow0 * SW - a.pw;
  uint4* sb = s_seg + wv * WSLOTS;

  // Channel-group slots past Cs (K padding of the last block) stay zero.
  const int CG = CF ? CF : a.Cs >> 3;  // 8-channel groups present (Cs % 8 == 0)
  const int npad = 2 * NC - CG;         // K-padding groups per position
  if (npad > 0)
    for (int q = lane; q < SEGP * npad; q += 64) {
      const int pos = q / npad, cg = CG + q % npad;
      sb[pos * PPS + cg] = make_uint4(0u, 0u, 0u, 0u);
    }
  // Channel-last: this lane's chunks of a segment, element offset within the
  // row (-1: none or outside the row) and LDS slot.
  int goff[NQ], loff[NQ];
  // CF: this lane's items, element offset of channel 8 cg at the run's first
  // position (-1: none or outside the row), first segment position (may be
  // below 0) and channel group.
  int coff[NQC], cpos[NQC], ccg[NQC];
  const int a0 = iw0 - (((iw0 % 8) + 8) % 8);  // iw0 rounded down to a multiple of 8
  if constexpr (!CF) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) {
      const int q = lane + 64 * i;
      const int pos = q / CG, cg = q - (q / CG) * CG;
      const int iw = iw0 + pos;
      const bool in = q < SEGP * CG;
      loff[i] = in ? pos * PPS + cg : -1;
      goff[i] = (in && (unsigned)iw < (unsigned)a.Sw) ? (int)((int64_t)iw * a.ss[4]) + 8 * cg : -1;
    }
  } else {
    const int ns8 = (iw0 - a0 + SEGP + 7) >> 3;
#pragma unroll
    for (int i = 0; i < NQC; ++i) {
      const int it = lane + 64 * i;
      const int ps = it / CF, cg = it - (it / CF) * CF;
      const int w8 = a0 + 8 * ps;
      const bool in = it < ns8 * CF;
      cpos[i] = in ? w8 - iw0 : SEGP;  // SEGP: no position of it is stored
      ccg[i] = cg;
      coff[i] = (in && w8 >= 0 && w8 < a.Sw) ? w8 + (int)(8 * cg * a.ss[1]) : -1;
    }
  }
  const uint16_t* src = a.src + (int64_t)n * a.ss[0];
  uint4 pf[NQ];
  uint4 pc[NQC][8];
  auto issue = [&](int st) __attribute__((always_inline)) {
    const int kd = st / 3, kh = st - (st / 3) * 3;
    const int id = rd * a.sd - a.pd + kd, ih = rh * a.sh - a.ph + kh;
    const bool row_ok = tile_ok && (unsigned)id < (unsigned)a.Sd && (unsigned)ih < (unsigned)a.Sh;
    const uint16_t* rowp = src + (int64_t)id * a.ss[2] + (int64_t)ih * a.ss[3];
    if constexpr (!CF) {
#pragma unroll
      for (int i = 0; i < NQ; ++i)
        pf[i] = (row_ok && goff[i] >= 0) ? *reinterpret_cast<const uint4*>(rowp + goff[i]) : make_uint4(0u, 0u, 0u, 0u);
    } else {
#pragma unroll
      for (int i = 0; i < NQC; ++i)
#pragma unroll
        for (int e = 0; e < 8; ++e)
          pc[i][e] = (row_ok && coff[i] >= 0)
                         ? *reinterpret_cast<const uint4*>(rowp + coff[i] + (int64_t)e * a.ss[1])
                         : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  auto commit = [&]() __attribute__((always_inline)) {
    if constexpr (!CF) {
#pragma unroll
      for (int i = 0; i < NQ; ++i)
        if (loff[i] >= 0) sb[loff[i]] = pf[i];
    } else {
      // 8 channels x 8 positions -> 8 slots of 8 channels (position p of
      // channel e is half p of pc[e]).
#pragma unroll
      for (int i = 0; i < NQC; ++i)
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const int pos = cpos[i] + p;
          if ((unsigned)pos >= (unsigned)SEGP) continue;
          const uint32_t sel = (p & 1) ? 0x07060302u : 0x05040100u;
          const int m = p >> 1;
          uint4 v;
          uint32_t* vv = reinterpret_cast<uint32_t*>(&v);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4& lo = pc[i][2 * q];
            const uint4& hi = pc[i][2 * q + 1];
            const uint32_t l = m == 0 ? lo.x : (m == 1 ? lo.y : (m == 2 ? lo.z : lo.w));
            const uint32_t h = m == 0 ? hi.x : (m == 1 ? hi.y : (m == 2 ? hi.z : hi.w));
            vv[q] = __builtin_amdgcn_perm(h, l, sel);
          }
          sb[pos * PPS + ccg[i]] = v;
        }
    }
  };

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[m][nb][e] = 0.f;
  // Weight fragments of a stage: loaded by the whole workgroup into s_w
  // ([kw][c][nb][lane]), the next stage's in registers meanwhile (one column
  // tile: ct == 0).
  const uint4* wsrc = reinterpret_cast<const uint4*>(a.wpk);
  const int tid = threadIdx.x;
  uint4 wreg[WIT];
  auto wissue = [&](int st) __attribute__((always_inline)) {
#pragma unroll
    for (int k2 = 0; k2 < WIT; ++k2) {
      const int f = tid + 256 * k2;
      const int ln = f & 63, rest = f >> 6;
      const int nb = rest % NB, c = (rest / NB) % NC, kw = rest / (NB * NC);
      wreg[k2] = (f < WFR && st < 9) ? wsrc[((int64_t)(c * a.taps + st * 3 + kw) * a.nbt + nb) * 64 + ln]
                                     : make_uint4(0u, 0u, 0u, 0u);
    }
  };
  (void)ct;
  wissue(0);
  issue(0);
  commit();
  issue(1);
  for (int st = 0; st < 9; ++st) {
    lds_barrier_w();  // every wave is done with the previous stage's weights
#pragma unroll
    for (int k2 = 0; k2 < WIT; ++k2)
      if (tid + 256 * k2 < WFR) s_w[tid + 256 * k2] = wreg[k2];
    lds_barrier_w();  // this stage's weights are in s_w
    wissue(st + 1);
    __asm__ volatile("" ::: "memory");  // the segment's LDS writes stay ahead of its reads
    uint4 wf[3][NC][NB];
#pragma unroll
    for (int kw = 0; kw < 3; ++kw)
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) wf[kw][c][nb] = s_w[((kw * NC + c) * NB + nb) * 64 + lane];
#pragma unroll
    for (int kw = 0; kw < 3; ++kw)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        uint4 bf[MB];
#pragma unroll
        for (int m = 0; m < MB; ++m) bf[m] = sb[((m * 32 + li) * SW + kw) * PPS + 2 * c + g];
#pragma unroll
        for (int m = 0; m < MB; ++m)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[m][nb] = mfma32<T>(wf[kw][c][nb], bf[m], acc[m][nb]);
      }
    __asm__ volatile("" ::: "memory");  // this segment's LDS reads are issued before the next one's writes
    if (st + 1 < 9) {
      commit();
      if (st + 2 < 9) issue(st + 2);
    }
  }

  // Epilogue: acc[m][nb][4q + r] = destination channel (ct NB + nb) 32 + 8 q + 4 g + r
  // at position ow0 + 32 m + li.
  if (!tile_ok) return;
  if (a.dtile) {
    uint16_t* tb = reinterpret_cast<uint16_t*>(sb);
    const int cpp = a.Cd >> 3;
#pragma unroll
    for (int m = 0; m < MB; ++m) {
      const int w0 = ow0 + 32 * m;
      if (w0 >= a.Rw) break;  // uniform
      __asm__ volatile("" ::: "memory");
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c0 = nb * 32 + 8 * q + 4 * g;
          float v[4];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            v[rr] = acc[m][nb][4 * q + rr] + ((a.b && c0 + rr < a.Cd) ? to_f32<T>(a.b[c0 + rr]) : 0.f);
          *reinterpret_cast<uint2*>(tb + li * P + c0) = make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])),
                                                                   pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
        }
      const int npos = min(32, a.Rw - w0);
      uint16_t* dp = a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] +
                     (int64_t)w0 * a.Cd;
      for (int k = lane; k < npos * cpp; k += 64) {
        const int pos = k / cpp, c8 = k - pos * cpp;
        *reinterpret_cast<uint4*>(dp + (int64_t)pos * a.Cd + 8 * c8) =
            *reinterpret_cast<const uint4*>(tb + pos * P + 8 * c8);
      }
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const int rw = ow0 + 32 * m + li;
    if (rw >= a.Rw) continue;
    uint16_t* dp =
        a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] + (int64_t)rw * a.sd5[4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = (ct * NB + nb) * 32 + 8 * q + 4 * g;
        if ((ct * NB + nb) * 32 + 8 * q >= a.Cd) break;  // uniform
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          v[rr] = acc[m][nb][4 * q + rr] + ((a.b && c0 + rr < a.Cd) ? to_f32<T>(a.b[c0 + rr]) : 0.f);
        if (a.dvec4) {
          if (c0 < a.Cd)
            *reinterpret_cast<uint2*>(dp + c0) = make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])),
                                                            pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
        } else {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (c0 + rr < a.Cd) dp[(int64_t)(c0 + rr) * a.sd5[1]] = from_f32<T>(v[rr]);
        }
      }
  }
}

// dX counterpart of strided_fwd_rs_kernel (k = 3, w stride SW 1 or 2, dY
// channel-contiguous with at most 64 channels): a tile is 32 MB positions of
// one residue class of w, whose dY positions for tap mw are consecutive
// (j + c0 - mw), so per (md, mh) the wave loads the dY row segment of
// 32 MB + tw.n - 1 positions into its LDS block as whole row runs and reads
// each tap's fragments from there.  Only the taps that reach the tile's
// residue class are visited (as in strided_kernel); a tile that none reach
// stores zeros.
template <typename T, int NB, int MB, int SW, int NC>
__global__ __launch_bounds__(256, 3) void strided_dx_rs_kernel(const StridedArgs a) {
  constexpr int SEGMAX = 32 * MB + 2;  // positions of a row segment, at most
  constexpr int PPS = 2 * NC + 1;
  constexpr int P = 32 * NB + 8;
  constexpr int SEGSLOTS = SEGMAX * PPS;
  constexpr int WSLOTS = SEGSLOTS > 4 * P ? SEGSLOTS : 4 * P;
  constexpr int NQ = (SEGMAX * 2 * NC + 63) / 64;
  __shared__ uint4 s_seg[4 * WSLOTS];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5, li = lane & 31;
  int64_t bid = blockIdx.x;
  const int64_t nblk = gridDim.x;
  if ((nblk & 7) == 0) bid = (bid & 7) * (nblk >> 3) + (bid >> 3);
  const int64_t wt = bid * 4 + wv;
  if (wt >= a.ntiles) return;  // no barrier in this kernel
  int64_t r = wt;
  const int ct = (int)(r % a.n_ctiles);
  r /= a.n_ctiles;
  const int wb = (int)(r % a.nwb);
  r /= a.nwb;
  const int res = (int)(r % SW);
  r /= SW;
  const int rh = (int)(r % a.Rh);
  r /= a.Rh;
  const int rd = (int)(r % a.Rd);
  const int n = (int)(r / a.Rd);
  const TapRange td = tap_range(true, rd, a.pd, a.sd, 3);
  const TapRange th = tap_range(true, rh, a.ph, a.sh, 3);
  const TapRange tw = tap_range(true, res, a.pw, SW, 3);
  const int j0 = wb * MB * 32;
  const int seg = 32 * MB + (tw.n > 0 ? tw.n - 1 : 0);  // positions loaded
  const int s0 = j0 + tw.c0 - (tw.n > 0 ? tw.n - 1 : 0);  // first dY w of the segment
  uint4* sb = s_seg + wv * WSLOTS;

  const int CG = a.Cs >> 3;
  for (int q = lane; q < SEGMAX * (2 * NC - CG); q += 64) {
    const int pos = q / (2 * NC - CG), cg = CG + q % (2 * NC - CG);
    sb[pos * PPS + cg] = make_uint4(0u, 0u, 0u, 0u);
  }
  int goff[NQ], loff[NQ];
#pragma unroll
  for (int i = 0; i < NQ; ++i) {
    const int q = lane + 64 * i;
    const int pos = q / CG, cg = q - (q / CG) * CG;
    const int cw = s0 + pos;
    const bool in = q < seg * CG;
    loff[i] = in ? pos * PPS + cg : -1;
    goff[i] = (in && (unsigned)cw < (unsigned)a.Sw) ? (int)((int64_t)cw * a.ss[4]) + 8 * cg : -1;
  }
  const uint16_t* src = a.src + (int64_t)n * a.ss[0];
  const int nst = td.n * th.n;
  uint4 pf[NQ];
  auto issue = [&](int st) __attribute__((always_inline)) {
    const int md = st / (th.n > 0 ? th.n : 1), mh = st - md * (th.n > 0 ? th.n : 1);
    const int cd = td.c0 + md * td.dc, ch = th.c0 + mh * th.dc;
    const bool row_ok = st < nst && (unsigned)cd < (unsigned)a.Sd && (unsigned)ch < (unsigned)a.Sh;
    const uint16_t* rowp = src + (int64_t)cd * a.ss[2] + (int64_t)ch * a.ss[3];
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      pf[i] = (row_ok && goff[i] >= 0) ? *reinterpret_cast<const uint4*>(rowp + goff[i]) : make_uint4(0u, 0u, 0u, 0u);
  };
  auto commit = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      if (loff[i] >= 0) sb[loff[i]] = pf[i];
  };

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int m = 0; m < MB; ++m)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[m][nb][e] = 0.f;
  const uint4* wpk = reinterpret_cast<const uint4*>(a.wpk) + (int64_t)ct * NB * 64 + lane;

  if (nst > 0 && tw.n > 0) {
    issue(0);
    commit();
    issue(1);
    for (int st = 0; st < nst; ++st) {
      __asm__ volatile("" ::: "memory");  // the segment's LDS writes stay ahead of its reads
      const int md = st / th.n, mh = st - md * th.n;
      const int kd = td.k0 + md * td.step, kh = th.k0 + mh * th.step;
      for (int mw = 0; mw < tw.n; ++mw) {  // uniform, at most 3
        const int kw = tw.k0 + mw * tw.step;
        const int t = (kd * 3 + kh) * 3 + kw;
        uint4 wf[NC][NB];
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) wf[c][nb] = wpk[((int64_t)(c * a.taps + t) * a.nbt + nb) * 64];
        const int pb = tw.n - 1 - mw;  // segment position of this tap's first lane, block 0
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          uint4 bf[MB];
#pragma unroll
          for (int m = 0; m < MB; ++m) bf[m] = sb[(m * 32 + li + pb) * PPS + 2 * c + g];
#pragma unroll
          for (int m = 0; m < MB; ++m)
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) acc[m][nb] = mfma32<T>(wf[c][nb], bf[m], acc[m][nb]);
        }
      }
      __asm__ volatile("" ::: "memory");  // this segment's LDS reads are issued before the next one's writes
      if (st + 1 < nst) {
        commit();
        if (st + 2 < nst) issue(st + 2);
      }
    }
  }

  // Epilogue: acc[m][nb][4q + r] = destination channel (ct NB + nb) 32 + 8 q + 4 g + r at
  // w = res + SW (j0 + 32 m + li).
#pragma unroll
  for (int m = 0; m < MB; ++m) {
    const int rw = res + SW * (j0 + 32 * m + li);
    if (rw >= a.Rw) continue;
    uint16_t* dp =
        a.dst + (int64_t)n * a.sd5[0] + (int64_t)rd * a.sd5[2] + (int64_t)rh * a.sd5[3] + (int64_t)rw * a.sd5[4];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c0 = (ct * NB + nb) * 32 + 8 * q + 4 * g;
        if ((ct * NB + nb) * 32 + 8 * q >= a.Cd) break;  // uniform
        float v[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) v[rr] = acc[m][nb][4 * q + rr];
        if (a.dvec4) {
          if (c0 < a.Cd)
            *reinterpret_cast<uint2*>(dp + c0) = make_uint2(pack2(from_f32<T>(v[0]), from_f32<T>(v[1])),
                                                            pack2(from_f32<T>(v[2]), from_f32<T>(v[3])));
        } else {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr)
            if (c0 + rr < a.Cd) dp[(int64_t)(c0 + rr) * a.sd5[1]] = from_f32<T>(v[rr]);
        }
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

// Direct strided dW + db: D[co][ci] of tap t summed over output positions.
// Wave w = (kd, kh) of a workgroup holds the 3 kw taps of one 32 x 32
// (Cout, Cin) block pair.  K block = 16 output positions (n, od, oh, ow0 ..
// ow0 + 15) of one row: the dY operand (rows = output channels) is one 16-byte
// load per lane (positions ow0 + 8 g ..), the x operand (columns = input
// channels) needs, for kw, input positions SW (ow0 + 8 g + e) - pw + kw: a
// window of aligned 16-byte loads plus edge dwords around SW (ow0 + 8 g),
// from which v_alignbit (SW 1) or v_perm (SW 2, every other element) picks
// the 8 values.  Input rows outside the volume (padding) contribute zeros; the
// loads of the next PF K blocks are in flight while the current one multiplies.
// db: wave 0 sums its dY fragments.  One partial per workgroup, added by the
// fixed-order reduce.  The w padding is 1: with W % 8 == 0 and OW % 16 == 0 it
// is the only padding a 3-tap window of w stride 1 or 2 allows, and it makes the
// window picks compile-time register selections.
template <typename T, int SW, int NCB>
__global__ __launch_bounds__(576) void strided_dw_kernel(const StridedDwArgs a) {
  constexpr int NW = SW == 1 ? 6 : 10;  // window dwords: edge, 16 (SW 1) or 32 (SW 2) bytes, edge
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // kd * 3 + kh
  const int kd = wv / 3, kh = wv % 3;
  const int g = lane >> 5, li = lane & 31;
  // Workgroups are dealt to the 8 XCDs in turn; renumber them so that each XCD
  // runs a contiguous run of (split, tile) pairs, tile fastest: the tiles of a
  // split and neighbouring splits (which share input planes) share an L2.
  const int ntile = a.ncg * a.ngb;
  const int total = a.nsplit * ntile;
  int bid = blockIdx.x;
  if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
  const int tile = bid % ntile, split = bid / ntile;
  const int cb = tile / a.ngb, gb = tile % a.ngb;
  const int64_t k0 = ((int64_t)split * a.nkb) / a.nsplit, k1 = ((int64_t)(split + 1) * a.nkb) / a.nsplit;
  const int ci = gb * 32 + li;
  const bool ci_ok = ci < a.Cin;
  int co[NCB];
  bool co_ok[NCB];
#pragma unroll
  for (int nc = 0; nc < NCB; ++nc) {
    co[nc] = (cb * NCB + nc) * 32 + li;
    co_ok[nc] = co[nc] < a.Cout;
  }
  const int kpr = a.OW >> 4;  // K blocks per output row
  f32x16_t acc[NCB][3];
#pragma unroll
  for (int nc = 0; nc < NCB; ++nc)
#pragma unroll
    for (int k = 0; k < 3; ++k)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[nc][k][e] = 0.f;
  float dbs[NCB];
#pragma unroll
  for (int nc = 0; nc < NCB; ++nc) dbs[nc] = 0.f;

  struct Frag {
    uint4 af[NCB];
    uint32_t win[NW];
  };
  // K block position (n, od, oh, owb), owb fastest; advanced by carries.
  struct KPos {
    int owb, oh, od, n;
  };
  auto load = [&](const KPos& kp, bool live, Frag& f) __attribute__((always_inline)) {
    const int ow0 = kp.owb * 16;
    const uint16_t* yr = a.dy + (int64_t)kp.n * a.ys0 + (int64_t)kp.od * a.ys2 + (int64_t)kp.oh * a.ys3 + ow0 + 8 * g;
#pragma unroll
    for (int nc = 0; nc < NCB; ++nc) {
      f.af[nc] = make_uint4(0u, 0u, 0u, 0u);
      if (live && co_ok[nc]) f.af[nc] = *reinterpret_cast<const uint4*>(yr + (int64_t)co[nc] * a.ys1);
    }
    const int id = kp.od * a.sd - a.pd + kd, ih = kp.oh * a.sh - a.ph + kh;
    const bool row_ok = live && ci_ok && (unsigned)id < (unsigned)a.D && (unsigned)ih < (unsigned)a.H;
    const uint16_t* xr =
        a.x + (int64_t)kp.n * a.xs0 + (int64_t)ci * a.xs1 + (int64_t)id * a.xs2 + (int64_t)ih * a.xs3;
    const int b = SW * (ow0 + 8 * g);  // first input position of the window's aligned part
#pragma unroll
    for (int k = 0; k < NW; ++k) f.win[k] = 0u;
    if (row_ok) {
      if (b >= 2) f.win[0] = *reinterpret_cast<const uint32_t*>(xr + b - 2);
#pragma unroll
      for (int c = 0; c < SW; ++c)
        if (b + 8 * c < a.W) {
          const uint4 m = *reinterpret_cast<const uint4*>(xr + b + 8 * c);
          f.win[1 + 4 * c] = m.x;
          f.win[2 + 4 * c] = m.y;
          f.win[3 + 4 * c] = m.z;
          f.win[4 + 4 * c] = m.w;
        }
      if (b + 8 * SW < a.W) f.win[NW - 1] = *reinterpret_cast<const uint32_t*>(xr + b + 8 * SW);
    }
  };
  auto compute = [&](const Frag& f) __attribute__((always_inline)) {
    if (wv == 0) {
#pragma unroll
      for (int nc = 0; nc < NCB; ++nc) {
        const uint32_t q[4] = {f.af[nc].x, f.af[nc].y, f.af[nc].z, f.af[nc].w};
#pragma unroll
        for (int e = 0; e < 4; ++e)
          dbs[nc] += to_f32<T>((uint16_t)(q[e] & 0xffff)) + to_f32<T>((uint16_t)(q[e] >> 16));
      }
    }
#pragma unroll
    for (int kw = 0; kw < 3; ++kw) {
      // Window element of value e: j = (kw - pw + 2) + SW e (window element 0 =
      // input position b - 2).
      const int o = kw + 1;  // 1 .. 3
      const int w0 = o >> 1;
      const bool odd = (o & 1) != 0;
      uint32_t bw[4];
      if (SW == 1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = w0 == 0 ? f.win[q] : (w0 == 1 ? f.win[q + 1] : f.win[q + 2]);
          const uint32_t hi = w0 == 0 ? f.win[q + 1] : (w0 == 1 ? f.win[q + 2] : (q + 3 < NW ? f.win[q + 3] : 0u));
          bw[q] = __builtin_amdgcn_alignbit(hi, lo, odd ? 16u : 0u);
        }
      } else {
        const uint32_t sel = odd ? 0x07060302u : 0x05040100u;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          // values 2q, 2q + 1: window elements o + 4q and o + 4q + 2 (same half)
          const uint32_t lo = w0 == 0 ? f.win[2 * q] : (w0 == 1 ? f.win[2 * q + 1] : f.win[2 * q + 2]);
          const uint32_t hi = w0 == 0 ? f.win[2 * q + 1] : (w0 == 1 ? f.win[2 * q + 2] : f.win[2 * q + 3]);
          bw[q] = __builtin_amdgcn_perm(hi, lo, sel);
        }
      }
      const uint4 bq = make_uint4(bw[0], bw[1], bw[2], bw[3]);
#pragma unroll
      for (int nc = 0; nc < NCB; ++nc) acc[nc][kw] = mfma32<T>(f.af[nc], bq, acc[nc][kw]);
    }
  };

  // Software pipeline, PF K blocks deep: slot u holds block kb + u and, after
  // its MFMAs, loads block kb + u + PF.  The count is padded to a multiple of
  // PF with zero fragments (live false), so each MFMA waits only for its slot.
  constexpr int PF = NCB == 1 ? 3 : 2;
  const int nk = (int)(k1 - k0);
  KPos kn;
  {
    int64_t r = k0;
    kn.owb = (int)(r % kpr);
    r /= kpr;
    kn.oh = (int)(r % a.OH);
    r /= a.OH;
    kn.od = (int)(r % a.OD);
    kn.n = (int)(r / a.OD);
  }
  auto advance = [&](KPos& kp) __attribute__((always_inline)) {
    if (++kp.owb < kpr) return;
    kp.owb = 0;
    if (++kp.oh < a.OH) return;
    kp.oh = 0;
    if (++kp.od < a.OD) return;
    kp.od = 0;
    ++kp.n;
  };
  int loaded = 0;
  Frag q[PF];
  auto fetch = [&](int u) __attribute__((always_inline)) {
    const bool live = loaded < nk;
    load(kn, live, q[u]);
    ++loaded;
    if (loaded < nk) advance(kn);
  };
#pragma unroll
  for (int u = 0; u < PF; ++u) fetch(u);
  for (int it = 0; it < nk; it += PF) {
#pragma unroll
    for (int u = 0; u < PF; ++u) {
      compute(q[u]);
      fetch(u);
    }
  }

  // Partials: acc[nc][kw][4 q + r] = D[co = (cb NCB + nc) 32 + 8 q + 4 g + r][ci = gb 32 + li]
  // of tap (kd, kh, kw).
  float* part = a.part + (size_t)split * a.Cout * 27 * a.Cin;
#pragma unroll
  for (int nc = 0; nc < NCB; ++nc)
#pragma unroll
    for (int kw = 0; kw < 3; ++kw) {
      const int t = wv * 3 + kw;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int c = (cb * NCB + nc) * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
        if (c < a.Cout && ci_ok) part[((size_t)c * 27 + t) * a.Cin + ci] = acc[nc][kw][v];
      }
    }
  if (wv == 0 && gb == 0 && a.dbpart) {
#pragma unroll
    for (int nc = 0; nc < NCB; ++nc) {
      const float tot = dbs[nc] + __shfl_xor(dbs[nc], 32);  // the two position halves of channel co, in a fixed order
      if (g == 0 && co_ok[nc]) a.dbpart[(size_t)split * a.Cout + co[nc]] = tot;
    }
  }
}

template <typename T, int SCL, int MB>
bool launch_ts(const StridedArgs& a, int nb, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ntiles + 3) / 4);
  switch (nb) {
    case 1: hipLaunchKernelGGL((strided_kernel<T, 1, SCL, MB>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((strided_kernel<T, 2, SCL, MB>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 3: hipLaunchKernelGGL((strided_kernel<T, 3, SCL, MB>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((strided_kernel<T, 4, SCL, MB>), dim3(blocks), dim3(256), 0, s, a); return true;
    default: return false;
  }
}
template <typename T>
bool launch_t(const StridedArgs& a, int nb, hipStream_t s) {
  if (a.mb == 2) return a.scl ? launch_ts<T, 1, 2>(a, nb, s) : false;  // two position blocks: 16-byte loads only
  return a.scl ? launch_ts<T, 1, 1>(a, nb, s) : launch_ts<T, 0, 1>(a, nb, s);
}

template <typename T, int NB, int MB>
bool launch_rs_sw(const StridedArgs& a, int nc, unsigned blocks, hipStream_t s) {
#define R3C_RS(SW_, NC_, CF_) \
  if (a.sw == SW_ && nc == NC_ && cf == CF_) { \
    hipLaunchKernelGGL((strided_fwd_rs_kernel<T, NB, MB, SW_, NC_, CF_>), dim3(blocks), dim3(256), 0, s, a); \
    return true; \
  }
  const int cf = a.chan_first;
  R3C_RS(1, 1, 0) R3C_RS(1, 2, 0) R3C_RS(2, 1, 0) R3C_RS(2, 2, 0)
  R3C_RS(1, 1, 1) R3C_RS(1, 1, 2) R3C_RS(1, 2, 3) R3C_RS(1, 2, 4)
  R3C_RS(2, 1, 1) R3C_RS(2, 1, 2) R3C_RS(2, 2, 3) R3C_RS(2, 2, 4)
#undef R3C_RS
  return false;
}
template <typename T>
bool launch_rs_t(const StridedArgs& a, int nb, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ntiles + 3) / 4);
  if (nb == 1) return a.mb == 2 ? launch_rs_sw<T, 1, 2>(a, a.nc16, blocks, s) : launch_rs_sw<T, 1, 1>(a, a.nc16, blocks, s);
  if (nb == 2) return a.mb == 2 ? launch_rs_sw<T, 2, 2>(a, a.nc16, blocks, s) : launch_rs_sw<T, 2, 1>(a, a.nc16, blocks, s);
  return false;
}

template <typename T, int NB, int MB, int SW>
bool launch_dxrs_nc(const StridedArgs& a, unsigned blocks, hipStream_t s) {
  switch (a.nc16) {
    case 1: hipLaunchKernelGGL((strided_dx_rs_kernel<T, NB, MB, SW, 1>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 2: hipLaunchKernelGGL((strided_dx_rs_kernel<T, NB, MB, SW, 2>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 3: hipLaunchKernelGGL((strided_dx_rs_kernel<T, NB, MB, SW, 3>), dim3(blocks), dim3(256), 0, s, a); return true;
    case 4: hipLaunchKernelGGL((strided_dx_rs_kernel<T, NB, MB, SW, 4>), dim3(blocks), dim3(256), 0, s, a); return true;
    default: return false;
  }
}
template <typename T, int NB, int MB>
bool launch_dxrs_sw(const StridedArgs& a, unsigned blocks, hipStream_t s) {
  return a.sw == 1 ? launch_dxrs_nc<T, NB, MB, 1>(a, blocks, s)
                   : (a.sw == 2 ? launch_dxrs_nc<T, NB, MB, 2>(a, blocks, s) : false);
}
template <typename T>
bool launch_dxrs_t(const StridedArgs& a, int nb, hipStream_t s) {
  const unsigned blocks = (unsigned)((a.ntiles + 3) / 4);
  if (nb == 1) return a.mb == 2 ? launch_dxrs_sw<T, 1, 2>(a, blocks, s) : launch_dxrs_sw<T, 1, 1>(a, blocks, s);
  if (nb == 2) return a.mb == 2 ? launch_dxrs_sw<T, 2, 2>(a, blocks, s) : launch_dxrs_sw<T, 2, 1>(a, blocks, s);
  return false;
}

}  // namespace

void launch_strided_pack(const StridedPackArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(strided_pack_kernel, dim3((unsigned)((a.total + 255) / 256)), dim3(256), 0, s, a);
}

bool launch_strided_fwd_rs(int dtype, int nb, const StridedArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_rs_t<bf16_tag>(a, nb, s) : launch_rs_t<f16_tag>(a, nb, s);
}

bool launch_strided_dx_rs(int dtype, int nb, const StridedArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_dxrs_t<bf16_tag>(a, nb, s) : launch_dxrs_t<f16_tag>(a, nb, s);
}

bool launch_strided(int dtype, int nb, const StridedArgs& a, hipStream_t s) {
  return dtype == DT_BF16 ? launch_t<bf16_tag>(a, nb, s) : launch_t<f16_tag>(a, nb, s);
}

template <typename T, int SW>
void launch_dw_ncb(int ncb, const StridedDwArgs& a, hipStream_t s) {
  const dim3 grid((unsigned)(a.nsplit * a.ncg * a.ngb));
  if (ncb == 2) hipLaunchKernelGGL((strided_dw_kernel<T, SW, 2>), grid, dim3(576), 0, s, a);
  else hipLaunchKernelGGL((strided_dw_kernel<T, SW, 1>), grid, dim3(576), 0, s, a);
}

bool launch_strided_dw(int dtype, int sw, int ncb, const StridedDwArgs& a, hipStream_t s) {
  if ((sw != 1 && sw != 2) || a.pw != 1 || (ncb != 1 && ncb != 2)) return false;
  if (dtype == DT_BF16) {
    if (sw == 1) launch_dw_ncb<bf16_tag, 1>(ncb, a, s);
    else launch_dw_ncb<bf16_tag, 2>(ncb, a, s);
  } else {
    if (sw == 1) launch_dw_ncb<f16_tag, 1>(ncb, a, s);
    else launch_dw_ncb<f16_tag, 2>(ncb, a, s);
  }
  return true;
}

void launch_dilate(const DilateArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(dilate_kernel, dim3((unsigned)((a.rows * (a.W1p / 8) + 255) / 256)), dim3(256), 0, s, a);
}

}  // namespace r3c
