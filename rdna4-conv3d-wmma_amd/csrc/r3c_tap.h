// r3c_tap.h -- Conv3d k=3 stride-1 implicit GEMM for gfx950 (forward and dX):
// the "tap kernel", on v_mfma_f32_32x32x16.
//
//   C[position][column] = sum_{tap, ci} X[position + tap - pad][ci] * W[ci, tap][column]
//
// Workgroup: 8 waves (512 threads), one per CU (its LDS takes most of the
// 160 KB).  It owns a box of TD x TH lines of 32 positions and NB column
// blocks of 32; wave w owns lines w*MB .. w*MB+MB-1.  A line is 32 consecutive
// w positions (LW = 32) or, for volumes at most 16 wide, two h rows of 16
// (LW = 16), so narrow layers fill every MFMA row.
//
// K walks (source-channel chunk of 8, tap): per chunk the box plus its
// one-voxel halo is staged into LDS as 16-byte slots (8 channels of one
// position), [position] with rows of LW + 2 slots; the A fragment of tap t is
// one ds_read_b128 per lane at slot row + offset(t).  One MFMA consumes two
// taps (lane halves g = 0, 1); 27 taps make 14 steps.  B fragments are the
// weights pre-packed in lane order (the row kernel's packed format).
//
// Pipeline, per stage (one chunk of one job):
//   barrier (LDS hand-off: buffer t%2 complete, buffer (t+1)%2 free)
//   14 steps of ds_read_b128 + MFMA, with, after the first step:
//     stage t+1's activations (in registers since stage t+1-DIST) -> buffer (t+1)%2
//     stage t+1+DIST's activation loads issued into the freed registers
//     (per-stage weights: stage t+1 committed, stage t+2 loaded)
// so the staging work rides in the MFMA stream instead of in a serial block
// between barriers.  Slot offsets (with the zero-padding test) are computed
// once per job, not per stage; a stage adds one uniform channel offset.
//
// Loads go through a buffer resource with 32-bit offsets; halo positions
// outside the volume use an offset past num_records, which the hardware
// returns as zero.
//
// Index math follows the reference's k3 forward kernel
// (src/rdna4_conv3d/conv3d_wmma.py:372-444); dX is the same computation over
// dY with the flipped, transposed weight and padding k-1-p
// (conv3d_wmma.py:1154-1162, with the padding corrected).
#pragma once
#include <type_traits>
#include <utility>

#include "r3c_row.h"

namespace r3c {

template <int MB, int LW>
struct TapGeom {
  static constexpr int NW = 8;
  static constexpr int NT = 512;
  static constexpr int NSTEP = 14;                    // 27 taps, two per MFMA
  static constexpr int HR = 32 / LW;                  // h rows per line
  // Box: TD x TH lines (8 * MB = NW * MB), fixed per MB so every LDS offset
  // of the K loop is a compile-time immediate.
  static constexpr int TD = MB == 1 ? 2 : 4;
  static constexpr int TH = MB == 4 ? 8 : 4;
  static constexpr int HD = TD + 2;
  static constexpr int HH = TH * HR + 2;
  static constexpr int HW = LW + 2;                   // tile row (slots)
  static constexpr int HPOS = HD * HH * HW;
  static constexpr int HPAD = (HPOS + 15) / 16 * 16;  // slots per activation buffer
  static constexpr int MAXK = (HPOS + NT - 1) / NT;   // staging slots per thread
  // Slot offset of tap t in the tile.
  static constexpr int tap_off(int t) { return ((t / 9) * HH + (t / 3) % 3) * HW + t % 3; }
  // Step s pairs taps 2s (g = 0) and 2s + 1 (g = 1; the 28th is K padding with
  // zero weights and reads tap 26's slot).  The g = 1 offset exceeds the
  // g = 0 one by one of four constants, so a lane keeps four bases per line.
  static constexpr int delta(int s) { return 2 * s + 1 < 27 ? tap_off(2 * s + 1) - tap_off(2 * s) : 0; }
  static constexpr int DELTAS[4] = {1, HW - 2, HH * HW - 2 * HW - 2, 0};
  static constexpr int delta_idx(int s) {
    return delta(s) == 1 ? 0 : delta(s) == HW - 2 ? 1 : delta(s) == 0 ? 3 : 2;
  }
};

// Calls f(integral_constant<int, S>) for S in order (compile-time unrolling).
template <int... S, typename F>
__device__ __forceinline__ void static_for(std::integer_sequence<int, S...>, F&& f) {
  (f(std::integral_constant<int, S>{}), ...);
}

struct TapCursor {
  int chunk, split, ct, bw, bh, bd, n;
  int job;  // job index (the workgroup takes jobs job, job + stride, ...)
};

__device__ __forceinline__ TapCursor tap_cursor_at(const RowArgs& a, int job) {
  TapCursor c;
  c.job = job;
  c.split = job % a.nsplit;
  c.chunk = c.split * a.cps;
  const int tile = job / a.nsplit;
  c.ct = tile % a.n_ctiles;
  int b = tile / a.n_ctiles;
  c.bw = b % a.nbw;
  b /= a.nbw;
  c.bh = b % a.nbh;
  b /= a.nbh;
  c.bd = b % a.nbd;
  c.n = b / a.nbd;
  return c;
}

// Next stage: the next chunk of the job, else the first chunk of job + stride.
// `st` holds the stride's digits in the job index's mixed radix (split, column
// tile, box w, h, d, sample; tap_cursor_at(a, stride)), so moving to the next
// job is a digit-wise add with carries instead of five divisions.  Each digit
// sum is below twice its radix, so one conditional subtraction normalises it.
__device__ __forceinline__ void tap_advance(const RowArgs& a, TapCursor& c, const TapCursor& st) {
  if (++c.chunk < (c.split + 1) * a.cps) return;
  int v = c.split + st.split;
  int cy = v >= a.nsplit;
  c.split = cy ? v - a.nsplit : v;
  v = c.ct + st.ct + cy;
  cy = v >= a.n_ctiles;
  c.ct = cy ? v - a.n_ctiles : v;
  v = c.bw + st.bw + cy;
  cy = v >= a.nbw;
  c.bw = cy ? v - a.nbw : v;
  v = c.bh + st.bh + cy;
  cy = v >= a.nbh;
  c.bh = cy ? v - a.nbh : v;
  v = c.bd + st.bd + cy;
  cy = v >= a.nbd;
  c.bd = cy ? v - a.nbd : v;
  c.n += st.n + cy;
  c.chunk = c.split * a.cps;
  c.job += st.job;
}

// Output tile (box, column tile) of a cursor.
__device__ __forceinline__ int tap_tile(const RowArgs& a, const TapCursor& c) {
  return (((c.n * a.nbd + c.bd) * a.nbh + c.bh) * a.nbw + c.bw) * a.n_ctiles + c.ct;
}

// Epilogue of one wave, straight from registers.  The MFMAs compute C^T (A =
// weights, B = activations), so lane (g, i) of a tile holds columns
// (output channels) 8q + 4g + r, q, r in 0..3, of row (position) i of its
// line: acc[4q + r].  With positions contiguous in memory (NCDHW) a 2-byte
// store per (q, r) writes 32 consecutive positions of a channel per half-wave;
// with channels contiguous (NDHWC) an 8-byte store per q writes 4 channels of
// a position.  Stores go through a buffer resource over the output sample;
// lanes outside the volume or past the last column get an offset with bit 31
// set (past num_records: dropped).  btab[c - bcol0] is the bias of column c.
template <typename T, int NB, int MB, int LW>
__device__ __forceinline__ void tap_epilogue(const RowArgs& a, f32x16_t (&acc)[MB][NB], int wv, int lane,
                                             const TapCursor& ec, const float* btab, int bcol0) {
  constexpr int HR = TapGeom<MB, LW>::HR;
  constexpr int TD = TapGeom<MB, LW>::TD, TH = TapGeom<MB, LW>::TH;
  const int g = lane >> 5, li = lane & 31;
  const int r0d = ec.bd * TD, r0h = ec.bh * TH * HR, r0w = ec.bw * LW;
  const int64_t* sd = a.sd;
  const __amdgpu_buffer_rsrc_t dst1 = make_rsrc(a.dst + (int64_t)ec.n * sd[0], a.dst_bytes);
  // Destination channels >= dsplit (a multiple of 8) go to the second tensor
  // of a channel concatenation.
  const __amdgpu_buffer_rsrc_t dst2 =
      a.dsplit > 0 ? make_rsrc(a.dst2 + (int64_t)ec.n * a.sd0_2, a.dst2_bytes) : dst1;
  const bool pos_contig = sd[4] == 1;
  const bool ch_contig = !pos_contig && sd[1] == 1;
  const int sd1 = (int)sd[1], sd2 = (int)sd[2], sd3 = (int)sd[3], sd4 = (int)sd[4];
  auto gate = [](uint32_t off, bool on) { return (int)(off | ((uint32_t)!on << 31)); };
  // Uniform: the whole box lies inside the volume.  A group of 8 columns of
  // such a box that lies inside the real columns is stored without gates
  // (the common case); only edge boxes and the last column group pay for the
  // per-store tests.
  const bool box_in = r0d + TD <= a.Rd && r0h + TH * HR <= a.Rh && r0w + LW <= a.Rw;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = wv * MB + mb;
    const int td = r / TH, th = r % TH;
    const int rd = r0d + td;
    const int h = r0h + th * HR + li / LW, w = r0w + li % LW;  // this lane's position
    const bool pos_ok = rd < a.Rd && h < a.Rh && w < a.Rw;
    const uint32_t poff = 2u * (uint32_t)(rd * sd2 + h * sd3 + w * sd4);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int colbase = (ec.ct * NB + nb) * 32;
      if (colbase >= a.ncols) continue;
      const float4* bt = reinterpret_cast<const float4*>(btab + (colbase - bcol0)) + g;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (colbase + 8 * q >= a.ncols) break;   // uniform: the rest of the block is padding
        const bool second = a.dsplit > 0 && colbase + 8 * q >= a.dsplit;  // uniform
        const __amdgpu_buffer_rsrc_t dst = second ? dst2 : dst1;
        const int cbase = second ? a.dsplit : 0;
        const int c0 = colbase + 8 * q + 4 * g - cbase;  // channels c0 .. c0+3 of this lane (in dst)
        const float4 bv = bt[2 * q];
        const float v0 = acc[mb][nb][4 * q + 0] + bv.x, v1 = acc[mb][nb][4 * q + 1] + bv.y;
        const float v2 = acc[mb][nb][4 * q + 2] + bv.z, v3 = acc[mb][nb][4 * q + 3] + bv.w;
        const bool clean = box_in && colbase + 8 * q + 8 <= a.ncols;  // uniform
        if (pos_contig || !ch_contig) {
          const float vv[4] = {v0, v1, v2, v3};
          if (clean) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              __builtin_amdgcn_raw_buffer_store_b16(from_f32<T>(vv[rr]), dst,
                                                    (int)(poff + 2u * (uint32_t)((c0 + rr) * sd1)), 0, 0);
          } else {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) {
              const uint32_t off = poff + 2u * (uint32_t)((c0 + rr) * sd1);
              __builtin_amdgcn_raw_buffer_store_b16(from_f32<T>(vv[rr]), dst, gate(off, pos_ok && cbase + c0 + rr < a.ncols), 0, 0);
            }
          }
        } else {
          typedef __attribute__((ext_vector_type(2))) uint32_t u32x2_t;
          const uint32_t off = poff + 2u * (uint32_t)c0;
          if (cbase + c0 + 4 <= a.ncols) {
            const u32x2_t v = {pack2(from_f32<T>(v0), from_f32<T>(v1)), pack2(from_f32<T>(v2), from_f32<T>(v3))};
            __builtin_amdgcn_raw_buffer_store_b64(v, dst, clean ? (int)off : gate(off, pos_ok), 0, 0);
          } else {
            const float vv[4] = {v0, v1, v2, v3};
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
              __builtin_amdgcn_raw_buffer_store_b16(from_f32<T>(vv[rr]), dst, gate(off + 2u * rr, pos_ok && cbase + c0 + rr < a.ncols),
                                                    0, 0);
          }
        }
      }
    }
  }
}

// SRC: 1 = channel-contiguous source (16-byte slot loads), 0 = any strides
// (eight 2-byte loads per slot), 3 = w-contiguous source with channel planes
// outermost in a sample (NCDHW, W % 8 == 0, RowArgs::chan_outer):
// a thread loads 8 positions of each of the chunk's 8 channels (eight 16-byte
// loads of one tile row segment) and transposes them in registers into 8 slots.
// WF: every chunk's weights resident in LDS (single column tile), else two
// per-stage buffers.
template <typename T, int NB, int MB, int SRC, int WF, int LW>
__global__ __launch_bounds__(512) void tap_kernel(const RowArgs a) {
  extern __shared__ uint4 smem4[];
  using G = TapGeom<MB, LW>;
  constexpr int NSTEP = G::NSTEP;
  constexpr int HW = G::HW;
  constexpr int HH = G::HH;
  constexpr int HR = G::HR;
  constexpr int HPOS = G::HPOS;
  constexpr int HPAD = G::HPAD;
  constexpr int MAXK = G::MAXK;
  constexpr int WFRAG = NSTEP * NB * 64;             // uint4 per chunk of weights
  constexpr int WIT = WF ? 1 : (WFRAG + 511) / 512;  // weight uint4 per thread per stage
  // Activation register sets = stages of load-latency cover (a stage is at
  // least 14 * MB * NB MFMAs per wave); one where two do not fit.
  constexpr int DIST = (SRC != 3 ? MB * NB <= 4 : (NB == 1 || MB * NB <= 2)) ? 2 : 1;
  // SRC 3: items (tile row, 8-position segment), segment j covering w in
  // [r0w - 8 + 8j, r0w + 8j); item i goes to thread i (packed into the fewest
  // waves: a wave's staging instructions cost the same for any number of
  // active lanes), segments varying fastest so a load instruction reads whole
  // row runs (coalesced) rather than 16 bytes of many rows.
  constexpr int NSEG = LW / 8 + 2;
  constexpr int NITEM = G::HD * HH * NSEG;
  static_assert(SRC != 3 || NITEM <= 512, "one staging item per thread");
  constexpr int NREG = SRC == 3 ? 8 : MAXK;          // uint4 registers per set
  constexpr int PD = MB * NB <= 4 ? 3 : 1;           // fragment read-ahead (steps)
  constexpr int HOOK = 1;                            // step after which the next stage is staged

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, known wave-uniform
  const int g = lane >> 5;
  const int li = lane & 31;
  uint4* act = smem4;              // [2][HPAD]
  uint4* wts = smem4 + 2 * HPAD;   // WF: [nchunks][WFRAG], else [2][WFRAG]
  const int wslots = WF ? a.nchunks * WFRAG : 2 * WFRAG;
  float* btab = reinterpret_cast<float*>(wts + wslots);  // bias per packed column (16-byte aligned)
  const int nbcol = a.nbt_pad * 32;
  // One 16-byte trash slot per thread past the bias table, as a slot index of `act`.
  const uint32_t tslot = (uint32_t)((reinterpret_cast<uint4*>(btab + nbcol) + tid) - act);

  // Job assignment.  Workgroups are dealt to the 8 XCDs round-robin; each XCD
  // owns a contiguous eighth of the jobs, and inside it its workgroups take
  // jobs round-robin (job = first + i + k * nx).  The workgroups running at
  // the same time then work on neighbouring boxes, whose shared halo rows meet
  // in the XCD's L2 instead of being fetched once per box.
  const int nwg = gridDim.x;
  const bool byxcd = (nwg & 7) == 0;
  const int xcd = byxcd ? (int)(blockIdx.x & 7) : 0;
  const int nx = byxcd ? nwg >> 3 : nwg;
  const int wi = byxcd ? (int)(blockIdx.x >> 3) : (int)blockIdx.x;
  const int jx0 = (int)(((int64_t)xcd * a.njobs) / (byxcd ? 8 : 1));
  const int jx1 = (int)(((int64_t)(xcd + 1) * a.njobs) / (byxcd ? 8 : 1));
  const int j0 = jx0 + wi;
  if (j0 >= jx1) return;
  const int myjobs = (jx1 - j0 + nx - 1) / nx;

  for (int c = tid; c < nbcol; c += 512) btab[c] = (a.bias && c < a.ncols) ? to_f32<T>(a.bias[c]) : 0.f;

  // Lane bases of the A reads: line mb's slot of this lane plus, for the
  // g = 1 half, each of the four tap-pair deltas.
  int lbase[MB][4];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = wv * MB + mb;
    const int td = r / G::TH, th = r % G::TH;
    const int rb = LW == 32 ? (td * HH + th) * HW + li : (td * HH + th * HR + (li >> 4)) * HW + (li & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) lbase[mb][j] = rb + g * G::DELTAS[j];
  }

  // Staging slot k of this thread = tile position 512 k + tid, coded (hd, hh, hw).
  int irel[MAXK];
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int hp = k * 512 + tid;
    const int t = hp / HW, hw = hp % HW;
    const int hd = t / HH, hh = t % HH;
    irel[k] = hp < HPOS ? (hd | (hh << 8) | (hw << 16)) : -1;
  }
  const int ss1 = (int)a.ss[1], ss2 = (int)a.ss[2], ss3 = (int)a.ss[3], ss4 = (int)a.ss[4];
  // SRC 3: this thread's item (row, segment) coded (hd | hh << 8 | j << 16),
  // its first slot's w index in the tile (may be negative), and the mask of
  // its 8 positions that fall inside the tile row.
  int item = -1, seg_hw = 0, seg_mask = 0;
  if (SRC == 3 && tid < NITEM) {
    const int row = tid / NSEG, j = tid % NSEG;
    item = (row / HH) | ((row % HH) << 8) | (j << 16);
    seg_hw = 8 * j - 8 + a.pw;
#pragma unroll
    for (int p = 0; p < 8; ++p) seg_mask |= ((unsigned)(seg_hw + p) < (unsigned)HW) ? (1 << p) : 0;
    seg_hw += row * HW;
  }

  // Per-job byte offsets of this thread's slots (kOob outside the volume).
  uint32_t soff[MAXK];  // unsigned: an out-of-volume offset plus a channel offset stays out of range
  int cached_key = -1;
  auto job_offsets = [&](const TapCursor& c) __attribute__((always_inline)) {
    if (SRC != 3) {  // SRC 3 recomputes (one item): no branch ahead of the loads
      const int key = ((c.n * a.nbd + c.bd) * a.nbh + c.bh) * a.nbw + c.bw;
      if (key == cached_key) return;
      cached_key = key;
    }
    const int s0d = c.bd * G::TD - a.pd, s0h = c.bh * (G::TH * HR) - a.ph, s0w = c.bw * LW - a.pw;
    if (SRC == 3) {
      const int gd = s0d + (item & 255), gh = s0h + ((item >> 8) & 255), gw = c.bw * LW - 8 + 8 * (item >> 16);
      const bool ok = (item >= 0) & ((unsigned)gd < (unsigned)a.Sd) & ((unsigned)gh < (unsigned)a.Sh) &
                      ((unsigned)gw < (unsigned)a.Sw);
      soff[0] = ok ? 2 * (gd * ss2 + gh * ss3 + gw) : kOob;
      return;
    }
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      const int r = irel[k];
      const int gd = s0d + (r & 255), gh = s0h + ((r >> 8) & 255), gw = s0w + ((r >> 16) & 255);
      const bool ok = (r >= 0) & ((unsigned)gd < (unsigned)a.Sd) & ((unsigned)gh < (unsigned)a.Sh) &
                      ((unsigned)gw < (unsigned)a.Sw);
      soff[k] = ok ? 2 * (gd * ss2 + gh * ss3 + gw * ss4) : kOob;
    }
  };

  uint4 pfa[DIST][NREG];
  u32x4_t pfw[WIT];
  const uint4* wsrc = reinterpret_cast<const uint4*>(a.wpk);

  // Activation loads of stage `cur` into register set `slot`.  An
  // out-of-volume slot's offset stays past num_records after the channel
  // offset is added (every in-sample offset is below 1 GiB).  The loads are
  // issued whether or not the stage exists (`live`): a stage past the end
  // reads with every offset out of range (zeros, no memory access) from
  // sample 0.  Unconditional loads keep the compiler's load counting exact,
  // so a commit waits only for its own stage's loads, not for every load in
  // flight.
  auto issue_act = [&](const TapCursor& cur, int slot, bool live) __attribute__((always_inline)) {
    job_offsets(cur);
    const int c0 = live ? cur.chunk * 8 : 0;
    const uint32_t coff = live ? 2u * c0 * ss1 : 0u;  // uniform
    // Disabled loads get bit 31 set in their offset: past any num_records
    // (every valid offset is below 1 GiB), by arithmetic rather than a select,
    // which the compiler would turn into branches around duplicated loads.
    auto gate = [&](uint32_t off, bool on) { return (int)(off | ((uint32_t)!on << 31)); };
    if constexpr (SRC == 3) {
      // The host takes this mode only with channel planes outermost in a
      // sample and the buffer range ending at channel Cs, so loads of channels
      // past Cs fall out of range by themselves; a stage past the end gets an
      // empty range.  No per-load gating.  A chunk at or past csplit (a
      // multiple of 8) comes from the concatenation's second tensor.
      const bool second = a.csplit > 0 && c0 >= a.csplit;  // uniform
      const uint16_t* sbase = second ? a.src2 : a.src;
      const int64_t s0 = second ? a.ss0_2 : a.ss[0];
      const uint32_t srange = second ? a.src2_bytes : a.src_bytes;
      const uint32_t coff2 = second ? 2u * (uint32_t)(c0 - a.csplit) * ss1 : coff;
      const __amdgpu_buffer_rsrc_t src = make_rsrc(sbase + (live ? (int64_t)cur.n * s0 : 0), live ? srange : 0u);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        pfa[slot][e] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(src, (int)(soff[0] + coff2 + 2u * e * ss1), 0, 0));
    } else {
      const __amdgpu_buffer_rsrc_t src = make_rsrc(a.src + (live ? (int64_t)cur.n * a.ss[0] : 0), a.src_bytes);
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      if (SRC == 1) {
        pfa[slot][k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src, gate(soff[k] + coff, live), 0, 0));
      } else {
        uint32_t wd[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(
              src, gate(soff[k] + coff + 4u * q * ss1, live && c0 + 2 * q < a.Cs), 0, 0);
          const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(
              src, gate(soff[k] + coff + (4u * q + 2) * ss1, live && c0 + 2 * q + 1 < a.Cs), 0, 0);
          wd[q] = lo | (hi << 16);
        }
        pfa[slot][k] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
    }
    }
  };
  auto commit_act = [&](int slot, int buf) __attribute__((always_inline)) {
    if constexpr (SRC == 3) {
      // 8 channels x 8 positions -> 8 slots of 8 channels (position p of
      // channel e is half p of pfa[e]).  A position outside the tile row goes
      // to this thread's trash slot instead of behind a branch.
      if (item >= 0) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          const uint32_t sel = (p & 1) ? 0x07060302u : 0x05040100u;
          const int m = p >> 1;
          u32x4_t v;
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint4& lo = pfa[slot][2 * q];
            const uint4& hi = pfa[slot][2 * q + 1];
            const uint32_t l = m == 0 ? lo.x : (m == 1 ? lo.y : (m == 2 ? lo.z : lo.w));
            const uint32_t h = m == 0 ? hi.x : (m == 1 ? hi.y : (m == 2 ? hi.z : hi.w));
            v[q] = __builtin_amdgcn_perm(h, l, sel);
          }
          // Slot index by masking (no select of pointers, which the compiler
          // turns into a branch per position).
          const uint32_t keep = 0u - (uint32_t)((seg_mask >> p) & 1);
          const uint32_t slot_i = tslot ^ (((uint32_t)(buf * HPAD + seg_hw + p) ^ tslot) & keep);
          *reinterpret_cast<u32x4_t*>(act + slot_i) = v;
        }
      }
      return;
    }
#pragma unroll
    for (int k = 0; k < MAXK; ++k)
      if (k * 512 + tid < HPOS) act[buf * HPAD + k * 512 + tid] = pfa[slot][k];
  };
  auto issue_w = [&](const TapCursor& cur) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WIT; ++i) {
      // uint4 index inside the chunk's fragments; the tail of the last
      // iteration re-reads the final fragment and is not committed.
      const int e = i * 512 + tid < WFRAG ? i * 512 + tid : WFRAG - 1;
      const int f = e >> 6, l = e & 63;
      const int s = f / NB, nb = f - (f / NB) * NB;
      pfw[i] = *reinterpret_cast<const u32x4_t*>(
          wsrc + (((size_t)cur.chunk * NSTEP + s) * a.nbt_pad + cur.ct * NB + nb) * 64 + l);
    }
  };
  auto commit_w = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < WIT; ++i) {
      const int e = i * 512 + tid;
      if (e < WFRAG) *reinterpret_cast<u32x4_t*>(wts + buf * WFRAG + e) = pfw[i];
    }
  };

  f32x16_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0.f;

  constexpr int PW = MB * NB * 16 * 64;  // partial floats per wave
  auto store_partial = [&](const TapCursor& c) __attribute__((always_inline)) {
    float* mine = a.part + (((size_t)tap_tile(a, c) * a.nsplit + c.split) * 8 + wv) * PW + lane;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) __builtin_nontemporal_store(acc[mb][nb][e], mine + ((mb * NB + nb) * 16 + e) * 64);
  };

  if (WF) {  // every chunk's weights, once (one column tile: fragments are contiguous)
    const u32x4_t* wsrc4 = reinterpret_cast<const u32x4_t*>(a.wpk);
    for (int e = tid; e < a.nchunks * WFRAG; e += 512) *reinterpret_cast<u32x4_t*>(wts + e) = wsrc4[e];
  }

  // Prologue: stages 0 .. DIST-1 into register sets 0 .. DIST-1, stage 0
  // into buffer 0, stage DIST into set 0; weights of stage 0 into buffer 0,
  // stage 1 in flight.
  const int nstage = myjobs * a.cps;
  TapCursor cc = tap_cursor_at(a, j0);
  const TapCursor stride = tap_cursor_at(a, nx);  // digits of the job stride
  TapCursor ca = cc, cw = cc;
  issue_act(ca, 0, true);
  tap_advance(a, ca, stride);
  if (DIST == 2) {
    issue_act(ca, DIST - 1, nstage > 1);
    tap_advance(a, ca, stride);
  }
  if (!WF) {
    issue_w(cw);
    tap_advance(a, cw, stride);
  }
  commit_act(0, 0);
  issue_act(ca, 0, nstage > DIST);
  tap_advance(a, ca, stride);
  if (!WF) {
    commit_w(0);
    issue_w(cw);
    tap_advance(a, cw, stride);
  }

  // Stage t (BUF = t % 2): data in buffer BUF; the activations of stage t+1
  // sit in register set SN = (t+1) % DIST and are committed during this
  // stage, after which that set loads stage t+1+DIST.
  auto run_stage = [&](int t, auto buf_c) __attribute__((always_inline)) {
    constexpr int BUF = decltype(buf_c)::value;
    constexpr int SN = DIST == 2 ? 1 - BUF : 0;
    lds_barrier();
    const uint4* wc = WF ? wts + cc.chunk * WFRAG : wts + BUF * WFRAG;
    uint4 bfr[PD + 1][NB], afr[PD + 1][MB];
    auto read_step = [&](auto st_c, int slot) __attribute__((always_inline)) {
      constexpr int ST = decltype(st_c)::value;
      constexpr int OFF = BUF * HPAD + G::tap_off(2 * ST);
      constexpr int DI = G::delta_idx(ST);
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bfr[slot][nb] = wc[(ST * NB + nb) * 64 + lane];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) afr[slot][mb] = act[lbase[mb][DI] + OFF];
    };
    auto step = [&](auto s_c) __attribute__((always_inline)) {
      constexpr int S = decltype(s_c)::value;
      constexpr int CUR = S % (PD + 1);
      if constexpr (S + PD < NSTEP) read_step(std::integral_constant<int, S + PD>{}, (S + PD) % (PD + 1));
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma32<T>(bfr[CUR][nb], afr[CUR][mb], acc[mb][nb]);  // C^T
      if constexpr (S == HOOK) {
        __builtin_amdgcn_sched_barrier(0);
        if (t + 1 < nstage) commit_act(SN, 1 - BUF);
        issue_act(ca, SN, t + 1 + DIST < nstage);
        tap_advance(a, ca, stride);
        if (!WF) {
          // Weight loads stay in range for any cursor (chunk < nchunks,
          // column tile < n_ctiles), so they too are issued unconditionally.
          if (t + 1 < nstage) commit_w(1 - BUF);
          issue_w(cw);
          tap_advance(a, cw, stride);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    read_step(std::integral_constant<int, 0>{}, 0);
    if constexpr (PD >= 2) read_step(std::integral_constant<int, 1>{}, 1);
    if constexpr (PD >= 3) read_step(std::integral_constant<int, 2>{}, 2);
    static_for(std::make_integer_sequence<int, NSTEP>{}, step);
    if (cc.chunk == (cc.split + 1) * a.cps - 1) {
      if (a.nsplit > 1) store_partial(cc);
      else tap_epilogue<T, NB, MB, LW>(a, acc, wv, lane, cc, btab, 0);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0.f;
    }
    tap_advance(a, cc, stride);
  };
  for (int t = 0; t < nstage; t += 2) {
    run_stage(t, std::integral_constant<int, 0>{});
    if (t + 1 < nstage) run_stage(t + 1, std::integral_constant<int, 1>{});
  }
}

// Split-K epilogue: one wave per (output tile, wave of the main pass); adds
// the tile's split partial sums in split order (the same order for every tile
// and run) and runs the epilogue.
template <typename T, int NB, int MB, int LW>
__global__ __launch_bounds__(64) void tap_split_epilogue(const RowArgs a) {
  __shared__ __attribute__((aligned(16))) float btab[NB * 32];
  constexpr int PW = MB * NB * 16 * 64;
  const int lane = threadIdx.x;
  const int tile = blockIdx.x >> 3, wv = blockIdx.x & 7;
  const int ct = tile % a.n_ctiles;
  for (int c = lane; c < NB * 32; c += 64) {
    const int col = ct * NB * 32 + c;
    btab[c] = (a.bias && col < a.ncols) ? to_f32<T>(a.bias[col]) : 0.f;
  }
  f32x16_t acc[MB][NB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0.f;
  const float* pt = a.part + ((size_t)tile * a.nsplit * 8 + wv) * PW + lane;
  for (int sp = 0; sp < a.nsplit; ++sp) {
    const float* ps = pt + (size_t)sp * 8 * PW;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[mb][nb][e] += __builtin_nontemporal_load(ps + ((mb * NB + nb) * 16 + e) * 64);
  }
  __syncthreads();
  const TapCursor ec = tap_cursor_at(a, tile * a.nsplit);
  tap_epilogue<T, NB, MB, LW>(a, acc, wv, lane, ec, btab, ct * NB * 32);
}

template <typename T, int NB, int MB, int SRC, int WF, int LW>
static void launch_tap_inst(const RowArgs& a, int cus, size_t lds, hipStream_t stream) {
  if (a.phase == 1) {
    hipLaunchKernelGGL((tap_split_epilogue<T, NB, MB, LW>), dim3(a.ntiles * 8), dim3(64), 0, stream, a);
    return;
  }
  auto kern = tap_kernel<T, NB, MB, SRC, WF, LW>;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 512, lds) != hipSuccess || occ < 1) occ = 1;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = (int)(a.njobs < cap ? a.njobs : cap);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(512), lds, stream, a);
}

}  // namespace r3c
