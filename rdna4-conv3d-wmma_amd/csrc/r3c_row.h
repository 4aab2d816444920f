// r3c_row.h -- implicit-GEMM "row" kernel for gfx950 on v_mfma_f32_32x32x16 (template body).
//
//   C[row position][column] = sum_k A[row][k] * B[k][column]
//
// A workgroup (4 waves) owns a box of TD x TH x 32 positions of the row grid
// and NB column blocks of 32.  Wave w owns MB row blocks; a row block is one
// 32-wide line along w, so MFMA row i is position w0 + i.
//
// Operand layouts (measured on gfx950, lane l, g = l / 32, i = l % 32):
//   A (32 x 16): lane holds A[i][8g .. 8g+7]
//   B (16 x 32): lane holds B[8g .. 8g+7][i]
//   C (32 x 32): acc[4q + r] = C[8q + 4g + r][i]
//
// K walks (tap, 8-channel group); one MFMA consumes two groups (g = 0, 1).
// Per source-channel chunk of CK channels, the box plus its halo is staged into
// LDS as [channel group][position] 16-byte slots (8 channels of one position).
// An A fragment is then one ds_read_b128 per lane at slot (cg, row + tap): the
// 32 lanes of a half-wave read 32 consecutive slots, so lanes l and l+16 sit
// 256 B apart and each 16-lane group covers 16 distinct slots -- the pattern
// gfx950's LDS serves at full rate.  ConvTranspose dX stores even and odd w
// of the 2x-wide dY box in separate halves of each row so its stride-2 taps
// read consecutive slots as well.  B fragments are 16-byte loads of the weight
// pre-packed in lane order.
//
// CL 2 (single-tap modes, w-contiguous source, NCDHW): the chunk's 32 channels
// are staged channel-major, [channel][CGS halves], each thread moving 8
// consecutive positions of one channel with one 16-byte load; an A fragment is
// then two ds_read_b64_tr_b16 (4 channels at 16 consecutive positions per
// 16-lane group each).  CGS = 32 (mod 128) keeps the 16-lane groups of a read
// on distinct banks.
//
// Loads go through a buffer resource with 32-bit offsets: out-of-range
// positions (the zero padding) use an offset past num_records, which the
// hardware returns as zero, so there are no bounds branches.
//
// Index math follows the reference kernels: K3 fwd (src/rdna4_conv3d/
// conv3d_wmma.py:372-444), K1 fwd (328-369), ConvTranspose fwd scatter
// (793-860) and ConvTranspose dX gather (863-931).
#pragma once
#include <type_traits>

#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

// n / d for n < 4096 and 1 <= d < 256, via a 20-bit reciprocal (exact in range).
struct FastDiv20 {
  uint32_t m;
  __device__ __forceinline__ explicit FastDiv20(uint32_t d) : m(((1u << 20) + d - 1) / d) {}
  __device__ __forceinline__ uint32_t div(uint32_t n) const { return (n * m) >> 20; }
};

constexpr int kOob = 0x7fffff00;  // byte offset past any num_records: the load returns 0

// Workgroup barrier for LDS hand-off only: waits for this wave's LDS accesses
// (lgkmcnt 0; vmcnt and expcnt left at their maxima) and not for its global
// loads, so register prefetches stay in flight across it.  __syncthreads()
// would also drain vmcnt.
__device__ __forceinline__ void lds_barrier() {
  __asm__ __volatile__("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
  __asm__ __volatile__("" ::: "memory");
}

template <int MODE>
struct RowGeom {
  static constexpr int TAPS = MODE == MODE_K3 ? 27 : (MODE == MODE_T2DX ? 8 : 1);
  static constexpr int HW = MODE == MODE_K3 ? 34 : (MODE == MODE_T2DX ? 64 : 32);
  // Row blocks (32 positions) per wave, and the largest LDS tile any allowed box
  // needs (K3: 2x4 or 4x2 boxes plus halo; T2DX: boxes of 4 rows, 2x in dY).
  // ConvTranspose fwd has 8 Cout columns per source channel: one row block per
  // wave leaves the registers for six column blocks, so a 24-channel output
  // (192 columns) is one column tile and each source box is staged once.
  static constexpr int MB = (MODE == MODE_T2DX || MODE == MODE_T2FWD) ? 1 : 2;
  static constexpr int MAXHPOS = MODE == MODE_K3 ? 4 * 6 * 34 : (MODE == MODE_T2DX ? 16 * 64 : 8 * 32);
  // A chunk is G8 8-channel groups: one group per tap when there are taps; four
  // (two MFMA steps) for the memory-bound single-tap modes, so each pipeline
  // stage moves more bytes per barrier.
  static constexpr int G8 = TAPS == 1 ? 4 : 1;
  static constexpr int NSTEP = (TAPS * G8 + 1) / 2;
  static constexpr int MAXK = (MAXHPOS + 255) / 256;  // staging slots per thread per group
};

typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// The same for a base and range that are equal in every lane but computed on
// the vector unit (divisions, 64-bit products): readfirstlane moves them to
// scalar registers.  A resource left in vector registers makes the compiler
// wrap every buffer load in a readfirstlane / compare / exec-mask loop.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc_u(const void* base, uint32_t bytes) {
  const uint64_t v = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}

// Half k of element q of a uint4 (q in 0..7), without taking its address.
__device__ __forceinline__ uint16_t u4_elem(const uint4& v, int q) {
  const uint32_t w = q < 2 ? v.x : (q < 4 ? v.y : (q < 6 ? v.z : v.w));
  return (uint16_t)((q & 1) ? (w >> 16) : (w & 0xffff));
}

// LDS: act[2][G8][HPAD] 16-byte slots (double-buffered tile, HPAD = HPOS rounded
// up to 16), the weight fragments (all of K when WF, else two chunk buffers of
// NSTEP x NB fragments), the per-wave epilogue scratch (4 x 2 KB) and the bias
// table (fp32, one per packed column).
//
// Pipeline: one stage = one 8-channel (16 for single-tap modes) chunk of one
// job.  Stage t+DIST's activations (DIST = 2 where the registers allow, else
// 1) and, without WF, stage t+1's weights are loaded into registers while
// stage t computes from LDS, and written to LDS at the start of their stage;
// one barrier per stage with double buffers.  The barrier waits for LDS
// traffic only, so the register prefetches stay in flight across it.
//
// Epilogue: a wave converts each 32 x 32 C tile (plus bias) to 16-bit and
// writes it to its scratch as [column][position] with 8-byte writes, then
// reads it back in store order -- 8 consecutive positions of one channel per
// lane when positions are contiguous in memory (NCDHW), or, through
// ds_read_tr16_b64, 8 consecutive channels of one position per lane when
// channels are contiguous (NDHWC) -- so every global store is 16 bytes.
template <typename T, int MODE, int NB, int CL, int WF>
// A 27-tap chunk with three column blocks of per-stage weights needs more than
// half the register file; those instantiations run one wave per SIMD.
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((MODE == MODE_K3 && NB == 3 && !WF) ? 1 : 2, 8))) void row_kernel(
    const RowArgs a) {
  extern __shared__ uint4 smem4[];
  constexpr int TAPS = RowGeom<MODE>::TAPS;
  constexpr int HW = RowGeom<MODE>::HW;
  constexpr int MB = RowGeom<MODE>::MB;
  constexpr int NSTEP = RowGeom<MODE>::NSTEP;
  constexpr int MAXK = RowGeom<MODE>::MAXK;
  constexpr int G8 = RowGeom<MODE>::G8;
  constexpr int WFRAG = NSTEP * NB * 64;              // uint4 per chunk of weights
  constexpr int WIT = WF ? 1 : (WFRAG + 255) / 256;   // weight uint4 per thread per chunk

  constexpr bool CM = CL == 2;  // channel-major staging
  static_assert(!CM || (TAPS == 1 && G8 == 4 && MAXK == 1), "channel-major staging: single-tap modes");
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const int g = lane >> 5;
  const int li = lane & 31;

  const int HH = a.HH;
  const int HPOS = a.HD * HH * HW;
  const int HPAD = a.CGS;  // HPOS rounded up to a multiple of 16
  const int ABUF = G8 * HPAD;  // slots per activation buffer
  const int nbuf = a.nbuf;     // 2: double-buffered stages; 1: single buffers, two barriers
  uint4* act = smem4;
  uint4* wts = smem4 + nbuf * ABUF;
  const int wslots = WF ? a.nchunks * WFRAG : nbuf * WFRAG;
  uint16_t* scr = reinterpret_cast<uint16_t*>(wts + wslots) + wv * 1024;
  float* btab = reinterpret_cast<float*>(wts + wslots + 4 * 128);
  const int nbcol = a.nbt_pad * 32;

  // Contiguous job range of this workgroup; a job is (box, column tile, split).
  // Workgroups are dealt to the 8 XCDs round-robin (blockIdx % 8); renumbering
  // them so each XCD owns one contiguous eighth of the jobs keeps boxes that
  // share tap halos (neighbours in d and h) on the same L2.
  const int nwg = gridDim.x;
  const int wg = (a.phase == 0 && (nwg & 7) == 0) ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int j0 = (int)(((int64_t)wg * a.njobs) / nwg);
  const int j1 = (int)(((int64_t)(wg + 1) * a.njobs) / nwg);
  if (j0 >= j1) return;

  // Slot offset of k group 2s + g (tap, channel group) for each step s of this
  // lane's half; held in registers so the fully unrolled K loop issues every
  // LDS read without waiting on a table.
  int kof[NSTEP];
#pragma unroll
  for (int st = 0; st < NSTEP; ++st) {
    const int kg = 2 * st + g;
    int off = 0;  // K padding: the row's own slot, times zero weights
    if (kg < TAPS * G8) {
      const int tap = kg / G8, cg = kg - (kg / G8) * G8;
      if (MODE == MODE_K3) off = ((tap / 9) * HH + (tap / 3) % 3) * HW + tap % 3;
      else if (MODE == MODE_T2DX) off = ((tap >> 2) * HH + ((tap >> 1) & 1)) * HW + (tap & 1) * 32;
      off += cg * HPAD;
    }
    kof[st] = off;
  }
  for (int c = tid; c < nbcol; c += 256) {
    float bv = 0.f;
    if (a.bias && c < a.ncols)
      bv = to_f32<T>(a.bias[MODE == MODE_T2FWD ? (a.t2kw ? (c >> 1) : c) % a.cout_t2 : c]);
    btab[c] = bv;
  }

  int rowbase[MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int r = wv * MB + mb;
    const int td = r / a.TH, th = r - (r / a.TH) * a.TH;
    if (MODE == MODE_T2DX) rowbase[mb] = ((2 * td) * HH + 2 * th) * HW + li;
    else rowbase[mb] = (td * HH + th) * HW + li;
  }

  // Staging slot k of this thread is tile position 256 k + tid.
  int irel[MAXK];
  {
    const FastDiv20 divHH((uint32_t)HH);
#pragma unroll
    for (int k = 0; k < MAXK; ++k) {
      const int hp = k * 256 + tid;
      const int t = hp / HW;
      int hw = hp - t * HW;
      if (MODE == MODE_T2DX) hw = (hw & 31) * 2 + (hw >> 5);  // de-interleaved row: slot -> w
      const int hd = (int)divHH.div((uint32_t)t);
      const int hh = t - hd * HH;
      irel[k] = hp < HPOS ? (hd | (hh << 8) | (hw << 16)) : -1;
    }
  }
  const int ss1 = (int)a.ss[1], ss2 = (int)a.ss[2], ss3 = (int)a.ss[3], ss4 = (int)a.ss[4];
  // Byte offset of each staging slot relative to the tile origin, so a stage
  // forms each address with one add to a uniform base.
  int roff[MAXK];
#pragma unroll
  for (int k = 0; k < MAXK; ++k) {
    const int r = irel[k] < 0 ? 0 : irel[k];
    roff[k] = 2 * ((r & 255) * ss2 + ((r >> 8) & 255) * ss3 + ((r >> 16) & 255) * ss4);
  }
  // CM: staging item k*256 + tid = (channel ci, 8-position chunk) of the tile,
  // coded (hd, hh, hw, ci) 8 bits each; byte offset relative to the tile origin.
  int cmi[CM ? 4 : 1], cmoff[CM ? 4 : 1];
  if (CM) {
    const int nchk = HPOS >> 3;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int it = k * 256 + tid;
      const int ci = it / nchk, pos = (it - ci * nchk) * 8;
      const int t = pos / HW, hw = pos - t * HW;
      const int hd = t / HH, hh = t - hd * HH;
      cmi[k] = ci < 32 ? (hd | (hh << 8) | (hw << 16) | (ci << 24)) : -1;
      cmoff[k] = ci < 32 ? 2 * (ci * ss1 + hd * ss2 + hh * ss3 + hw) : 0;
    }
  }
  // CM: this lane's A-fragment half offset for row block mb at step 0
  // (channel 8g + (lane & 15) / 4, position line start + 16 ((lane >> 4) & 1) + 4 (lane & 3)).
  int cmrow[CM ? MB : 1];
  if (CM) {
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const int r = wv * MB + mb;
      const int td = r / a.TH, th = r - (r / a.TH) * a.TH;
      cmrow[mb] = (8 * g + ((lane & 15) >> 2)) * HPAD + (td * HH + th) * HW + 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    }
  }
  // Activation prefetch depth in stages: two where the registers allow it.
  constexpr int DIST = (NB == 1 || (NB == 2 && WF) || (MODE == MODE_K3 && NB == 3 && !WF)) ? 2 : 1;
  uint4 pfa[DIST][G8 * MAXK];
  u32x4_t pfw[WIT];

  // A stage cursor: (chunk, column tile, box w, h, d, sample), advanced with
  // carries so the per-stage index math is a few scalar adds (the divisions
  // happen once per workgroup).
  struct Cursor {
    int chunk, split, ct, bw, bh, bd, n;
  };
  auto cursor_at = [&](int job) {
    Cursor c;
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
  };
  auto advance = [&](Cursor& c) {
    if (++c.chunk < (c.split + 1) * a.cps) return;
    if (++c.split < a.nsplit) return;  // chunk is already split * cps
    c.split = 0;
    c.chunk = 0;
    if (++c.ct < a.n_ctiles) return;
    c.ct = 0;
    if (++c.bw < a.nbw) return;
    c.bw = 0;
    if (++c.bh < a.nbh) return;
    c.bh = 0;
    if (++c.bd < a.nbd) return;
    c.bd = 0;
    ++c.n;
  };
  const uint4* wsrc = reinterpret_cast<const uint4*>(a.wpk);
  // Issue the activation loads of stage `cur` into register slot `slot`.
  auto issue_act = [&](const Cursor& cur, int slot) {
    const int n = cur.n, bd = cur.bd, bh = cur.bh, bw = cur.bw, chunk = cur.chunk;
    int s0d, s0h, s0w;
    if (MODE == MODE_K3 || MODE == MODE_K1) {
      s0d = bd * a.TD - a.pd;
      s0h = bh * a.TH - a.ph;
      s0w = bw * 32 - a.pw;
    } else if (MODE == MODE_T2DX) {
      s0d = 2 * bd * a.TD;
      s0h = 2 * bh * a.TH;
      s0w = 64 * bw;
    } else {
      s0d = bd * a.TD;
      s0h = bh * a.TH;
      s0w = bw * 32;
    }
    const __amdgpu_buffer_rsrc_t src = make_rsrc(a.src + (int64_t)n * a.ss[0], a.src_bytes);
    if (CM) {  // 8 positions of one channel per item (the host keeps Sw % 8 == 0 and s0w >= 0)
      const int c0 = chunk * 32;
      const int base = 2 * (s0d * ss2 + s0h * ss3 + s0w + c0 * ss1);  // uniform
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = cmi[k];
        const int gd = s0d + (r & 255), gh = s0h + ((r >> 8) & 255), gw = s0w + ((r >> 16) & 255);
        const bool ok = r >= 0 && (unsigned)gd < (unsigned)a.Sd && (unsigned)gh < (unsigned)a.Sh && gw < a.Sw &&
                        c0 + (r >> 24) < a.Cs;
        pfa[slot][k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src, ok ? base + cmoff[k] : kOob, 0, 0));
      }
      return;
    }
#pragma unroll
    for (int cg = 0; cg < G8; ++cg) {
      const int c0 = chunk * 8 * G8 + cg * 8;
      const int base = 2 * (s0d * ss2 + s0h * ss3 + s0w * ss4 + c0 * ss1);  // uniform
#pragma unroll
      for (int k = 0; k < MAXK; ++k) {
        const int r = irel[k];
        const int gd = s0d + (r & 255), gh = s0h + ((r >> 8) & 255), gw = s0w + ((r >> 16) & 255);
        const bool ok = r >= 0 && (unsigned)gd < (unsigned)a.Sd && (unsigned)gh < (unsigned)a.Sh &&
                        (unsigned)gw < (unsigned)a.Sw && c0 < a.Cs;
        const int off = base + roff[k];
        if (CL) {
          pfa[slot][cg * MAXK + k] =
              __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src, ok ? off : kOob, 0, 0));
        } else {
          uint32_t wd[4];
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t lo = __builtin_amdgcn_raw_buffer_load_b16(
                src, (ok && c0 + 2 * q < a.Cs) ? off + 4 * q * ss1 : kOob, 0, 0);
            const uint32_t hi = __builtin_amdgcn_raw_buffer_load_b16(
                src, (ok && c0 + 2 * q + 1 < a.Cs) ? off + (4 * q + 2) * ss1 : kOob, 0, 0);
            wd[q] = lo | (hi << 16);
          }
          pfa[slot][cg * MAXK + k] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
        }
      }
    }
  };
  // Issue the weight loads of stage `cur` (per-stage weights only).
  auto issue_w = [&](const Cursor& cur) {
    {
      const int ct = cur.ct, chunk = cur.chunk;
#pragma unroll
      for (int i = 0; i < WIT; ++i) {
        // uint4 index inside the chunk's fragments; the tail of the last
        // iteration re-reads the final fragment and is not committed.
        const int e = i * 256 + tid < WFRAG ? i * 256 + tid : WFRAG - 1;
        const int f = e >> 6, l = e & 63;
        const int s = f / NB, nb = f - (f / NB) * NB;
        pfw[i] = *reinterpret_cast<const u32x4_t*>(wsrc + (((size_t)chunk * NSTEP + s) * a.nbt_pad + ct * NB + nb) * 64 + l);
      }
    }
  };
  auto commit_act = [&](int slot, int buf) {
    if (CM) {
      uint16_t* ah = reinterpret_cast<uint16_t*>(act + buf * ABUF);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int r = cmi[k];
        if (r >= 0) {
          const int pos = (((r & 255) * HH + ((r >> 8) & 255)) * HW) + ((r >> 16) & 255);
          *reinterpret_cast<u32x4_t*>(ah + (r >> 24) * HPAD + pos) = __builtin_bit_cast(u32x4_t, pfa[slot][k]);
        }
      }
      return;
    }
#pragma unroll
    for (int cg = 0; cg < G8; ++cg)
#pragma unroll
      for (int k = 0; k < MAXK; ++k)
        if (k * 256 + tid < HPOS) act[buf * ABUF + cg * HPAD + k * 256 + tid] = pfa[slot][cg * MAXK + k];
  };
  auto commit_w = [&](int buf) {
#pragma unroll
    for (int i = 0; i < WIT; ++i) {
      const int e = i * 256 + tid;
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

  // Epilogue of output tile `ec`: acc (+ bias) -> 16-bit -> per-wave scratch
  // -> 16-byte global stores in the destination's layout.
  auto epilogue = [&](const Cursor& ec) __attribute__((always_inline)) {
      // Epilogue: lane (g, i) holds rows 8q + 4g + r (w positions) of column i.
      const int n = ec.n, bd = ec.bd, bh = ec.bh, bw = ec.bw, ct = ec.ct;
      const int r0d = bd * a.TD, r0h = bh * a.TH, r0w = bw * 32;
      const int64_t* sd = a.sd;
      uint16_t* dstn = a.dst + (int64_t)n * sd[0];
      const bool pos_contig = sd[4] == 1;
      const bool ch_contig = !pos_contig && sd[1] == 1;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const int r = wv * MB + mb;
        const int td = r / a.TH, th = r - (r / a.TH) * a.TH;
        const int rd = r0d + td, rh = r0h + th;
        if (rd < a.Rd && rh < a.Rh) {
          // Uniform base of this output line at w = r0w; per-lane offsets are
          // 32-bit when the host found they fit (off32).
          uint16_t* lineb = dstn + (int64_t)rd * sd[2] + (int64_t)rh * sd[3] + (int64_t)r0w * sd[4];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const int colbase = (ct * NB + nb) * 32;
            if (colbase >= a.ncols) continue;
            {  // C tile (+ bias) -> scratch [column][position]
              const float bv = btab[colbase + li];
#pragma unroll
              for (int q = 0; q < 4; ++q) {
                uint2 v;
                v.x = pack2(from_f32<T>(acc[mb][nb][4 * q + 0] + bv), from_f32<T>(acc[mb][nb][4 * q + 1] + bv));
                v.y = pack2(from_f32<T>(acc[mb][nb][4 * q + 2] + bv), from_f32<T>(acc[mb][nb][4 * q + 3] + bv));
                *reinterpret_cast<uint2*>(scr + li * 32 + 8 * q + 4 * g) = v;
              }
            }
            // A wave's LDS operations execute in order, so only the compiler
            // must be kept from reordering the scratch writes and reads.
            __builtin_amdgcn_wave_barrier();
            if (MODE == MODE_T2FWD && pos_contig && a.t2kw) {
              // ConvTranspose into a w-contiguous output: columns 2j, 2j+1 are
              // kw = 0, 1 of one (kd, kh, co), so positions w of the pair
              // interleave into 64 consecutive outputs 2w + kw; a lane builds
              // 8 of them (4 positions x 2 kw) and stores 16 bytes.
#pragma unroll
              for (int rd2 = 0; rd2 < 2; ++rd2) {
                const int id = rd2 * 64 + lane;
                const int j = id >> 3, kq = id & 7;
                const int col = colbase + 2 * j;
                const int w0 = r0w + 4 * kq;
                const uint2 e0 = *reinterpret_cast<const uint2*>(scr + (2 * j) * 32 + 4 * kq);
                const uint2 e1 = *reinterpret_cast<const uint2*>(scr + (2 * j + 1) * 32 + 4 * kq);
                if (col < a.ncols && w0 < a.Rw) {
                  const int rest = col >> 1, kdkh = rest / a.cout_t2, co = rest - kdkh * a.cout_t2;
                  uint16_t* p = dstn + (int64_t)co * sd[1] + (int64_t)(2 * rd + (kdkh >> 1)) * sd[2] +
                                (int64_t)(2 * rh + (kdkh & 1)) * sd[3] + 2 * w0;
                  const uint4 v = make_uint4(__builtin_amdgcn_perm(e1.x, e0.x, 0x05040100u),
                                             __builtin_amdgcn_perm(e1.x, e0.x, 0x07060302u),
                                             __builtin_amdgcn_perm(e1.y, e0.y, 0x05040100u),
                                             __builtin_amdgcn_perm(e1.y, e0.y, 0x07060302u));
                  if (w0 + 4 <= a.Rw && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
                    *reinterpret_cast<uint4*>(p) = v;
                  } else {
                    for (int k = 0; k < 8 && w0 + (k >> 1) < a.Rw; ++k) p[k] = u4_elem(v, k);
                  }
                }
              }
            } else if (MODE != MODE_T2FWD && pos_contig) {
              // 8 consecutive positions of one channel per lane (NCDHW).
#pragma unroll
              for (int rd2 = 0; rd2 < 2; ++rd2) {
                const int id = rd2 * 64 + lane;
                const int c = id >> 2, pc = id & 3;
                const int col = colbase + c;
                const int rw = r0w + pc * 8;
                const uint4 v = *reinterpret_cast<const uint4*>(scr + c * 32 + pc * 8);
                if (col < a.ncols && rw < a.Rw) {
                  uint16_t* p = lineb + (a.off32 ? (int64_t)(col * (int)sd[1] + pc * 8) : (int64_t)col * sd[1] + pc * 8);
                  if (rw + 8 <= a.Rw && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
                    *reinterpret_cast<uint4*>(p) = v;
                  } else {
                    for (int k = 0; k < 8 && rw + k < a.Rw; ++k) p[k] = u4_elem(v, k);
                  }
                }
              }
            } else if (ch_contig && (MODE != MODE_T2FWD || a.cout_t2 % 8 == 0)) {
              // 8 consecutive channels of one position per lane (NDHWC).
              const int sl = lane & 15;
#pragma unroll
              for (int rd2 = 0; rd2 < 2; ++rd2) {
                const int task = rd2 * 4 + (lane >> 4);
                const int p0 = 16 * (task & 1), c0 = 8 * (task >> 1);
                const int a0 = (c0 + (sl >> 2)) * 32 + p0 + 4 * (sl & 3);
                const uint4 v = lds_tr_pair(scr, a0, a0 + 4 * 32);
                const int col = colbase + c0;
                const int rw = r0w + p0 + sl;
                if (col < a.ncols && rw < a.Rw) {
                  uint16_t* p;
                  int nvalid;
                  if (MODE == MODE_T2FWD) {
                    const int tap = col / a.cout_t2, co = col - tap * a.cout_t2;
                    const int kd = tap >> 2, kh = (tap >> 1) & 1, kw = tap & 1;
                    p = dstn + (int64_t)co + (int64_t)(2 * rd + kd) * sd[2] + (int64_t)(2 * rh + kh) * sd[3] +
                        (int64_t)(2 * rw + kw) * sd[4];
                    nvalid = 8;
                  } else {
                    p = lineb + (a.off32 ? (int64_t)(col + (p0 + sl) * (int)sd[4]) : col + (int64_t)(p0 + sl) * sd[4]);
                    nvalid = a.ncols - col < 8 ? a.ncols - col : 8;
                  }
                  if (nvalid == 8 && ((reinterpret_cast<uintptr_t>(p) & 15) == 0)) {
                    *reinterpret_cast<uint4*>(p) = v;
                  } else {
                    for (int k = 0; k < nvalid; ++k) p[k] = u4_elem(v, k);
                  }
                }
              }
            } else {
              // Any other strides: one element per lane from the scratch.
              for (int e = lane; e < 32 * 32; e += 64) {
                const int c = e >> 5, pp = e & 31;
                const int col = colbase + c;
                const int rw = r0w + pp;
                if (col >= a.ncols || rw >= a.Rw) continue;
                const uint16_t v = scr[c * 32 + pp];
                if (MODE == MODE_T2FWD) {
                  const int tap = col / a.cout_t2, co = col - tap * a.cout_t2;
                  const int kd = tap >> 2, kh = (tap >> 1) & 1, kw = tap & 1;
                  dstn[(int64_t)co * sd[1] + (int64_t)(2 * rd + kd) * sd[2] + (int64_t)(2 * rh + kh) * sd[3] +
                       (int64_t)(2 * rw + kw) * sd[4]] = v;
                } else {
                  dstn[(int64_t)col * sd[1] + (int64_t)rd * sd[2] + (int64_t)rh * sd[3] + (int64_t)rw * sd[4]] = v;
                }
              }
            }
            __builtin_amdgcn_wave_barrier();
          }
        }
      }
  };
  // Split K: the tile's partial sums of this split, in lane order
  // [tile][split][wave][MB*NB*16][64]; the epilogue phase adds the splits.
  constexpr int PW = MB * NB * 16 * 64;  // floats per wave
  auto tile_of = [&](const Cursor& c) {
    return (((c.n * a.nbd + c.bd) * a.nbh + c.bh) * a.nbw + c.bw) * a.n_ctiles + c.ct;
  };
  auto store_partial = [&](const Cursor& c) __attribute__((always_inline)) {
    float* mine = a.part + (((size_t)tile_of(c) * a.nsplit + c.split) * 4 + wv) * PW + lane;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int e = 0; e < 16; ++e) __builtin_nontemporal_store(acc[mb][nb][e], mine + ((mb * NB + nb) * 16 + e) * 64);
  };
  if (a.phase == 1) {
    // Epilogue phase: one workgroup per output tile, acc = ((0 + p_0) + p_1) + ...
    // in split order (the same order for every tile and every run).
    const Cursor ec = cursor_at(blockIdx.x * a.nsplit);
    const float* pt = a.part + ((size_t)blockIdx.x * a.nsplit * 4 + wv) * PW + lane;
    for (int sp = 0; sp < a.nsplit; ++sp) {
      const float* ps = pt + (size_t)sp * 4 * PW;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[mb][nb][e] += __builtin_nontemporal_load(ps + ((mb * NB + nb) * 16 + e) * 64);
    }
    __syncthreads();  // the bias table is complete
    epilogue(ec);
    return;
  }
  if (WF) {  // every chunk's weights, once (a single column tile: fragments are contiguous)
    const u32x4_t* wsrc4 = reinterpret_cast<const u32x4_t*>(a.wpk);
    for (int e = tid; e < a.nchunks * WFRAG; e += 256)
      *reinterpret_cast<u32x4_t*>(wts + e) = wsrc4[e];
  }
  // Stage t walks (job, chunk) from (j0, first chunk of j0's split).  Activations are loaded DIST
  // stages ahead, per-stage weights one stage ahead; `cc` is the stage being
  // computed, `ca` / `cw` the next activation / weight stage to issue.
  const int nstage = (j1 - j0) * a.cps;
  Cursor cc = cursor_at(j0);
  Cursor ca = cc, cw = cc;
  issue_act(ca, 0);
  advance(ca);
  if (!WF) {
    issue_w(cw);
    advance(cw);
  }
  if (DIST == 2 && nstage > 1) {
    issue_act(ca, DIST - 1);
    advance(ca);
  }
  // With two slots the loop is unrolled by two so each slot is a fixed set of
  // registers (no copies of loads still in flight).
  auto run_stage = [&](int t, auto slot_c) {
    constexpr int SL = decltype(slot_c)::value;
    const int chunk = cc.chunk;
    const int buf = nbuf == 2 ? (t & 1) : 0;
    commit_act(SL, buf);
    if (!WF) commit_w(buf);
    lds_barrier();
    if (t + DIST < nstage) {
      issue_act(ca, SL);  // in flight during the next DIST stages
      advance(ca);
    }
    if (!WF && t + 1 < nstage) {
      issue_w(cw);
      advance(cw);
    }

    const int ct = cc.ct;
    const uint4* wc = WF ? wts + chunk * WFRAG : wts + buf * WFRAG;
    const uint4* ab = act + buf * ABUF;
    // Fragments are read PD steps ahead of the MFMAs that use them (two steps
    // when a step has only MB MFMAs, fewer than an LDS read's latency covers).
    constexpr int PD = NB == 1 ? 2 : 1;
    uint4 bfr[PD + 1][NB], afr[PD + 1][MB];
    auto read_step = [&](int st, int slot) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) bfr[slot][nb] = wc[(st * NB + nb) * 64 + lane];
      if (CM) {
        const uint16_t* ah = reinterpret_cast<const uint16_t*>(ab);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
          afr[slot][mb] = lds_tr_pair(ah, cmrow[mb] + st * 16 * HPAD, cmrow[mb] + st * 16 * HPAD + 4 * HPAD);
      } else {
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) afr[slot][mb] = ab[rowbase[mb] + kof[st]];
      }
    };
#pragma unroll
    for (int st = 0; st < PD; ++st)
      if (st < NSTEP) read_step(st, st);
#pragma unroll
    for (int s = 0; s < NSTEP; ++s) {
      const int cur = s % (PD + 1);
      if (s + PD < NSTEP) read_step(s + PD, (s + PD) % (PD + 1));
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of this step's MFMAs
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc[mb][nb] = mfma32<T>(afr[cur][mb], bfr[cur][nb], acc[mb][nb]);
    }

    if (chunk == (cc.split + 1) * a.cps - 1) {
      if (a.nsplit > 1) store_partial(cc);
      else epilogue(cc);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[mb][nb][e] = 0.f;
    }
    if (nbuf == 1 && t + 1 < nstage) lds_barrier();  // the next commit overwrites the buffers
    advance(cc);
  };
  if (DIST == 2) {
    for (int t = 0; t < nstage; t += 2) {
      run_stage(t, std::integral_constant<int, 0>{});
      if (t + 1 < nstage) run_stage(t + 1, std::integral_constant<int, DIST - 1>{});
    }
  } else {
    for (int t = 0; t < nstage; ++t) run_stage(t, std::integral_constant<int, 0>{});
  }
}

template <typename T, int MODE, int NB, int CL, int WF>
static void launch_row_inst(const RowArgs& a, int cus, size_t lds, hipStream_t stream) {
  auto kern = row_kernel<T, MODE, NB, CL, WF>;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, 256, lds) != hipSuccess || occ < 1) occ = 1;
  const int64_t cap = (int64_t)cus * occ;
  const int grid = a.phase == 1 ? a.ntiles : (int)(a.njobs < cap ? a.njobs : cap);
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), lds, stream, a);
}

}  // namespace r3c
