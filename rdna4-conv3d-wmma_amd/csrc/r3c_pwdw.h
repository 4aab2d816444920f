// r3c_pwdw.h -- register-direct weight gradient of the single-tap passes for
// gfx950 on v_mfma_f32_32x32x16 (template body).
//
//   C[f][c] = sum over positions p of F[f][p] * G_c(p)
//
//   Conv3d k=1, no padding (MODE_K1): F = dY, column c = input channel,
//       G_c(p) = x[c][p], dW[co = f][ci = c]
//       (src/rdna4_conv3d/conv3d_wmma.py:544-634 with kvol 1)
//   ConvTranspose k2s2 (MODE_T2DW): F = x, column c = (gch, tap) with the tap
//       fastest, G_c(p) = dY[gch][2p + tap], dW[ci = f][co = gch][tap]
//       (conv3d_wmma.py:934-1012)
//
// With w-contiguous dense planes K (the positions) is contiguous in memory for
// both operands, and that is the MFMA's per-lane k run: lane (g, i) holds
// A[i][8g .. 8g+7] and B[8g .. 8g+7][i].  Each lane therefore loads its
// fragments straight from global memory: no LDS tile and no barrier in the K
// loop.  A K block is 16 NJ consecutive positions of one sample; lane half g
// owns positions [8 NJ g, 8 NJ g + 8 NJ) of it and MFMA j of the block takes
// positions 8 NJ g + 8 j .. + 7 (one fixed permutation of k, applied to both
// operands), so a lane reads 16 NJ contiguous bytes of an F row.  For
// ConvTranspose a G lane reads the 32 NJ contiguous bytes of dY row
// (2d + kd, 2h + kh) at w' = 2w .. 2w + 16 NJ - 1 and keeps the halves of
// parity kw (lanes kw = 0 and 1 of one (gch, kd, kh) read the same bytes).
//
// The bias gradient rides along as a virtual all-ones column (db_mode 1:
// db[f] = sum_p F[f][p]) or row (db_mode 2: db[c] = sum_p G_c(p), summed over
// the taps by the reduce).
//
// Workgroup: 8 waves, one tile group (TR row blocks x TC column blocks of 32)
// and one K split of interleaved K blocks, each wave with its next block's
// loads in flight while the current one is multiplied.  At the
// end the waves' tiles are added in LDS in wave order and written as the
// split's partial [split][f][tap][gch]; the reduce kernels add the splits in a
// fixed order, so the result is bitwise reproducible.
#pragma once
#include "r3c_row.h"

namespace r3c {

template <typename T, int MODE, int TR, int TC, int NJ>
__global__ __launch_bounds__(512) void pwdw_kernel(const PwdwArgs a) {
  __shared__ float red[8][16][64];  // one 32 x 32 tile per wave (32 KB)
  constexpr int TAPS = MODE == MODE_T2DW ? 8 : 1;
  constexpr int KB = 16 * NJ;                  // positions per K block
  constexpr int GL = MODE == MODE_T2DW ? 2 : 1;  // 16-byte G loads per MFMA fragment
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, known wave-uniform
  const int g = lane >> 5;
  const int li = lane & 31;

  // Workgroups are dealt to the 8 XCDs round-robin; renumbered so each XCD
  // owns a contiguous eighth, the tile groups of one split (which read the same
  // F rows) share an L2.
  const int ntg = a.ngr * a.ngc;
  const int nwg = gridDim.x;
  const int wid = (nwg & 7) == 0 ? (blockIdx.x & 7) * (nwg >> 3) + (blockIdx.x >> 3) : blockIdx.x;
  const int tg = wid % ntg;
  const int split = wid / ntg;
  const int tgr = tg % a.ngr, tgc = tg / a.ngr;

  // This lane's F rows and G columns; kind 1 = data, 2 = the all-ones
  // operand of the bias gradient, 0 = padding (zeros).  Offsets in bytes,
  // relative to the K block's first position of the sample.
  uint32_t aoff[TR], boff[TC], bsel[TC];
  int akind[TR], bkind[TC];
#pragma unroll
  for (int i = 0; i < TR; ++i) {
    const int f = (tgr * TR + i) * 32 + li;
    akind[i] = f < a.Fc ? 1 : ((a.db_mode == 2 && f == a.Fc) ? 2 : 0);
    aoff[i] = f < a.Fc ? 2u * (uint32_t)(f * a.fs1 + 8 * NJ * g) : 0u;
  }
#pragma unroll
  for (int j = 0; j < TC; ++j) {
    const int c = (tgc * TC + j) * 32 + li;
    const int ncd = TAPS * a.Gc;
    bkind[j] = c < ncd ? 1 : ((a.db_mode == 1 && c == ncd) ? 2 : 0);
    const int gch = c < ncd ? c / TAPS : 0, tap = c < ncd ? c % TAPS : 0;
    if (MODE == MODE_T2DW) {
      // dY row (2d + kd, 2h + kh) of the G grid (2D x 2H x 2W, dense planes),
      // w' from 2 (w0 + 8 NJ g).
      boff[j] = 2u * (uint32_t)(gch * a.gs1 + (tap >> 2) * 4 * a.HW + ((tap >> 1) & 1) * 2 * a.W + 16 * NJ * g);
      bsel[j] = (tap & 1) ? 0x07060302u : 0x05040100u;  // odd / even halves
    } else {
      boff[j] = 2u * (uint32_t)(gch * a.gs1 + 8 * NJ * g);
      bsel[j] = 0u;
    }
  }
  u32x4_t ones;
  ones[0] = ones[1] = ones[2] = ones[3] = pack2(T::one, T::one);

  f32x16_t acc[TR][TC];
#pragma unroll
  for (int i = 0; i < TR; ++i)
#pragma unroll
    for (int j = 0; j < TC; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Raw loads of one K block: F fragments, and G loads (ConvTranspose: two
  // 16-byte loads per fragment, parity picked at use).
  u32x4_t ra[2][TR][NJ], rb[2][TC][NJ * GL];
  auto gate = [](uint32_t off, bool on) { return (int)(off | ((uint32_t)!on << 31)); };
  // A block past the split (`live` false) is loaded anyway, with every offset
  // out of range (zeros, no memory access): unconditional loads keep the
  // compiler's count of loads in flight exact, so a block's use waits for its
  // own loads only.
  auto issue = [&](int kb, int buf, bool live) __attribute__((always_inline)) {
    const int p0 = live ? kb * KB : 0;  // N * S < 2^31 (host)
    const int n = p0 / a.S;
    const int s0 = p0 - n * a.S;
    const __amdgpu_buffer_rsrc_t fr = make_rsrc_u(a.fsrc + (int64_t)n * a.fs0, a.f_bytes);
    const __amdgpu_buffer_rsrc_t gr = make_rsrc_u(a.gsrc + (int64_t)n * a.gs0, a.g_bytes);
    uint32_t gu;  // uniform G offset (bytes)
    if (MODE == MODE_T2DW) {
      const int d = s0 / a.HW, rem = s0 - d * a.HW;
      const int h = rem / a.W, w0 = rem - h * a.W;
      gu = 2u * (uint32_t)(8 * d * a.HW + 4 * h * a.W + 2 * w0);
    } else {
      gu = 2u * (uint32_t)s0;
    }
    const uint32_t fu = 2u * (uint32_t)s0;
#pragma unroll
    for (int i = 0; i < TR; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        ra[buf][i][j] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(fr, gate(aoff[i] + fu + 16u * j, live & (akind[i] == 1)), 0, 0));
#pragma unroll
    for (int c = 0; c < TC; ++c)
#pragma unroll
      for (int j = 0; j < NJ * GL; ++j)
        rb[buf][c][j] = __builtin_bit_cast(
            u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(gr, gate(boff[c] + gu + 16u * j, live & (bkind[c] == 1)), 0, 0));
  };
  auto compute = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      uint4 af[TR], bf[TC];
#pragma unroll
      for (int i = 0; i < TR; ++i) {
        const u32x4_t v = akind[i] == 2 ? ones : ra[buf][i][j];
        af[i] = __builtin_bit_cast(uint4, v);
      }
#pragma unroll
      for (int c = 0; c < TC; ++c) {
        u32x4_t v;
        if (MODE == MODE_T2DW) {
          const u32x4_t lo = rb[buf][c][2 * j], hi = rb[buf][c][2 * j + 1];
          v[0] = __builtin_amdgcn_perm(lo[1], lo[0], bsel[c]);
          v[1] = __builtin_amdgcn_perm(lo[3], lo[2], bsel[c]);
          v[2] = __builtin_amdgcn_perm(hi[1], hi[0], bsel[c]);
          v[3] = __builtin_amdgcn_perm(hi[3], hi[2], bsel[c]);
        } else {
          v = rb[buf][c][j];
        }
        if (bkind[c] == 2) v = ones;
        bf[c] = __builtin_bit_cast(uint4, v);
      }
#pragma unroll
      for (int i = 0; i < TR; ++i)
#pragma unroll
        for (int c = 0; c < TC; ++c) acc[i][c] = mfma32<T>(af[i], bf[c], acc[i][c]);
    }
  };

  // K blocks of a split, wave w taking every 8th: with kil, blocks
  // (8 i + w) nsplit + s over the whole K axis (the workgroups in flight
  // together stream one window of every plane; measured faster for
  // ConvTranspose), else w, w + 8, ... of the split's contiguous range (faster
  // for k=1, whose streams then spread over all of HBM).  Block kb computes
  // while the wave's next block loads.
  const int kbeg = a.kil ? split : (int)((int64_t)split * a.nkb / a.nsplit);
  const int kend = a.kil ? a.nkb : (int)((int64_t)(split + 1) * a.nkb / a.nsplit);
  const int kstep = a.kil ? 8 * a.nsplit : 8;
  int kb = kbeg + wv * (a.kil ? a.nsplit : 1);
  issue(kb, 0, kb < kend);
  for (; kb < kend; kb += 2 * kstep) {
    issue(kb + kstep, 1, kb + kstep < kend);
    compute(0);
    if (kb + kstep >= kend) break;
    issue(kb + 2 * kstep, 0, kb + 2 * kstep < kend);
    compute(1);
  }

  // Fixed-order sum of the 8 waves' tiles, then the split's partials.
  const int ncd = TAPS * a.Gc;
#pragma unroll
  for (int i = 0; i < TR; ++i) {
#pragma unroll
    for (int c = 0; c < TC; ++c) {
#pragma unroll
      for (int e = 0; e < 16; ++e) red[wv][e][lane] = acc[i][c][e];
      __syncthreads();
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int el = h * 512 + tid;
        const int e = el >> 6, l = el & 63;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < 8; ++w) sum += red[w][e][l];
        // acc[4q + r] of lane (g', i') = C[8q + 4g' + r][i']
        const int f = (tgr * TR + i) * 32 + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
        const int col = (tgc * TC + c) * 32 + (l & 31);
        if (f < a.Fc && col < ncd) {
          const int gch = col / TAPS, tap = col % TAPS;
          a.part[(((size_t)split * a.Fc + f) * TAPS + tap) * a.Gc + gch] = sum;
        } else if (a.db_mode == 1 && f < a.Fc && col == ncd) {
          a.dbpart[(size_t)split * a.Fc + f] = sum;
        } else if (a.db_mode == 2 && f == a.Fc && col < ncd) {
          const int gch = col / TAPS, tap = col % TAPS;
          a.dbpart[((size_t)split * 8 + tap) * a.Gc + gch] = sum;
        }
      }
      __syncthreads();
    }
  }
}

template <typename T, int MODE, int TR, int TC, int NJ>
static void launch_pwdw_inst(const PwdwArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((pwdw_kernel<T, MODE, TR, TC, NJ>), dim3(a.ngr * a.ngc * a.nsplit), dim3(512), 0, stream, a);
}

}  // namespace r3c
