// r3c_t2dx.h -- register-direct ConvTranspose k2s2 dX for gfx950 on
// v_mfma_f32_32x32x16 (template body), for a w-contiguous dY and a dX with
// dense planes (NCDHW):
//
//   dX[ci][p] = sum_{co, tap} w[ci][co][tap] * dY[co][2p + tap]
//   (src/rdna4_conv3d/conv3d_wmma.py:863-931)
//
// as C^T[ci][p] = sum_k A[ci][k] B[k][p] with k = 8 co + tap (taps in kd, kh,
// kw order), A[ci][k] = w[ci][co][tap].
//
// MFMA operand placement (lane l, g = l / 32, i = l % 32): A[i][8g .. 8g+7],
// B[8g .. 8g+7][i], acc[4q + r] = C[8q + 4g + r][i].  Columns are 32
// consecutive positions p of one sample, so lane (g, i)'s B fragment for
// k-step s is the 2 x 2 x 2 dY block of channel co = 2s + g under its own
// position: four 4-byte loads of (kw = 0, 1) pairs at rows (kd, kh), with the
// 32 lanes of a half-wave reading 128 contiguous bytes per load, straight from
// global memory into the fragment (no LDS tile, no transposition).  The
// stores write acc[4q + r] (channel 8q + 4g + r, position i) as 2-byte stores,
// 64 contiguous bytes per half-wave.
//
// Workgroup: 8 waves, one row group (RB row blocks of 32 input channels) whose
// A fragments sit in LDS, and a set of column blocks taken round-robin by the
// waves.  A stage is (column block, chunk of KC k-steps); its B loads are
// issued one stage ahead into a second register set, so a wave always has a
// stage of loads in flight.  No barrier after the A staging.
//
// The row kernel's staging of a w-contiguous dY for this pass moves 8 scalar
// halves per 16-byte slot; reading the pairs directly is what makes this
// layout fast (measured 143 -> 66 us at [4,48,32,64,64] <- 24 channels).
#pragma once
#include "r3c_row.h"

namespace r3c {

template <typename T, int RB, int KC>
__global__ __launch_bounds__(512) void t2dx_kernel(const T2dxArgs a) {
  extern __shared__ uint4 afr[];  // [RB][nks][64] A fragments of this row group
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, known wave-uniform
  const int g = lane >> 5;
  const int li = lane & 31;
  const int nks = a.nks;
  const int rg = blockIdx.x % a.nrg;
  const int wc = blockIdx.x / a.nrg;
  {
    const uint4* src = reinterpret_cast<const uint4*>(a.apk) + (size_t)rg * RB * nks * 64;
    for (int e = tid; e < RB * nks * 64; e += 512) afr[e] = src[e];
  }
  __syncthreads();

  const int nkc = (nks + KC - 1) / KC;
  const int cstride = a.ncw * 8;
  const int cb_first = wc * 8 + wv;
  const int nmy = cb_first < a.ncb ? (a.ncb - cb_first + cstride - 1) / cstride : 0;
  const int nstage = nmy * nkc;

  // Per-lane position of a column block: sample n, position s in it, and the
  // dY offset (elements) of the 2 x 2 x 2 block at (2d, 2h, 2w).
  struct Pos {
    int n, s, ybase;
  };
  auto pos_of = [&](int cb) __attribute__((always_inline)) {
    Pos P;
    const int p0 = cb * 32;
    P.n = p0 / a.S;
    P.s = p0 - P.n * a.S + li;
    const int d = P.s / a.HW, rem = P.s - d * a.HW;
    const int h = rem / a.W, w = rem - h * a.W;
    P.ybase = 2 * d * a.ys2 + 2 * h * a.ys3 + 2 * w;
    return P;
  };

  u32x4_t breg[2][KC];
  auto gate = [](uint32_t off, bool on) { return (int)(off | ((uint32_t)!on << 31)); };
  // B loads of one stage (chunk kc of a column block) into register set
  // `set`; a stage past the end is loaded with every offset out of range
  // (zeros, no memory access), which keeps the compiler's load counting exact.
  auto issue = [&](const Pos& P, int kc, int set, bool live) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t src = make_rsrc_u(a.dy + (live ? (int64_t)P.n * a.ys0 : 0), a.dy_bytes);
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int co = 2 * (kc * KC + j) + g;
      const bool ok = live && co < a.Cout;
      const uint32_t base = 2u * (uint32_t)(co * a.ys1 + P.ybase);
#pragma unroll
      for (int q = 0; q < 4; ++q)  // q = 2 kd + kh: taps (kd, kh, kw = 0 / 1)
        breg[set][j][q] = __builtin_amdgcn_raw_buffer_load_b32(
            src, gate(base + 2u * (uint32_t)((q >> 1) * a.ys2 + (q & 1) * a.ys3), ok), 0, 0);
    }
  };

  f32x16_t acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[rb][e] = 0.f;

  auto epilogue = [&](const Pos& P) __attribute__((always_inline)) {
    const __amdgpu_buffer_rsrc_t dst = make_rsrc_u(a.dx + (int64_t)P.n * a.xs0, a.dx_bytes);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int ci = (rg * RB + rb) * 32 + 8 * q + 4 * g + r;
          const uint32_t off = 2u * (uint32_t)(ci * a.xs1 + P.s);
          __builtin_amdgcn_raw_buffer_store_b16(from_f32<T>(acc[rb][4 * q + r]), dst, gate(off, ci < a.Cin), 0, 0);
        }
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[rb][e] = 0.f;
    }
  };

  // Stage t = (column block cb_first + (t / nkc) * cstride, chunk t % nkc).
  int cb_i = cb_first, kc_i = 0;  // next stage to issue
  Pos Pi = pos_of(cb_i < a.ncb ? cb_i : 0);
  Pos Pc = Pi;                    // column block being computed
  issue(Pi, 0, 0, nstage > 0);
  auto adv = [&]() __attribute__((always_inline)) {
    if (++kc_i == nkc) {
      kc_i = 0;
      cb_i += cstride;
      Pi = pos_of(cb_i < a.ncb ? cb_i : 0);
    }
  };
  adv();
  auto run = [&](int t, auto set_c) __attribute__((always_inline)) {
    constexpr int SET = decltype(set_c)::value;
    issue(Pi, kc_i, 1 - SET, t + 1 < nstage);
    const int kc = t % nkc;
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int ks = kc * KC + j;
      if (ks < nks) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          acc[rb] = mfma32<T>(afr[(rb * nks + ks) * 64 + lane], __builtin_bit_cast(uint4, breg[SET][j]), acc[rb]);
      }
    }
    if (kc == nkc - 1) {
      epilogue(Pc);
      Pc = Pi;  // stage t + 1 (already issued) starts the next column block
    }
    adv();
  };
  for (int t = 0; t < nstage; t += 2) {
    run(t, std::integral_constant<int, 0>{});
    if (t + 1 < nstage) run(t + 1, std::integral_constant<int, 1>{});
  }
}

// A-fragment packing: out[rb][ks][lane] = 8 weights A[32 rb + i][16 ks + 8g + e]
// = w[ci][co][tap] with k = 8 co + tap (zero outside Cin x 8 Cout).
__global__ __launch_bounds__(256) void t2dx_pack_kernel(const T2dxPackArgs a) {
  const int v = (int)(blockIdx.x * 256 + threadIdx.x);
  if (v >= a.total) return;
  const int lane = v & 63;
  const int rest = v >> 6;
  const int ks = rest % a.nks, rb = rest / a.nks;
  const int ci = rb * 32 + (lane & 31);
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = ks * 16 + 8 * (lane >> 5) + e;
    const uint32_t h = (ci < a.cin && k < 8 * a.cout) ? a.w[((int64_t)ci * a.cout + (k >> 3)) * 8 + (k & 7)] : 0u;
    w[e >> 1] |= h << (16 * (e & 1));
  }
  reinterpret_cast<uint4*>(a.out)[v] = make_uint4(w[0], w[1], w[2], w[3]);
}

template <typename T, int RB, int KC>
static void launch_t2dx_inst(const T2dxArgs& a, size_t lds, hipStream_t stream) {
  auto kern = t2dx_kernel<T, RB, KC>;
  if (lds > 65536) (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  hipLaunchKernelGGL(kern, dim3(a.nrg * a.ncw), dim3(512), lds, stream, a);
}

}  // namespace r3c
