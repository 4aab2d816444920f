// r3c_stem.hip -- Conv3d k=3 stride 1 with ONE input channel: the first layer
// of a volumetric network (the reference's UNet3D enc0 conv, benches/
// unet_e2e.py:32-34, input [4, 1, 64, 128, 128]; the reference planned a
// dedicated dX kernel for it, _dgrad_k3_n1_kernel, conv3d_wmma.py:709-758).
//
// With Cin = 1 the general kernels pad the channel axis to an 8-channel chunk
// (7/8 of their MFMA work and staging is zeros).  Here the 27 taps ARE the
// short GEMM axis instead:
//
//   forward  y[co][p] = b[co] + sum_t w[co][t] x[p + off(t)]
//            D = W (co x 32 taps, zero past 27) * X (32 taps x 32 positions):
//            two v_mfma_f32_32x32x16 per 32 positions and 32 output channels.
//            The B operand (taps x positions) is gathered from LDS with 2-byte
//            reads; the weight operand comes straight from the OIDHW tensor
//            (no pack launch).  Writes |y|: HBM-bound.
//   dW + db  dw[co][t] = sum_p dy[co][p] x[p + off(t)],  db[co] = sum_p dy[co][p]
//            D = dY (co x 16 positions) * X (16 positions x 32 taps): one MFMA
//            per 16 positions and 32 output channels, dY fragments loaded
//            straight from HBM (16 bytes per lane), X fragments as one aligned
//            16-byte LDS read plus its two neighbouring dwords, shifted by the
//            tap's kw with v_alignbit.  Tap column 27 is an all-ones operand,
//            so D[co][27] is db.  Reads |dy| + |x|: HBM-bound.
//
// A job is kStemRows consecutive output rows (n, od, oh0 .. oh0+3), one per
// wave; its workgroup stages the 3 x 6 input rows they read into LDS, row r at
// [r][P] with element w at index 8 + w and zeros around it (the halo of the
// zero padding, pad <= 2).  dW: workgroups walk jobs with a grid stride,
// accumulate in registers, sum their 4 waves in a fixed order and write one
// fp32 partial each; the weight-gradient reduce adds the partials in split
// order, so dW and db are bitwise reproducible.
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

namespace {

constexpr int kStemThreads = 256;                 // kStemRows waves
constexpr int kStemLoads = 5;                     // 16-byte staging loads per thread (W <= kStemMaxW)
static_assert(kStemThreads == 64 * kStemRows, "one wave per output row");
static_assert(kStemLoads * kStemThreads * 8 >= kStemXRows * (kStemMaxW + 24), "staging covers the widest row");

// Input rows of a job into registers: item i = (row, 16-byte group q) of the
// LDS tile, group 0 and groups past the row's data are zeros, as are rows
// outside the volume.
__device__ __forceinline__ void stem_issue(const StemArgs& a, int n, int od, int oh0, uint4 (&v)[kStemLoads]) {
  const int gpr = a.P >> 3;
  const int wg = a.W >> 3;
  const int total = kStemXRows * gpr;
  const uint16_t* xn = a.x + (int64_t)n * a.xs0;
#pragma unroll
  for (int k = 0; k < kStemLoads; ++k) {
    const int i = (int)threadIdx.x + k * kStemThreads;
    const int row = i / gpr, q = i - row * gpr;
    const int kd = row / (kStemRows + 2), rr = row - kd * (kStemRows + 2);
    const int id = od - a.pd + kd, ih = oh0 - a.ph + rr;
    v[k] = make_uint4(0u, 0u, 0u, 0u);
    if (i < total && q >= 1 && q <= wg && (unsigned)id < (unsigned)a.D && (unsigned)ih < (unsigned)a.H)
      v[k] = *reinterpret_cast<const uint4*>(xn + id * a.xs2 + ih * a.xs3 + (q - 1) * 8);
  }
}

__device__ __forceinline__ void stem_commit(const StemArgs& a, uint16_t* xs, const uint4 (&v)[kStemLoads]) {
  const int total = kStemXRows * (a.P >> 3);
#pragma unroll
  for (int k = 0; k < kStemLoads; ++k) {
    const int i = (int)threadIdx.x + k * kStemThreads;
    if (i < total) *reinterpret_cast<uint4*>(xs + i * 8) = v[k];  // row * P + 8 q
  }
}

__device__ __forceinline__ void stem_job(const StemArgs& a, int job, int& n, int& od, int& oh0) {
  const int rb = job % a.nrb;
  const int t = job / a.nrb;
  od = t % a.OD;
  n = t / a.OD;
  oh0 = rb * kStemRows;
}

// Tap t = (kd, kh, kw) -> LDS offset of its input element relative to the
// element of tap (0, 0, 0) of the same output position.
__device__ __forceinline__ int stem_tap_off(int t, int P) {
  const int kd = t / 9, kh = (t / 3) % 3, kw = t % 3;
  return (kd * (kStemRows + 2) + kh) * P + kw;
}

// Forward output staging: per wave [32 NB][kStemTP] values after the input
// tile (pitch of 144 bytes: 16-byte aligned rows, the two lane halves' rows
// 4 apart land 16 banks apart).
constexpr int kStemTP = 72;
__device__ __forceinline__ int stem_tile_elems(const StemArgs& a) { return kStemXRows * a.P; }

template <typename T, int NB>
__global__ __launch_bounds__(kStemThreads) void stem_fwd_kernel(const StemArgs a) {
  extern __shared__ uint4 stem_smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(stem_smem);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, li = lane & 31;
  int n, od, oh0;
  stem_job(a, blockIdx.x, n, od, oh0);
  {
    uint4 v[kStemLoads];
    stem_issue(a, n, od, oh0, v);
    stem_commit(a, xs, v);
  }
  // Weight operand (rows = output channels): lane (co = 32 nb + li, g) holds
  // taps 16 m + 8 g .. +7 of its channel, zero past tap 26 or channel Cout-1.
  uint4 wa[NB][2];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int co = nb * 32 + li;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      uint32_t wd[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const int t0 = 16 * m + 8 * g + 2 * p;
        const uint16_t lo = (co < a.Cout && t0 < 27) ? a.w[co * 27 + t0] : (uint16_t)0;
        const uint16_t hi = (co < a.Cout && t0 + 1 < 27) ? a.w[co * 27 + t0 + 1] : (uint16_t)0;
        wd[p] = pack2(lo, hi);
      }
      wa[nb][m] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
  }
  // Bias of the lane's output channels co = 32 nb + 8 q + 4 g + r.
  float bias[NB][16];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int co = nb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
      bias[nb][v] = (a.b && co < a.Cout) ? to_f32<T>(a.b[co]) : 0.f;
    }
  // LDS offsets of the lane's 16 taps (taps past 26 read tap 0's element and
  // are zeroed after the read).
  int toff[2][8];
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 16 * m + 8 * g + e;
      toff[m][e] = t < 27 ? stem_tap_off(t, a.P) : 0;
    }
  __syncthreads();
  const int oh = oh0 + wv;
  if (oh >= a.OH) return;  // no barrier follows
  const int rowb = wv * a.P + 8 - a.pw + li;
  uint16_t* yrow = a.y + (int64_t)n * a.ys0 + (int64_t)od * a.ys2 + (int64_t)oh * a.ys3;
  // Positions contiguous (yvec8): a pair of tiles goes through this wave's
  // LDS block [32 NB channels][kStemTP] as output values, then out as 16-byte
  // stores, 8 lanes per channel row of 64 positions (one 128-byte line).
  uint16_t* tb = xs + stem_tile_elems(a) + wv * (32 * NB * kStemTP);
  const int step = a.yvec8 ? 64 : 32;
  for (int w0 = 0; w0 < a.OW; w0 += step) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int wt = w0 + 32 * h;
      if (h == 1 && (!a.yvec8 || wt >= a.OW)) break;  // uniform
      const int base = rowb + wt;
      uint4 bx[2];
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        uint32_t wd[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) wd[p] = pack2(xs[base + toff[m][2 * p]], xs[base + toff[m][2 * p + 1]]);
        bx[m] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
      }
      if (g) {  // taps 24 .. 31 of the second product: keep 24, 25, 26
        bx[1].y &= 0xffffu;
        bx[1].z = 0u;
        bx[1].w = 0u;
      }
      f32x16_t acc[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;
        acc[nb] = mfma32<T>(wa[nb][0], bx[0], acc[nb]);
        acc[nb] = mfma32<T>(wa[nb][1], bx[1], acc[nb]);
      }
      // acc[nb][4q + r] = y[co = 32 nb + 8 q + 4 g + r][position wt + li].
      if (a.yvec8) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int co = nb * 32 + 8 * (v >> 2) + 4 * g + (v & 3);
            tb[co * kStemTP + 32 * h + li] = from_f32<T>(acc[nb][v] + bias[nb][v]);
          }
        continue;
      }
      const int pos = wt + li;
      if (pos < a.OW) {
        uint16_t* yp = yrow + (int64_t)pos * a.ys4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int c0 = nb * 32 + 8 * q + 4 * g;
            if (nb * 32 + 8 * q >= a.Cout) break;  // uniform
            if (a.yvec4) {                         // channels contiguous: 4 channels in one 8-byte store
              if (c0 < a.Cout) {
                const uint32_t lo = pack2(from_f32<T>(acc[nb][4 * q] + bias[nb][4 * q]),
                                          from_f32<T>(acc[nb][4 * q + 1] + bias[nb][4 * q + 1]));
                const uint32_t hi = pack2(from_f32<T>(acc[nb][4 * q + 2] + bias[nb][4 * q + 2]),
                                          from_f32<T>(acc[nb][4 * q + 3] + bias[nb][4 * q + 3]));
                *reinterpret_cast<uint2*>(yp + c0) = make_uint2(lo, hi);
              }
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (c0 + r < a.Cout) yp[(int64_t)(c0 + r) * a.ys1] = from_f32<T>(acc[nb][4 * q + r] + bias[nb][4 * q + r]);
            }
          }
      }
    }
    if (a.yvec8) {
      // Item (co, 8-position segment); OW % 8 == 0, so a segment is whole or absent.
      for (int it = lane; it < a.Cout * 8; it += 64) {
        const int co = it >> 3, sg = it & 7;
        const int p0 = w0 + 8 * sg;
        if (p0 < a.OW)
          *reinterpret_cast<uint4*>(yrow + (int64_t)co * a.ys1 + p0) =
              *reinterpret_cast<const uint4*>(tb + co * kStemTP + 8 * sg);
      }
    }
  }
}

template <typename T, int NB>
__global__ __launch_bounds__(kStemThreads) void stem_dw_kernel(const StemArgs a) {
  extern __shared__ uint4 stem_smem[];
  uint16_t* xs = reinterpret_cast<uint16_t*>(stem_smem);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 5, li = lane & 31;
  // This lane's tap column t = li: its input row in the tile and its kw
  // shift.  The 8 elements it needs start o = kw - pw + 2 elements into the
  // 12-element window [base - 2, base + 10) (pre dword, 16 aligned bytes,
  // post dword): dword widx, plus one element when o is odd.
  const int t = li;
  const int kd = t / 9, kh = (t / 3) % 3, kw = t % 3;
  const int o = (t < 27 ? kw : 1) - a.pw + 2;
  const int widx = o >> 1;
  const uint32_t sh = (uint32_t)(o & 1) * 16u;
  const int roff = ((t < 27 ? kd * (kStemRows + 2) + kh : 0) + wv) * a.P + 8 + 8 * g;
  const uint32_t ones = pack2(T::one, T::one);
  f32x16_t acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[nb][e] = 0.f;

  // dY operand (rows = output channels) of one 128-position segment: lane
  // (co = 32 nb + li, g) holds positions w0 + 16 kb + 8 g .. +7 of its channel.
  auto load_dy = [&](int n, int od, int oh, int w0, uint4 (&af)[8][NB]) __attribute__((always_inline)) {
    const bool rv = oh < a.OH;
    const uint16_t* dyr = a.dy + (int64_t)n * a.ys0 + (int64_t)od * a.ys2 + (int64_t)(rv ? oh : 0) * a.ys3 + 8 * g;
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int co = nb * 32 + li;
        af[kb][nb] = make_uint4(0u, 0u, 0u, 0u);
        if (rv && co < a.Cout && w0 + 16 * kb < a.OW)
          af[kb][nb] = *reinterpret_cast<const uint4*>(dyr + (int64_t)co * a.ys1 + w0 + 16 * kb);
      }
  };

  // Software pipeline: while a job computes, the next job's input rows and
  // first dY segment are in flight (issued unconditionally -- past the last
  // job they re-read the current one -- so the compiler's load counting lets
  // each use wait only for its own loads).
  int n, od, oh0;
  stem_job(a, blockIdx.x, n, od, oh0);
  uint4 v[kStemLoads], afn[8][NB];
  stem_issue(a, n, od, oh0, v);
  load_dy(n, od, oh0 + wv, 0, afn);
  for (int job = blockIdx.x; job < a.njobs; job += gridDim.x) {
    const int cn = n, cod = od, coh = oh0 + wv;
    __syncthreads();  // the previous job's LDS reads are done
    stem_commit(a, xs, v);
    __syncthreads();
    uint4 af[8][NB];
#pragma unroll
    for (int kb = 0; kb < 8; ++kb)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) af[kb][nb] = afn[kb][nb];
    {
      const int nj = job + (int)gridDim.x < a.njobs ? job + (int)gridDim.x : job;
      stem_job(a, nj, n, od, oh0);
      stem_issue(a, n, od, oh0, v);
      load_dy(n, od, oh0 + wv, 0, afn);
    }
    if (coh < a.OH) {
      for (int w0 = 0; w0 < a.OW; w0 += 128) {
        if (w0 > 0) load_dy(cn, cod, coh, w0, af);  // rows past 128 positions
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
          if (w0 + 16 * kb >= a.OW) break;  // uniform
          const int base = roff + w0 + 16 * kb;
          const u32x4_t mid = *reinterpret_cast<const u32x4_t*>(xs + base);
          const uint32_t win[6] = {*reinterpret_cast<const uint32_t*>(xs + base - 2), mid[0], mid[1], mid[2], mid[3],
                                   *reinterpret_cast<const uint32_t*>(xs + base + 8)};
          uint32_t s5[5];
#pragma unroll
          for (int k = 0; k < 5; ++k) s5[k] = widx == 0 ? win[k] : (widx == 1 ? win[k + 1] : (k + 2 < 6 ? win[k + 2] : 0u));
          uint32_t bw[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) bw[i] = __builtin_amdgcn_alignbit(s5[i + 1], s5[i], sh);
          if (t == 27) bw[0] = bw[1] = bw[2] = bw[3] = ones;          // db column
          else if (t > 27) bw[0] = bw[1] = bw[2] = bw[3] = 0u;
          const uint4 b = make_uint4(bw[0], bw[1], bw[2], bw[3]);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc[nb] = mfma32<T>(af[kb][nb], b, acc[nb]);
        }
      }
    }
  }
  // The workgroup's partial: its 4 waves summed in wave order through LDS.
  __syncthreads();
  float* red = reinterpret_cast<float*>(stem_smem);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int e = 0; e < 16; ++e) red[((wv * NB + nb) * 16 + e) * 64 + lane] = acc[nb][e];
  __syncthreads();
  constexpr int PER = NB * 16 * 64;
  for (int e = tid; e < PER; e += kStemThreads) {
    const float s = ((red[e] + red[PER + e]) + red[2 * PER + e]) + red[3 * PER + e];
    const int l = e & 63, v = (e >> 6) & 15, nb = e >> 10;
    const int co = nb * 32 + 8 * (v >> 2) + 4 * (l >> 5) + (v & 3), tt = l & 31;
    if (co < a.Cout) {
      if (tt < 27) a.part[((size_t)blockIdx.x * a.Cout + co) * 27 + tt] = s;
      else if (tt == 27 && a.dbpart) a.dbpart[(size_t)blockIdx.x * a.Cout + co] = s;
    }
  }
}

template <typename T, int NB>
void launch_nb(int pass, const StemArgs& a, size_t lds, hipStream_t s) {
  if (pass == 0)
    hipLaunchKernelGGL((stem_fwd_kernel<T, NB>), dim3((unsigned)a.njobs), dim3(kStemThreads), lds, s, a);
  else
    hipLaunchKernelGGL((stem_dw_kernel<T, NB>), dim3((unsigned)a.nsplit), dim3(kStemThreads), lds, s, a);
}

template <typename T>
bool launch_t(int pass, const StemArgs& a, size_t lds, hipStream_t s) {
  if (a.Cout <= 32) launch_nb<T, 1>(pass, a, lds, s);
  else if (a.Cout <= 64) launch_nb<T, 2>(pass, a, lds, s);
  else return false;
  return true;
}

}  // namespace

bool launch_stem(int dtype, int pass, const StemArgs& a, size_t lds, hipStream_t s) {
  return dtype == DT_BF16 ? launch_t<bf16_tag>(pass, a, lds, s) : launch_t<f16_tag>(pass, a, lds, s);
}

}  // namespace r3c
