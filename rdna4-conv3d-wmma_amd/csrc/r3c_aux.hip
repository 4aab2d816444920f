// r3c_aux.hip -- weight packing into MFMA fragment order, and the fixed-order
// reduction of the weight-gradient split partials.
#include "r3c_device.h"
#include "r3c_kernels.h"

namespace r3c {

// Packed layout: [chunk][step][colblock][lane][8], lane = 32 * g + j.  Lane
// (g, j) of step s holds k group kg = 2 s + g = (tap, 8-channel group cg) and
// column colblock * 32 + j, i.e. exactly the B operand the row kernel feeds to
// v_mfma_f32_32x32x16.  Out-of-range k or columns are zero.
//
// Weight index maps (w is PyTorch's parameter layout):
//   K1/K3 forward   : Conv3d w (Cout, Cin, t)      -> w[col][ci][tap]
//                     (_pack_weight, src/rdna4_conv3d/conv3d_wmma.py:1023-1026)
//   K1/K3 dX (+16)  : source channel = Cout index, column = Cin index,
//                     tap flipped: w[ci][col][taps-1-tap]
//                     (flip(2,3,4).transpose(0,1), conv3d_wmma.py:1156-1157)
//   T2DX            : ConvTranspose w (Cin, Cout, 8) -> w[col][ci][tap]
//   T2FWD           : column = tap * Cout + co     -> w[ci][co][tap]
//                     (_tr_pack_w, conv3d_wmma.py:1453-1455, columns (tap, co))
__global__ __launch_bounds__(256) void pack_weight_kernel(const PackArgs a) {
  // One thread = one lane's 8-element fragment (16 bytes): index v over
  // [chunk][step][colblock][lane]; 32-bit arithmetic (total < 2^31 elements).
  const int v = (int)(blockIdx.x * 256 + threadIdx.x);
  if ((int64_t)v * 8 >= a.total) return;
  const int lane = v & 63;
  int rest = v >> 6;
  const int nb = rest % a.nbt_pad;
  rest /= a.nbt_pad;
  const int s = rest % a.nstep;
  const int chunk = rest / a.nstep;
  const int g = lane >> 5, j = lane & 31;
  const int g8 = a.ck / 8;
  const int kg = 2 * s + g;
  const int col = nb * 32 + j;
  const int mode = a.mode & 15;
  const bool dx = (a.mode & 16) != 0;
  uint32_t w[4] = {0u, 0u, 0u, 0u};
  if (kg < a.taps * g8 && col < a.ncols) {
    const int tap = kg / g8, cg = kg - (kg / g8) * g8;
    const int ci0 = chunk * a.ck + cg * 8;
    // Element e reads w[base + e * estride] (channel ci0 + e).
    int64_t base, estride;
    if (mode == MODE_K1 || mode == MODE_K3) {
      if (!dx) {
        base = ((int64_t)col * a.w_cin + ci0) * a.taps + tap;
        estride = a.taps;
      } else {
        base = ((int64_t)ci0 * a.w_cin + col) * a.taps + (a.taps - 1 - tap);
        estride = (int64_t)a.w_cin * a.taps;
      }
    } else if (mode == MODE_T2DX) {
      base = ((int64_t)col * a.w_cout + ci0) * 8 + tap;
      estride = 8;
    } else {  // MODE_T2FWD: column (tap, co), or ((kd, kh), co, kw) with kw fastest
      int t8, co;
      if (a.t2kw) {
        const int rest = col >> 1, kdkh = rest / a.w_cout;
        co = rest - kdkh * a.w_cout;
        t8 = kdkh * 2 + (col & 1);
      } else {
        t8 = col / a.w_cout;
        co = col - t8 * a.w_cout;
      }
      base = ((int64_t)ci0 * a.w_cout + co) * 8 + t8;
      estride = (int64_t)a.w_cout * 8;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t h = ci0 + e < a.cs ? a.w[base + e * estride] : 0u;
      w[e >> 1] |= h << (16 * (e & 1));
    }
  }
  reinterpret_cast<uint4*>(a.out)[v] = make_uint4(w[0], w[1], w[2], w[3]);
}

void launch_pack(int dtype, const PackArgs& a, hipStream_t stream) {
  (void)dtype;  // a raw 16-bit copy: the element type does not matter
  const int64_t blocks = (a.total / 8 + 255) / 256;
  hipLaunchKernelGGL(pack_weight_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

// Tile = 512 positions x up to 32 channels of one sample, through LDS:
//   load:  16-byte loads of 8 positions of one channel (lanes along positions,
//          so each instruction reads 1 KB of a channel plane) -> LDS [c][p];
//   store: each lane gathers 8 channels of one position from LDS and stores
//          them as one 16-byte vector; consecutive lanes take consecutive
//          vectors of the output, so each instruction writes 1 KB contiguously
//          when C <= 32 (64-byte runs otherwise).
constexpr int kLayoutTileP = 512;
constexpr int kLayoutPitch = kLayoutTileP + 8;  // halves per LDS row (spreads banks)

__global__ __launch_bounds__(256) void to_channels_last_kernel(const LayoutArgs a) {
  __shared__ uint16_t tile[32 * kLayoutPitch];
  const int ncb = (a.C + 31) >> 5;
  const int64_t ntiles = (a.S + kLayoutTileP - 1) / kLayoutTileP;
  int64_t b = blockIdx.x;
  const int64_t pt = b % ntiles;
  b /= ntiles;
  const int cb = (int)(b % ncb);
  const int64_t n = b / ncb;
  const int c0 = cb * 32;
  const int cw = a.C - c0 >= 32 ? 32 : a.C - c0;  // channels in this block (multiple of 8)
  const int64_t p0 = pt * kLayoutTileP;
  const int np = a.S - p0 >= kLayoutTileP ? kLayoutTileP : (int)(a.S - p0);  // multiple of 8
  const int tid = threadIdx.x;

  const uint16_t* src = a.src + ((size_t)n * a.C + c0) * a.S + p0;
  const int ngrp = np >> 3;
  for (int it = tid; it < cw * ngrp; it += 256) {
    const int c = it / ngrp, j = it - (it / ngrp) * ngrp;
    const uint4 v = *reinterpret_cast<const uint4*>(src + (size_t)c * a.S + j * 8);
    *reinterpret_cast<uint4*>(tile + c * kLayoutPitch + j * 8) = v;
  }
  __syncthreads();
  const int cgw = cw >> 3;
  uint16_t* dst = a.dst + ((size_t)n * a.S + p0) * a.C + c0;
  for (int u = tid; u < np * cgw; u += 256) {
    const int p = u / cgw, cg = u - (u / cgw) * cgw;
    const uint16_t* t = tile + cg * 8 * kLayoutPitch + p;
    uint4 v;
    v.x = pack2(t[0], t[kLayoutPitch]);
    v.y = pack2(t[2 * kLayoutPitch], t[3 * kLayoutPitch]);
    v.z = pack2(t[4 * kLayoutPitch], t[5 * kLayoutPitch]);
    v.w = pack2(t[6 * kLayoutPitch], t[7 * kLayoutPitch]);
    *reinterpret_cast<uint4*>(dst + (size_t)p * a.C + cg * 8) = v;
  }
}

void launch_to_channels_last(const LayoutArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.S + kLayoutTileP - 1) / kLayoutTileP * ((a.C + 31) >> 5) * a.N;
  hipLaunchKernelGGL(to_channels_last_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

// The inverse copy (NDHWC -> NCDHW), same tiles: each lane loads 8 channels of
// one position as one 16-byte vector (consecutive lanes on consecutive vectors
// of the source) and scatters them into LDS [c][p]; then 16-byte stores of 8
// positions of one channel, lanes along positions.
__global__ __launch_bounds__(256) void to_channels_first_kernel(const LayoutArgs a) {
  __shared__ __align__(16) uint16_t tile[32 * kLayoutPitch];
  const int ncb = (a.C + 31) >> 5;
  const int64_t ntiles = (a.S + kLayoutTileP - 1) / kLayoutTileP;
  int64_t b = blockIdx.x;
  const int64_t pt = b % ntiles;
  b /= ntiles;
  const int cb = (int)(b % ncb);
  const int64_t n = b / ncb;
  const int c0 = cb * 32;
  const int cw = a.C - c0 >= 32 ? 32 : a.C - c0;  // channels in this block (multiple of 8)
  const int64_t p0 = pt * kLayoutTileP;
  const int np = a.S - p0 >= kLayoutTileP ? kLayoutTileP : (int)(a.S - p0);  // multiple of 8
  const int tid = threadIdx.x;

  const uint16_t* src = a.src + ((size_t)n * a.S + p0) * a.C + c0;
  const int cgw = cw >> 3;
  for (int u = tid; u < np * cgw; u += 256) {
    const int p = u / cgw, cg = u - (u / cgw) * cgw;
    const uint4 v = *reinterpret_cast<const uint4*>(src + (size_t)p * a.C + cg * 8);
    uint16_t* t = tile + cg * 8 * kLayoutPitch + p;
    const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      t[(2 * e) * kLayoutPitch] = (uint16_t)(q[e] & 0xffffu);
      t[(2 * e + 1) * kLayoutPitch] = (uint16_t)(q[e] >> 16);
    }
  }
  __syncthreads();
  uint16_t* dst = a.dst + ((size_t)n * a.C + c0) * a.S + p0;
  const int ngrp = np >> 3;
  for (int it = tid; it < cw * ngrp; it += 256) {
    const int c = it / ngrp, j = it - (it / ngrp) * ngrp;
    *reinterpret_cast<uint4*>(dst + (size_t)c * a.S + j * 8) =
        *reinterpret_cast<const uint4*>(tile + c * kLayoutPitch + j * 8);
  }
}

void launch_to_channels_first(const LayoutArgs& a, hipStream_t stream) {
  const int64_t blocks = (a.S + kLayoutTileP - 1) / kLayoutTileP * ((a.C + 31) >> 5) * a.N;
  hipLaunchKernelGGL(to_channels_first_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
}

template <typename T>
__device__ __forceinline__ void store_elem(void* base, int64_t i, int dtype, float v) {
  (void)sizeof(T);
  if (dtype == DT_F32) reinterpret_cast<float*>(base)[i] = v;
  else if (dtype == DT_BF16) reinterpret_cast<uint16_t*>(base)[i] = from_f32<bf16_tag>(v);
  else reinterpret_cast<uint16_t*>(base)[i] = from_f32<f16_tag>(v);
}

// Element e of the reduce: [0, Fc*taps*Gc) are dW, walked with G fastest
// (matching the partial layout, so a wave reads consecutive floats); the tail
// holds db.  split_sum adds splits s0, s0 + step, ... below s1 of one element
// in increasing order.
__device__ __forceinline__ float split_sum(const ReduceArgs& a, int64_t e, int64_t nw, int s0, int s1, int step = 1) {
  float sum = 0.f;
  if (e < nw) {
    const int gch = (int)(e % a.Gc);
    const int64_t r = e / a.Gc;
    const int tap = (int)(r % a.taps);
    const int f = (int)(r / a.taps);
    const size_t stride = (size_t)a.Fpad * a.taps * a.Gpad;
    const float* p = a.part + ((size_t)f * a.taps + tap) * a.Gpad + gch;
#pragma unroll 8
    for (int s = s0; s < s1; s += step) sum += p[(size_t)s * stride];
  } else {
    const int c = (int)(e - nw);
    if (a.db_mode == 1) {
#pragma unroll 8
      for (int s = s0; s < s1; s += step) sum += a.dbpart[(size_t)s * a.Fpad + c];
    } else if (a.taps == 8) {  // ConvTranspose: the 8 tap partials of a split, loads issued together
#pragma unroll 4
      for (int s = s0; s < s1; s += step) {
        const float* q = a.dbpart + (size_t)s * 8 * a.Gpad + c;
        float t = 0.f;
#pragma unroll
        for (int tap = 0; tap < 8; ++tap) t += q[(size_t)tap * a.Gpad];
        sum += t;
      }
    } else {
      for (int s = s0; s < s1; s += step) {
        float t = 0.f;
        for (int tap = 0; tap < a.taps; ++tap) t += a.dbpart[((size_t)s * a.taps + tap) * a.Gpad + c];
        sum += t;
      }
    }
  }
  return sum;
}

// Few splits (at most 32): one thread per element adds them in
// split order and converts to the output dtype.  Bitwise reproducible run to
// run: every sum has a fixed order.
__global__ __launch_bounds__(256) void wgrad_reduce_final_kernel(const ReduceArgs a, int64_t nw, int64_t ne) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= ne) return;
  const float tot = split_sum(a, e, nw, 0, a.nsplit);
  if (e < nw) {
    const int gch = (int)(e % a.Gc);
    const int64_t r = e / a.Gc;
    const int tap = (int)(r % a.taps);
    const int f = (int)(r / a.taps);
    store_elem<float>(a.dw, ((int64_t)f * a.Gc + gch) * a.taps + tap, a.dw_dtype, tot);
  } else {
    store_elem<float>(a.db, e - nw, a.db_dtype, tot);
  }
}

// One launch for many splits: a workgroup owns 256 / SG consecutive elements,
// SG threads per element each add every SG-th split in increasing order, and
// thread 0 of each element adds the SG sums in order.  Bitwise reproducible.
template <int SG>
__global__ __launch_bounds__(256) void wgrad_reduce_tree_kernel(const ReduceArgs a, int64_t nw, int64_t ne) {
  constexpr int EPB = 256 / SG;
  __shared__ float sh[256];
  const int t = threadIdx.x;
  const int el = t % EPB, sg = t / EPB;
  const int64_t e = (int64_t)blockIdx.x * EPB + el;
  sh[t] = e < ne ? split_sum(a, e, nw, sg, a.nsplit, SG) : 0.f;
  __syncthreads();
  if (sg != 0 || e >= ne) return;
  float tot = 0.f;
#pragma unroll
  for (int j = 0; j < SG; ++j) tot += sh[j * EPB + el];
  if (e < nw) {
    const int gch = (int)(e % a.Gc);
    const int64_t r = e / a.Gc;
    const int tap = (int)(r % a.taps);
    const int f = (int)(r / a.taps);
    store_elem<float>(a.dw, ((int64_t)f * a.Gc + gch) * a.taps + tap, a.dw_dtype, tot);
  } else {
    store_elem<float>(a.db, e - nw, a.db_dtype, tot);
  }
}

template <int SG>
void launch_tree(const ReduceArgs& a, int64_t nw, int64_t ne, hipStream_t stream) {
  const unsigned blocks = (unsigned)((ne + 256 / SG - 1) / (256 / SG));
  hipLaunchKernelGGL(wgrad_reduce_tree_kernel<SG>, dim3(blocks), dim3(256), 0, stream, a, nw, ne);
}

void launch_wgrad_reduce(const ReduceArgs& a, hipStream_t stream) {
  const int64_t nw = (int64_t)a.Fc * a.taps * a.Gc;
  const int ndb = a.db_mode == 1 ? a.Fc : (a.db_mode == 2 ? a.Gc : 0);
  const int64_t ne = nw + ndb;
  if (a.nsplit <= 32) {  // one thread per element
    const unsigned blocks = (unsigned)((ne + 255) / 256);
    hipLaunchKernelGGL(wgrad_reduce_final_kernel, dim3(blocks), dim3(256), 0, stream, a, nw, ne);
    return;
  }
  // Large partial sets are read at HBM speed only while a wave's load covers
  // long runs of one split row (256 / SG consecutive elements): the fewest
  // threads per element that keep each thread at 16 splits or so.
  if (a.nsplit <= 128) launch_tree<8>(a, nw, ne, stream);
  else if (a.nsplit <= 256) launch_tree<16>(a, nw, ne, stream);
  else if (a.nsplit <= 512) launch_tree<32>(a, nw, ne, stream);
  else launch_tree<64>(a, nw, ne, stream);
}

}  // namespace r3c
