/*
 * conv3d_oracle.c -- CPU oracle for the Conv3d / ConvTranspose3d hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product links or calls this file;
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only as the checker.
 *
 * It restates, as direct loops with double accumulation, the arithmetic the
 * reference's kernels implement (all tensors NCDHW contiguous, float32 in/out):
 *
 *   conv3d_fwd  y[n,co,o] = b[co] + sum_{ci,t} x[n,ci,o+t-p] w[co,ci,t]
 *               (reference src/rdna4_conv3d/conv3d_wmma.py:372-444, K3 kernel;
 *               328-369, K1 kernel; oracle there: F.conv3d)
 *   conv3d_dx   dx[n,ci,i] = sum_{co,t} dy[n,co,i-t+p] w[co,ci,t]
 *               (the transpose of fwd; conv3d_wmma.py:1108-1179; oracle:
 *               torch.nn.grad.conv3d_input)
 *   conv3d_dw   dw[co,ci,t] = sum_{n,o} dy[n,co,o] x[n,ci,o+t-p];
 *               db[co] = sum_{n,o} dy[n,co,o]
 *               (conv3d_wmma.py:544-634 and 1318)
 *   convt_fwd   y[n,co,2i+t] = b[co] + sum_ci x[n,ci,i] w[ci,co,t]   (k=2, s=2)
 *               (conv3d_wmma.py:793-860)
 *   convt_dx    dx[n,ci,i] = sum_{co,t} dy[n,co,2i+t] w[ci,co,t]     (863-931)
 *   convt_dw    dw[ci,co,t] = sum_{n,i} x[n,ci,i] dy[n,co,2i+t];
 *               db[co] = sum dy                                        (934-1012, 1576)
 *
 * Taps t are (kd,kh,kw) in row-major order.  Out-of-range input positions are
 * zero (zero padding).
 *
 * oracle_set_fault() plants a known mistake (tests use it to prove that the
 * oracle's pins catch that class of error); 0 means no fault.
 */
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static int g_fault = 0;

void oracle_set_fault(int f) { g_fault = f; }
int oracle_get_fault(void) { return g_fault; }

enum {
  FAULT_NONE = 0,
  FAULT_FWD_PAD_OFF_BY_ONE = 1, /* fwd reads x[o + t - p + 1] */
  FAULT_DX_NO_FLIP = 2,         /* dx uses w[t] at i + t - p instead of i - t + p */
  FAULT_DW_SWAP_HW = 3,         /* dw writes tap (kd,kw,kh) */
  FAULT_CONVT_TAP_ORDER = 4,    /* convt fwd uses tap kw*4+kh*2+kd */
  FAULT_DB_DROPPED = 5          /* conv db left at zero */
};

static inline size_t idx5(int n, int c, int d, int h, int w, int C, int D, int H, int W) {
  return ((((size_t)n * C + c) * D + d) * H + h) * W + w;
}

void oracle_conv3d_fwd(const float* x, const float* w, const float* b, float* y, int N, int Cin, int D, int H,
                       int W, int Cout, int K, int pd, int ph, int pw) {
  const int OD = D + 2 * pd - K + 1, OH = H + 2 * ph - K + 1, OW = W + 2 * pw - K + 1;
  const int shift = g_fault == FAULT_FWD_PAD_OFF_BY_ONE ? 1 : 0;
  for (int n = 0; n < N; ++n)
    for (int co = 0; co < Cout; ++co)
      for (int od = 0; od < OD; ++od)
        for (int oh = 0; oh < OH; ++oh)
          for (int ow = 0; ow < OW; ++ow) {
            double acc = b ? (double)b[co] : 0.0;
            for (int ci = 0; ci < Cin; ++ci)
              for (int kd = 0; kd < K; ++kd) {
                const int id = od + kd - pd + shift;
                if (id < 0 || id >= D) continue;
                for (int kh = 0; kh < K; ++kh) {
                  const int ih = oh + kh - ph + shift;
                  if (ih < 0 || ih >= H) continue;
                  for (int kw = 0; kw < K; ++kw) {
                    const int iw = ow + kw - pw + shift;
                    if (iw < 0 || iw >= W) continue;
                    acc += (double)x[idx5(n, ci, id, ih, iw, Cin, D, H, W)] *
                           (double)w[idx5(co, ci, kd, kh, kw, Cin, K, K, K)];
                  }
                }
              }
            y[idx5(n, co, od, oh, ow, Cout, OD, OH, OW)] = (float)acc;
          }
}

void oracle_conv3d_dx(const float* dy, const float* w, float* dx, int N, int Cin, int D, int H, int W, int Cout,
                      int K, int pd, int ph, int pw) {
  const int OD = D + 2 * pd - K + 1, OH = H + 2 * ph - K + 1, OW = W + 2 * pw - K + 1;
  const int sgn = g_fault == FAULT_DX_NO_FLIP ? 1 : -1;
  for (int n = 0; n < N; ++n)
    for (int ci = 0; ci < Cin; ++ci)
      for (int id = 0; id < D; ++id)
        for (int ih = 0; ih < H; ++ih)
          for (int iw = 0; iw < W; ++iw) {
            double acc = 0.0;
            for (int co = 0; co < Cout; ++co)
              for (int kd = 0; kd < K; ++kd) {
                const int od = id + sgn * kd + pd;
                if (od < 0 || od >= OD) continue;
                for (int kh = 0; kh < K; ++kh) {
                  const int oh = ih + sgn * kh + ph;
                  if (oh < 0 || oh >= OH) continue;
                  for (int kw = 0; kw < K; ++kw) {
                    const int ow = iw + sgn * kw + pw;
                    if (ow < 0 || ow >= OW) continue;
                    acc += (double)dy[idx5(n, co, od, oh, ow, Cout, OD, OH, OW)] *
                           (double)w[idx5(co, ci, kd, kh, kw, Cin, K, K, K)];
                  }
                }
              }
            dx[idx5(n, ci, id, ih, iw, Cin, D, H, W)] = (float)acc;
          }
}

void oracle_conv3d_dw(const float* x, const float* dy, float* dw, float* db, int N, int Cin, int D, int H, int W,
                      int Cout, int K, int pd, int ph, int pw) {
  const int OD = D + 2 * pd - K + 1, OH = H + 2 * ph - K + 1, OW = W + 2 * pw - K + 1;
  for (int co = 0; co < Cout; ++co)
    for (int ci = 0; ci < Cin; ++ci)
      for (int kd = 0; kd < K; ++kd)
        for (int kh = 0; kh < K; ++kh)
          for (int kw = 0; kw < K; ++kw) {
            double acc = 0.0;
            for (int n = 0; n < N; ++n)
              for (int od = 0; od < OD; ++od) {
                const int id = od + kd - pd;
                if (id < 0 || id >= D) continue;
                for (int oh = 0; oh < OH; ++oh) {
                  const int ih = oh + kh - ph;
                  if (ih < 0 || ih >= H) continue;
                  for (int ow = 0; ow < OW; ++ow) {
                    const int iw = ow + kw - pw;
                    if (iw < 0 || iw >= W) continue;
                    acc += (double)dy[idx5(n, co, od, oh, ow, Cout, OD, OH, OW)] *
                           (double)x[idx5(n, ci, id, ih, iw, Cin, D, H, W)];
                  }
                }
              }
            const int th = g_fault == FAULT_DW_SWAP_HW ? kw : kh;
            const int tw = g_fault == FAULT_DW_SWAP_HW ? kh : kw;
            dw[idx5(co, ci, kd, th, tw, Cin, K, K, K)] = (float)acc;
          }
  if (db) {
    for (int co = 0; co < Cout; ++co) {
      double acc = 0.0;
      if (g_fault != FAULT_DB_DROPPED)
        for (int n = 0; n < N; ++n)
          for (int o = 0; o < OD * OH * OW; ++o) acc += (double)dy[((size_t)n * Cout + co) * OD * OH * OW + o];
      db[co] = (float)acc;
    }
  }
}

static inline int convt_tap(int kd, int kh, int kw) {
  return g_fault == FAULT_CONVT_TAP_ORDER ? kw * 4 + kh * 2 + kd : kd * 4 + kh * 2 + kw;
}

void oracle_convt_fwd(const float* x, const float* w, const float* b, float* y, int N, int Cin, int D, int H, int W,
                      int Cout) {
  const int OD = 2 * D, OH = 2 * H, OW = 2 * W;
  for (int n = 0; n < N; ++n)
    for (int co = 0; co < Cout; ++co)
      for (int id = 0; id < D; ++id)
        for (int ih = 0; ih < H; ++ih)
          for (int iw = 0; iw < W; ++iw)
            for (int kd = 0; kd < 2; ++kd)
              for (int kh = 0; kh < 2; ++kh)
                for (int kw = 0; kw < 2; ++kw) {
                  double acc = b ? (double)b[co] : 0.0;
                  const int t = convt_tap(kd, kh, kw);
                  for (int ci = 0; ci < Cin; ++ci)
                    acc += (double)x[idx5(n, ci, id, ih, iw, Cin, D, H, W)] * (double)w[((size_t)ci * Cout + co) * 8 + t];
                  y[idx5(n, co, 2 * id + kd, 2 * ih + kh, 2 * iw + kw, Cout, OD, OH, OW)] = (float)acc;
                }
}

void oracle_convt_dx(const float* dy, const float* w, float* dx, int N, int Cin, int D, int H, int W, int Cout) {
  const int OD = 2 * D, OH = 2 * H, OW = 2 * W;
  for (int n = 0; n < N; ++n)
    for (int ci = 0; ci < Cin; ++ci)
      for (int id = 0; id < D; ++id)
        for (int ih = 0; ih < H; ++ih)
          for (int iw = 0; iw < W; ++iw) {
            double acc = 0.0;
            for (int co = 0; co < Cout; ++co)
              for (int t = 0; t < 8; ++t) {
                const int kd = t >> 2, kh = (t >> 1) & 1, kw = t & 1;
                acc += (double)dy[idx5(n, co, 2 * id + kd, 2 * ih + kh, 2 * iw + kw, Cout, OD, OH, OW)] *
                       (double)w[((size_t)ci * Cout + co) * 8 + t];
              }
            dx[idx5(n, ci, id, ih, iw, Cin, D, H, W)] = (float)acc;
          }
}

void oracle_convt_dw(const float* x, const float* dy, float* dw, float* db, int N, int Cin, int D, int H, int W,
                     int Cout) {
  const int OD = 2 * D, OH = 2 * H, OW = 2 * W;
  for (int ci = 0; ci < Cin; ++ci)
    for (int co = 0; co < Cout; ++co)
      for (int t = 0; t < 8; ++t) {
        const int kd = t >> 2, kh = (t >> 1) & 1, kw = t & 1;
        double acc = 0.0;
        for (int n = 0; n < N; ++n)
          for (int id = 0; id < D; ++id)
            for (int ih = 0; ih < H; ++ih)
              for (int iw = 0; iw < W; ++iw)
                acc += (double)x[idx5(n, ci, id, ih, iw, Cin, D, H, W)] *
                       (double)dy[idx5(n, co, 2 * id + kd, 2 * ih + kh, 2 * iw + kw, Cout, OD, OH, OW)];
        dw[((size_t)ci * Cout + co) * 8 + t] = (float)acc;
      }
  if (db) {
    for (int co = 0; co < Cout; ++co) {
      double acc = 0.0;
      for (int n = 0; n < N; ++n)
        for (int o = 0; o < OD * OH * OW; ++o) acc += (double)dy[((size_t)n * Cout + co) * OD * OH * OW + o];
      db[co] = (float)acc;
    }
  }
}

/* Round-to-nearest-even float32 -> bfloat16 -> float32 (IEEE definition, NaN kept quiet). */
void oracle_round_bf16(float* v, int64_t count) {
  for (int64_t i = 0; i < count; ++i) {
    uint32_t u;
    memcpy(&u, &v[i], 4);
    if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu)) {
      u |= 0x00400000u;
    } else {
      u += 0x7fffu + ((u >> 16) & 1u);
    }
    u &= 0xffff0000u;
    memcpy(&v[i], &u, 4);
  }
}
