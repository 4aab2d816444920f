/*
 * rdna4_conv3d.h -- C ABI of the gfx950 (MI355X) Conv3d / ConvTranspose3d library.
 *
 * The library (librdna4_conv3d_hip.so) implements the hot path of the
 * reference package's autograd Functions as hand-written HIP kernels on CDNA4
 * bf16/fp16 MFMA (v_mfma_f32_32x32x16_{bf16,f16}, fp32 accumulate):
 *
 *   Conv3d k=1 / k=3, stride 1, dilation 1, groups 1: forward, dX, dW (+ fused db)
 *   ConvTranspose3d k=2, stride 2, pad 0:            forward, dX, dW (+ fused db)
 *
 * Conventions shared by every entry point
 *   - All pointers are device pointers on the current HIP device.  The caller
 *     owns every buffer (inputs, outputs and the workspace); nothing is
 *     allocated inside the library.
 *   - Activations are 5-D [n, c, d, h, w] with arbitrary element strides given
 *     in the descriptor, so NCDHW (contiguous) and NDHWC (channels_last_3d) are
 *     both read and written natively, without layout copies.
 *   - Weights are contiguous in PyTorch's parameter layout: Conv3d
 *     (Cout, Cin, k, k, k); ConvTranspose3d (Cin, Cout, 2, 2, 2).
 *   - `stream` is a hipStream_t (0 = the null stream).  Work is enqueued
 *     asynchronously; nothing synchronises.
 *   - Return value: R3C_OK (0), R3C_UNSUPPORTED (1: the caller should run its
 *     own fallback, e.g. F.conv3d), R3C_INVALID (2: bad argument) or
 *     R3C_HIP_ERROR (3: a HIP launch failed).  On any non-zero return,
 *     r3c_last_error() describes the problem (thread-local string).
 *   - Calls are re-entrant.  Global state: a thread-safe cache of per-device
 *     properties, and the optional launch-timing records (r3c_timing_*),
 *     which are off unless enabled and are guarded by a mutex.
 *   - The workspace holds the packed weight, dW partial sums and, for some
 *     NCDHW inputs, an NDHWC copy of an operand; its size depends on the
 *     descriptor only (strides included), so one query serves every call
 *     with the same descriptor.
 *
 * Which reference interface each entry replaces is cited per function
 * (paths relative to the reference repository root).
 */
#ifndef RDNA4_CONV3D_H
#define RDNA4_CONV3D_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define R3C_ABI_VERSION 1

enum r3c_status {
  R3C_OK = 0,
  R3C_UNSUPPORTED = 1,
  R3C_INVALID = 2,
  R3C_HIP_ERROR = 3
};

enum r3c_dtype {
  R3C_F16 = 0,
  R3C_BF16 = 1,
  R3C_F32 = 2
};

/* Geometry of one convolution, described in forward terms.
 *   x: [n, cin, d, h, w]      y: [n, cout, od, oh, ow]
 * Conv3d:          kernel 1 or 3, od = d + 2*pad_d - kernel + 1 (likewise h, w).
 * ConvTranspose3d: kernel 2 (stride 2, pad 0), od = 2*d (likewise h, w).
 * For the backward entry points x_strides describe dX (or x) and y_strides
 * describe dY, i.e. the same tensors' roles as in forward. */
typedef struct r3c_conv_desc {
  int32_t dtype;                 /* R3C_F16 or R3C_BF16: x, w, bias, y, dy, dx */
  int32_t n, cin, d, h, w;
  int32_t cout, od, oh, ow;
  int32_t kernel;                /* 1, 3 (Conv3d) or 2 (ConvTranspose3d k2s2) */
  int32_t pad_d, pad_h, pad_w;   /* Conv3d zero padding; 0 for ConvTranspose3d */
  int64_t x_strides[5];          /* element strides of x / dX, order (n, c, d, h, w) */
  int64_t y_strides[5];          /* element strides of y / dY, order (n, c, d, h, w) */
} r3c_conv_desc;

/* Library identity.  No reference counterpart (the reference's native module
 * is JIT-built by hip_backend.py:10-25 and has no version query). */
int32_t r3c_abi_version(void);
const char* r3c_last_error(void);
/* 1 when `device` is a gfx950 GPU the kernels were built for, else 0.
 * Replaces the arch gate _is_rdna4() (src/rdna4_conv3d/conv3d_wmma.py:44-48). */
int32_t r3c_device_supported(int32_t device);

/* ---- Conv3d forward: y = conv3d(x, w) + bias ------------------------------
 * Replaces _launch_fwd -> _fwd_k3_kernel / _fwd_k1_kernel / _fwd_kernel
 * (src/rdna4_conv3d/conv3d_wmma.py:1048-1105, 328-444) and the HIP fprop
 * fwd_k3 (src/rdna4_conv3d/conv3d_wmma_hip.hip:148-195).
 * bias may be NULL.  Workspace holds the MFMA-packed weight. */
int64_t r3c_conv3d_fwd_workspace(const r3c_conv_desc* desc);
int32_t r3c_conv3d_fwd(const r3c_conv_desc* desc, const void* x, const void* w,
                       const void* bias, void* y, void* workspace,
                       int64_t workspace_bytes, void* stream);

/* ---- Conv3d dX = conv3d_input(dy, w) ---------------------------------------
 * Replaces _launch_dgrad (src/rdna4_conv3d/conv3d_wmma.py:1108-1179): k3 dX is
 * the forward kernel over dy with the flipped, transposed weight and padding
 * kernel-1-pad (the reference reuses `pad`, correct only for pad=1). */
int64_t r3c_conv3d_dx_workspace(const r3c_conv_desc* desc);
int32_t r3c_conv3d_dx(const r3c_conv_desc* desc, const void* dy, const void* w,
                      void* dx, void* workspace, int64_t workspace_bytes,
                      void* stream);

/* ---- Conv3d dW = conv3d_weight(x, dy) and db = sum(dy) ---------------------
 * Replaces _launch_wgrad -> _wgrad_kernel + partial.sum(0)
 * (src/rdna4_conv3d/conv3d_wmma.py:1182-1214, 544-634) and the bias gradient
 * go.sum(dim=(0,2,3,4)) (conv3d_wmma.py:1318).  Deterministic: fixed split of
 * the position range, fp32 partials, fixed-order reduction, no float atomics.
 * dw is (Cout, Cin, k, k, k) contiguous of dw_dtype (R3C_F32 or desc->dtype);
 * db (may be NULL) is [Cout] of db_dtype. */
int64_t r3c_conv3d_dw_workspace(const r3c_conv_desc* desc);
int32_t r3c_conv3d_dw(const r3c_conv_desc* desc, const void* x, const void* dy,
                      void* dw, int32_t dw_dtype, void* db, int32_t db_dtype,
                      void* workspace, int64_t workspace_bytes, void* stream);

/* ---- Conv3d with stride > 1 (downsampling) ----------------------------------
 * The reference admits stride 1 only (_geom_ok, src/rdna4_conv3d/
 * conv3d_wmma.py:89-95) and sends strided convolutions to F.conv3d /
 * torch.nn.grad (conv3d_wmma.py:1233-1319 fallback legs); these entry points
 * replace those legs.  `stride` points to (sd, sh, sw), each 1 .. 8; `desc`
 * is a Conv3d descriptor whose output dims are (in + 2 pad - k) / stride + 1,
 * kernel 1 or 3, any x / y strides.  Forward and dX: a direct kernel (tiles
 * of one residue class of w for dX; for k = 3, w stride 1 or 2 and up to 32
 * (forward, NCDHW read in place when W % 8 == 0) or 64 (dX) source channels,
 * the source rows staged through LDS);
 * dW + db: a direct kernel for k = 3, w
 * stride 1 or 2, w padding 1, w-contiguous 16-byte aligned rows with W % 8 ==
 * 0 and OW % 16 == 0 (dense NDHWC operands with channels and positions
 * multiples of 8: on NCDHW copies in the workspace), else dY scattered onto
 * the stride-1 output grid and the stride-1 weight-gradient kernels
 * (deterministic either way).
 * pass: 0 forward, 1 dX, 2 dW; the query returns -1 for what no plan runs. */
int64_t r3c_conv3d_strided_workspace(const r3c_conv_desc* desc, const int32_t* stride, int32_t pass);
int32_t r3c_conv3d_strided_fwd(const r3c_conv_desc* desc, const int32_t* stride, const void* x, const void* w,
                               const void* bias, void* y, void* workspace, int64_t workspace_bytes, void* stream);
int32_t r3c_conv3d_strided_dx(const r3c_conv_desc* desc, const int32_t* stride, const void* dy, const void* w,
                              void* dx, void* workspace, int64_t workspace_bytes, void* stream);
int32_t r3c_conv3d_strided_dw(const r3c_conv_desc* desc, const int32_t* stride, const void* x, const void* dy,
                              void* dw, int32_t dw_dtype, void* db, int32_t db_dtype, void* workspace,
                              int64_t workspace_bytes, void* stream);

/* ---- Conv3d over a channel concatenation ------------------------------------
 * No counterpart in the reference package: it replaces the pair
 * torch.cat((a, b), dim=1) + conv3d of the UNet3D decoder (the skip
 * connection, benches/unet_e2e.py:38, examples/drop_in_unet.py:33) without
 * writing the concatenated tensor.  `desc` describes the virtual x =
 * cat(a, b): cin = channels of a + channels of b, x_strides those of a; `ca`
 * is a's channel count (a positive multiple of 8 below cin), and b has the
 * same channel / spatial strides with its own sample stride.  k = 3, NCDHW
 * tensors whose (d, h, w) planes are dense, 16-byte aligned pointers; else
 * R3C_UNSUPPORTED (and the workspace query returns -1): the caller then
 * concatenates and calls r3c_conv3d_fwd / _dx / _dw.  The dX entry point
 * writes the gradients of a and b into two tensors.  pass: 0 forward, 1 dX,
 * 2 dW. */
int64_t r3c_conv3d_cat_workspace(const r3c_conv_desc* desc, int32_t ca,
                                 int64_t xb_sample_stride, int32_t pass);
int32_t r3c_conv3d_cat_fwd(const r3c_conv_desc* desc, int32_t ca,
                           const void* xa, const void* xb,
                           int64_t xb_sample_stride, const void* w,
                           const void* bias, void* y, void* workspace,
                           int64_t workspace_bytes, void* stream);
int32_t r3c_conv3d_cat_dx(const r3c_conv_desc* desc, int32_t ca,
                          const void* dy, const void* w, void* dxa, void* dxb,
                          int64_t xb_sample_stride, void* workspace,
                          int64_t workspace_bytes, void* stream);
int32_t r3c_conv3d_cat_dw(const r3c_conv_desc* desc, int32_t ca,
                          const void* xa, const void* xb,
                          int64_t xb_sample_stride, const void* dy, void* dw,
                          int32_t dw_dtype, void* db, int32_t db_dtype,
                          void* workspace, int64_t workspace_bytes,
                          void* stream);

/* ---- Conv3d dW without a caller workspace -------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): r3c_conv3d_dw with the workspace taken from a static
 * device array of the library (64 MiB, one per GPU, resident until the process
 * ends) instead of an argument.  The caller still passes x, dy, dw and db.
 * Allocates nothing (no hipMalloc / hipFree).  Returns R3C_UNSUPPORTED, with
 * r3c_last_error() naming the bytes needed, when the pass needs more than the
 * array holds (r3c_conv3d_dw_workspace > 64 MiB).  Every call on one GPU uses
 * the same array and overwrites it (no part of it needs to start at zero):
 * calls that overlap on one GPU (different streams or threads) race. */
int32_t r3c_conv3d_dw_static(const r3c_conv_desc* desc, const void* x,
                             const void* dy, void* dw, int32_t dw_dtype,
                             void* db, int32_t db_dtype, void* stream);

/* ---- ConvTranspose3d k=2 s=2 ------------------------------------------------
 * Replace transpose_k2s2_fwd / _dx / _dw (src/rdna4_conv3d/conv3d_wmma.py:
 * 1462-1542, kernels 793-1012) and db = go.sum (conv3d_wmma.py:1576).
 * w is (Cin, Cout, 2, 2, 2) contiguous; dw has the same layout. */
int64_t r3c_convt_k2s2_fwd_workspace(const r3c_conv_desc* desc);
int32_t r3c_convt_k2s2_fwd(const r3c_conv_desc* desc, const void* x,
                           const void* w, const void* bias, void* y,
                           void* workspace, int64_t workspace_bytes,
                           void* stream);
int64_t r3c_convt_k2s2_dx_workspace(const r3c_conv_desc* desc);
int32_t r3c_convt_k2s2_dx(const r3c_conv_desc* desc, const void* dy,
                          const void* w, void* dx, void* workspace,
                          int64_t workspace_bytes, void* stream);
int64_t r3c_convt_k2s2_dw_workspace(const r3c_conv_desc* desc);
int32_t r3c_convt_k2s2_dw(const r3c_conv_desc* desc, const void* x,
                          const void* dy, void* dw, int32_t dw_dtype, void* db,
                          int32_t db_dtype, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* ---- BatchNorm3d + ReLU (the conv -> BN -> ReLU block) ----------------------
 * No counterpart in the reference package: it replaces the nn.BatchNorm3d +
 * nn.ReLU pair of the UNet3D block the reference accelerates
 * (benches/unet_e2e.py:13-21; examples/drop_in_unet.py), with PyTorch's
 * training-mode semantics (batch statistics, biased variance for the
 * normalisation, running statistics updated with the unbiased variance and
 * `momentum`) or evaluation semantics (running statistics).
 * Tensors are [n, c, positions] with each (sample, channel) plane of `s`
 * positions contiguous (NCDHW); element strides of sample and channel are
 * given per tensor.  s, the strides and every pointer must allow 16-byte
 * vectors (s and strides multiples of 8 elements for 16-bit types, 4 for
 * fp32; 16-byte aligned pointers), else R3C_UNSUPPORTED.  gamma / beta may be
 * NULL (no affine transform); running_mean / running_var may be NULL in
 * training mode (no running statistics).  Every reduction has a fixed order:
 * results are bitwise reproducible. */
typedef struct r3c_bn_desc {
  int32_t dtype;              /* R3C_F16, R3C_BF16 or R3C_F32: y, z, dz, dy */
  int32_t n, c;
  int64_t s;                  /* positions per (sample, channel) plane */
  int64_t y_strides[2];       /* sample, channel strides of y (elements) */
  int64_t g_strides[2];       /* of dz (backward) */
  int64_t o_strides[2];       /* of z (forward) or dy (backward) */
  int32_t training;           /* 1: batch statistics; 0: running statistics */
  float eps, momentum;        /* momentum: weight of the batch statistics in the running update */
} r3c_bn_desc;

/* Workspace for both passes (partial sums and per-channel coefficients). */
int64_t r3c_bn_relu_workspace(const r3c_bn_desc* desc);
/* z = relu(batchnorm(y)); save_mean / save_invstd [c] receive the statistics
 * used (batch or running), which the backward takes back. */
int32_t r3c_bn_relu_fwd(const r3c_bn_desc* desc, const void* y, const float* gamma,
                        const float* beta, float* running_mean, float* running_var,
                        void* z, float* save_mean, float* save_invstd,
                        void* workspace, int64_t workspace_bytes, void* stream);
/* dy, dgamma, dbeta (either may be NULL) from dz = dL/dz and the forward's y
 * and saved statistics. */
int32_t r3c_bn_relu_bwd(const r3c_bn_desc* desc, const void* dz, const void* y,
                        const float* gamma, const float* beta,
                        const float* save_mean, const float* save_invstd,
                        void* dy, float* dgamma, float* dbeta,
                        void* workspace, int64_t workspace_bytes, void* stream);

/* ---- MaxPool3d(kernel 2, stride 2) ------------------------------------------
 * No counterpart in the reference package: it replaces nn.MaxPool3d(2) of the
 * UNet3D down path (benches/unet_e2e.py:27-37) with the semantics of
 * PyTorch's CPU kernel (the first maximum of each 2x2x2 window in (kd, kh, kw)
 * order; NaN propagates; an all -inf window picks its first element).
 * The forward also writes a one-byte index per output (kd*4 + kh*2 + kw)
 * that the backward uses; idx is [n][c][d/2][h/2][w/2]
 * contiguous.  Tensors are [n, c, d, h, w] with dense (d, h, w) planes and the
 * given sample / channel strides; d and h must be even and w a multiple of 8,
 * x / dx strides multiples of 8 elements (4 for fp32), y / dy strides
 * multiples of 4, x, y, dx, dy 16-byte and idx 4-byte aligned, else
 * R3C_UNSUPPORTED.  The backward writes every element of dx. */
typedef struct r3c_pool_desc {
  int32_t dtype;              /* R3C_F16, R3C_BF16 or R3C_F32 */
  int32_t n, c, d, h, w;      /* input (x / dx) dims */
  int64_t x_strides[2];       /* sample, channel strides of x / dx (elements) */
  int64_t y_strides[2];       /* of y / dy */
} r3c_pool_desc;
int32_t r3c_maxpool2_fwd(const r3c_pool_desc* desc, const void* x, void* y,
                         uint8_t* idx, void* stream);
int32_t r3c_maxpool2_bwd(const r3c_pool_desc* desc, const void* dy,
                         const uint8_t* idx, void* dx, void* stream);
/* dx = MaxPool3d backward of dy + add: the UNet3D encoder output feeds both
 * the pooling and the decoder's skip connection (benches/unet_e2e.py:33-38),
 * so its gradient is the sum of the two; this writes the sum in the backward's
 * one pass (no counterpart in the reference, where autograd adds them).  `add`
 * has x's shape, sample / channel strides add_strides[0..1] (the x_strides
 * rules) and may be dx itself. */
int32_t r3c_maxpool2_bwd_add(const r3c_pool_desc* desc, const void* dy,
                             const uint8_t* idx, const void* add,
                             const int64_t* add_strides, void* dx, void* stream);

/* ---- MFMA shape probe (measurement only) -------------------------------------
 * No counterpart in the reference.  `blocks` workgroups of 256 threads each
 * issue `iters` rounds of independent bf16 MFMAs of one shape (0:
 * v_mfma_f32_32x32x16, 4 per round, 32768 flops each; 1: 16x16x32, 8 per
 * round, 16384 flops each) and write one float per thread to out
 * (blocks * 256 floats).  The caller times the launch on `stream`. */
int32_t r3c_probe_mfma(int32_t shape, int32_t blocks, int32_t iters,
                       float* out, void* stream);

/* ---- Kernel timing hook (measurement only) ----------------------------------
 * No counterpart in the reference (its benches time whole calls with
 * time.perf_counter, benches/isolated.py:26-34).  While enabled, each kernel
 * launch is bracketed by HIP events on its own launch stream and tagged with
 * the calling thread's current tag and a kernel family
 * (0 weight pack, 1 row kernel, 2 weight-gradient kernel, 3 split reduce,
 * 4 NCDHW-to-NDHWC copy, 5 row-kernel split-K epilogue pass, 6 BatchNorm +
 * ReLU pass: all kernels of one forward or backward call, 7 MaxPool3d pass).
 * r3c_timing_collect waits for the recorded events, writes up to max_records
 * (tag, kind, milliseconds) triples, clears the records and returns how many
 * launches were recorded.  r3c_timing_filter limits recording to launches
 * with the given tag and kind (-1 = any; the default), so one kernel can be
 * timed inside a run without bracketing every other launch. */
int32_t r3c_timing_enable(int32_t on);
void r3c_timing_set_tag(int32_t tag);
void r3c_timing_filter(int32_t tag, int32_t kind);
int32_t r3c_timing_collect(int32_t max_records, int32_t* tags, int32_t* kinds, float* ms);

#ifdef __cplusplus
}
#endif

#endif /* RDNA4_CONV3D_H */
