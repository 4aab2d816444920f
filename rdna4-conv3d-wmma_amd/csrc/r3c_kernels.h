// r3c_kernels.h -- kernel argument blocks and host-side launchers.
//
// Two kernel families cover the whole hot path, both on v_mfma_f32_32x32x16:
//
//  * row kernel (r3c_row.h): C[row position][column] = sum_k A[row][k] B[k][col]
//      rows    = positions of a TD x TH x 32 box of the row grid
//      k       = (tap, source channel), walked in 8-channel groups
//      columns = destination channels (or (tap, Cout) for ConvTranspose fwd)
//    Modes: K3 / K1 (Conv3d fwd and dX), T2DX (ConvTranspose dX), T2FWD
//    (ConvTranspose fwd, scatter epilogue).
//
//  * weight-gradient kernel (r3c_wgrad.h): C[f][(tap, g)] = sum_pos F[pos][f] G[pos (+) tap][g]
//      K = positions (the huge N*D*H*W axis), split deterministically into
//      `nsplit` contiguous box ranges; every split writes fp32 partials that a
//      second kernel sums in a fixed order.
//    Modes: K3 / K1 (Conv3d dW: F = dY, G = x) and T2DW (ConvTranspose dW:
//    F = x, G = dY at 2p + tap).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace r3c {

enum Mode { MODE_K1 = 0, MODE_K3 = 1, MODE_T2DX = 2, MODE_T2FWD = 3, MODE_T2DW = 4 };

struct RowArgs {
  const uint16_t* src;   // x (fwd) or dy (dX)
  const uint16_t* wpk;   // packed fragments [chunk][step][colblock][lane][8]
  const uint16_t* bias;  // may be null
  uint16_t* dst;
  int64_t ss[5];         // source strides (n, c, d, h, w)
  int64_t sd[5];         // destination strides (n, c, d, h, w)
  uint32_t src_bytes;    // bytes of one source sample reachable from its base (buffer range)
  uint32_t dst_bytes;    // the same for one destination sample (k=3 tap kernel stores)
  int32_t Cs, Sd, Sh, Sw;  // source channels and spatial dims
  int32_t Rd, Rh, Rw;      // row grid (destination grid; source grid for T2FWD)
  int32_t pd, ph, pw;      // Conv3d padding (K1/K3)
  int32_t TD, TH;          // box = TD x TH x 32 rows of the row grid
  int32_t nbd, nbh, nbw;   // boxes per dimension
  int32_t n_ctiles;        // column tiles of NB blocks
  int32_t nbt_pad;         // column blocks in the packed weight (n_ctiles * NB)
  int32_t nchunks;         // source-channel chunks of CK
  int32_t ncols;           // real columns (Cd, or 8 * Cout for T2FWD)
  int32_t cout_t2;         // T2FWD: Cout, to split a column into (tap, channel)
  int32_t HD, HH;          // LDS tile dims (the w extent is fixed per mode)
  int32_t CGS;             // 16-byte slots per channel-group plane (HD*HH*HW rounded up to 16)
  int32_t wfull;           // 1: every chunk's weights stay resident in LDS
  int32_t nbuf;            // 2: double-buffered stages; 1: single buffers, two barriers per stage
  int32_t src_cl;          // 1: channel-contiguous 16-byte source loads are legal
  int32_t njobs;           // (box, column tile, split) jobs; workgroups take contiguous ranges
  int32_t nsplit, cps;     // K splits per output tile and chunks per split (nchunks = nsplit * cps)
  float* part;             // nsplit > 1: fp32 partial tiles [tile][split][wave][MB*NB*16][64]
  int32_t ntiles;          // output tiles (box, column tile)
  int32_t off32;           // 1: epilogue per-lane offsets (columns x c-stride + 32 x w-stride) fit in int32
  int32_t t2kw;            // T2FWD: 1 = columns ((kd, kh), co, kw) with kw fastest (w-contiguous output),
                           //        0 = columns (tap, co)
  int32_t phase;           // 0: main pass; 1: split-K epilogue pass, one workgroup per tile
  int32_t chan_outer;      // 1: src_bytes ends at channel Cs (channel planes outermost in a sample),
                           //    so loads of channels past Cs fall out of range by themselves
  // A channel concatenation [A, B] without a copy (k=3 tap kernel, NCDHW): source
  // channels >= csplit are channels - csplit of src2, destination channels
  // >= dsplit go to dst2 (0: one tensor).  Channel and spatial strides are
  // those of ss / sd; src2 / dst2 have their own sample stride and range.
  const uint16_t* src2;
  uint16_t* dst2;
  int64_t ss0_2, sd0_2;
  uint32_t src2_bytes, dst2_bytes;
  int32_t csplit, dsplit;
};

// Weight-gradient box geometry, fixed per mode: TD x TH lines of 16
// positions along w (the K block of one staging round), and the G tile = the
// box plus its tap halo.  Both LDS tiles are [position][32 channels].
template <int MODE>
struct WgGeom {
  static constexpr int TAPS = MODE == MODE_K3 ? 27 : (MODE == MODE_T2DW ? 8 : 1);
  static constexpr int TD = MODE == MODE_T2DW ? 2 : 4;
  static constexpr int TH = MODE == MODE_T2DW ? 2 : 4;
  static constexpr int HD = MODE == MODE_K3 ? TD + 2 : (MODE == MODE_T2DW ? 2 * TD : TD);
  static constexpr int HH = MODE == MODE_K3 ? TH + 2 : (MODE == MODE_T2DW ? 2 * TH : TH);
  static constexpr int HW = MODE == MODE_K3 ? 18 : (MODE == MODE_T2DW ? 32 : 16);
  static constexpr int LINES = TD * TH;
  static constexpr int BOXPOS = LINES * 16;
  static constexpr int HPOS = HD * HH * HW;
  static constexpr int THREADS = 512;                                 // 8 waves
  static constexpr int NFI = (BOXPOS * 4 + THREADS - 1) / THREADS;   // F staging items (16 bytes) per thread
  // F tile: [position][32 channels], or [32 channels][FP positions] when F is
  // staged channel-major (w-contiguous source); FT halves either way.
  static constexpr int FP = BOXPOS + 8;
  static constexpr int FT = BOXPOS * 32 > 32 * FP ? BOXPOS * 32 : 32 * FP;
  static constexpr int NGI = (HPOS * 4 + THREADS - 1) / THREADS;     // G staging items per thread at GCW = 32
  // G tile: [position][32 channels], or (k=1 without padding, no tap shift)
  // channel-major [32 channels][FP positions] like F.
  static constexpr int GT = HPOS * 32 > 32 * FP ? HPOS * 32 : 32 * FP;
  static constexpr int LDS_BYTES = 2 * (FT + GT) * 2;                 // double-buffered tiles
  static constexpr int TRASH_BYTES = THREADS * 16;                    // k=3 NCDHW G staging: one slot per thread
};

// Geometry of the row-walking k=3 weight-gradient kernel (r3c_wgrow.h): rows
// of W = 16 WL positions padded by 8 zero halves (pitch P); a step covers
// RS = min(16 / WL, 8) output rows (16 MFMA k-steps for W >= 32); x rows sit in a
// ring of NSLOT = 2 RS + 2 slots of 3 x GCW rows, dY in two buffers of
// RS x 32 rows.
template <int GCW, int WL>
struct WrGeom {
  static constexpr int W = 16 * WL, P = W + 8;
  static constexpr int RS = 16 / WL < 8 ? 16 / WL : 8;
  static constexpr int NSLOT = 2 * RS + 2;
  static constexpr int NCOL = 9 * GCW;
  static constexpr int NTRIP = (NCOL + 31) / 32;
  static constexpr int RING_HALVES = NSLOT * 3 * GCW * P;
  static constexpr int FBUF_HALVES = RS * 32 * P;
  static constexpr int THREADS = 512;
  static constexpr int NFS = RS * 32 * (W / 8);        // dY staging items per step
  static constexpr int NFI = (NFS + THREADS - 1) / THREADS;
  static constexpr int NGS = RS * 3 * GCW * (W / 8);   // x staging items per step (RS rows of 3 planes)
  static constexpr int NGI = (NGS + THREADS - 1) / THREADS;
  static constexpr int LDS_BYTES = (RING_HALVES + 8 + 2 * FBUF_HALVES) * 2;
  static_assert(NTRIP <= 7, "one wave per block and a free wave for the bias");
  static_assert(16 % WL == 0, "rows per step");
};

struct WgArgs {
  const uint16_t* fsrc;  // F operand tensor (dY for Conv3d, x for ConvTranspose)
  const uint16_t* gsrc;  // G operand tensor (x for Conv3d, dY for ConvTranspose)
  float* part;           // [nsplit][Fpad][TAPS][Gpad] fp32 partials
  float* dbpart;         // [nsplit][Fpad] (db from F) or [nsplit][TAPS][Gpad] (db from G)
  int64_t fs[5], gs[5];
  uint32_t f_bytes, g_bytes;  // per-sample buffer ranges
  int32_t Fc, Gc;          // channel counts
  int32_t Rd, Rh, Rw;      // F (row) grid
  int32_t Gd, Gh, Gw;      // G grid
  int32_t pd, ph, pw;      // Conv3d padding
  int32_t nbd, nbh, nbw, nbox;  // boxes (WgGeom) per dimension and in total
  int32_t nsplit;
  int32_t n_ftiles, n_gtiles;
  int32_t GCW;             // G channels per tile (multiple of 8, at most 32)
  int32_t Fpad, Gpad;
  int32_t db_mode;         // 0 none, 1 db = sum over F, 2 db = sum over G
  int32_t nblocks;
  // G over a channel concatenation [A, B] (row-walking kernel): G channels
  // >= gsplit are channels - gsplit of gsrc2 (0: one tensor); G tiles do not
  // straddle gsplit.
  const uint16_t* gsrc2;
  int64_t gs0_2;
  uint32_t g2_bytes;
  int32_t gsplit;
};

// Register-direct weight gradient of the single-tap passes (Conv3d k=1
// unpadded, ConvTranspose k2s2) on w-contiguous dense operands: r3c_pwdw.h.
struct PwdwArgs {
  const uint16_t* fsrc;   // F rows: dY (k=1) or x (ConvTranspose), [N][Fc][S] planes dense
  const uint16_t* gsrc;   // G columns: x (k=1) or dY (ConvTranspose, grid 2D x 2H x 2W)
  float* part;            // [nsplit][Fc][taps][Gc] fp32 partials
  float* dbpart;          // db_mode 1: [nsplit][Fc]; 2: [nsplit][8][Gc]
  int64_t fs0, fs1;       // F sample / channel strides (elements)
  int64_t gs0, gs1;       // G sample / channel strides
  uint32_t f_bytes, g_bytes;  // per-sample buffer ranges
  int32_t Fc, Gc, taps;
  int32_t S;              // F-grid positions per sample
  int32_t W, HW;          // ConvTranspose: F-grid w extent and h*w extent
  int32_t M, ncols;       // GEMM rows (Fc, +1 ones row for db_mode 2), columns (taps*Gc, +1 ones column for db_mode 1)
  int32_t ngr, ngc;       // tile groups along rows / columns
  int32_t nkb;            // K blocks (16 NJ positions) over N * S
  int32_t nsplit;         // K splits (workgroups per tile group)
  int32_t db_mode;        // 0 none, 1 db = row sums of F, 2 db = column sums of G
  int32_t kil;            // 1: K blocks interleaved over the splits; 0: contiguous range per split
};

// Register-direct ConvTranspose k2s2 dX on a w-contiguous dY and a dX with
// dense planes: r3c_t2dx.h.
struct T2dxArgs {
  const uint16_t* dy;
  const uint16_t* apk;    // A fragments [row group][RB][nks][64 lanes][8]
  uint16_t* dx;
  int64_t ys0, ys1;       // dY sample / channel strides (elements)
  int32_t ys2, ys3;       // dY d / h strides (the w stride is 1)
  int64_t xs0, xs1;       // dX sample / channel strides (planes dense)
  uint32_t dy_bytes, dx_bytes;  // per-sample buffer ranges
  int32_t Cin, Cout;
  int32_t nks;            // k-steps of 16 over k = 8 Cout
  int32_t S, W, HW;       // dX positions per sample; its w and h*w extents
  int32_t ncb;            // column blocks of 32 positions over N * S
  int32_t nrg, ncw;       // row groups; workgroups per row group
};

struct T2dxPackArgs {
  const uint16_t* w;      // ConvTranspose weight (Cin, Cout, 2, 2, 2)
  uint16_t* out;
  int32_t cin, cout, nks, total;
};

struct ReduceArgs {
  const float* part;
  const float* dbpart;
  void* dw;
  void* db;
  int32_t nsplit, Fc, Gc, taps, Fpad, Gpad;
  int32_t dw_dtype, db_dtype;
  int32_t db_mode;        // 0 none, 1 from F partials, 2 from G partials
};


struct PackArgs {
  const uint16_t* w;
  uint16_t* out;
  int32_t mode;           // MODE_K1 / MODE_K3 fwd, +16: Conv3d dX, MODE_T2DX, MODE_T2FWD
  int32_t cs;             // source channels (k dimension)
  int32_t ncols;          // real columns
  int32_t taps;           // taps in k (27, 8 or 1)
  int32_t ck;             // channels per chunk
  int32_t nchunks, nstep, nbt_pad;
  int32_t w_cin, w_cout;  // parameter dims of the weight tensor
  int64_t total;
  int32_t t2kw;           // T2FWD column order, as RowArgs::t2kw
};

// NCDHW -> NDHWC copy of a fully contiguous tensor (C % 8 == 0, S % 8 == 0,
// both pointers 16-byte aligned): dst[n][s][c] = src[n][c][s], s = (d, h, w).
struct LayoutArgs {
  const uint16_t* src;
  uint16_t* dst;
  int64_t S;     // positions per channel plane
  int32_t C, N;
};

// BatchNorm3d + ReLU on NCDHW planes (r3c_bn.hip).  Positions of a
// (sample, channel) plane are contiguous; chunks of kBnChunk positions are the
// unit of work and of the fixed-order partial sums.
constexpr int kBnChunk = 8192;
struct BnArgs {
  const void* y;          // BN input
  const void* dz;         // backward: gradient of the BN + ReLU output
  void* out;              // forward: z; backward: dy
  int64_t sn, sc;         // y sample / channel strides (elements)
  int64_t gn, gc;         // dz strides
  int64_t on, oc;         // out strides
  int64_t S;              // positions per plane
  int32_t N, C, nchunk, training;
  float eps, momentum;
  const float* gamma;     // may be null (no affine)
  const float* beta;
  float* running_mean;    // may be null (no running statistics)
  float* running_var;
  float* save_mean;       // [C] batch (or running) mean and invstd, written by the forward
  float* save_invstd;
  float* dgamma;          // backward outputs, may be null
  float* dbeta;
  float* part;            // [N * nchunk][C][2] partial results (workspace)
  float* coef;            // [C][4] per-channel coefficients (workspace)
};

// MaxPool3d(2, stride 2) on NCDHW planes (r3c_pool.hip).  Even d, h, w with
// w % 8 == 0: every input element belongs to exactly one window.
// k=1 Conv3d with at most 4 output channels on dense NCDHW planes (r3c_skinny.hip).
constexpr int kSkinnyMaxC = 64;  // input channels (weights staged in LDS)
struct SkinnyArgs {
  uint16_t* x;           // x (fwd, dW) or dx (dX): [n][C][P]
  uint16_t* y;           // y (fwd) or dy (dX, dW): [n][O][P]
  const uint16_t* w;     // [O][C]
  const uint16_t* b;     // [O] or null (fwd)
  float* part;           // dW: [nsplit][O][C] partial sums
  float* dbpart;         // dW: [nsplit][O] or null
  int64_t xs0, xs1, ys0, ys1;  // sample / channel strides (elements)
  int64_t P;             // positions per plane (multiple of 8)
  int64_t ngroups;       // n * P / 8
  int32_t C, O, nsplit;
};

// Conv3d k=3 with one input channel (a volume's first layer): forward and
// dW + db as dedicated kernels (r3c_stem.hip).  A job is one output plane's
// block of kStemRows consecutive output rows; its workgroup stages the 3 x
// (kStemRows + 2) input rows those rows read into LDS, each row at element
// offset 8 of a zero-padded pitch.
constexpr int kStemRows = 4;                       // output rows per job (one wave each)
constexpr int kStemXRows = 3 * (kStemRows + 2);    // staged input rows per job
constexpr int kStemMaxW = 512;                     // widest input row
constexpr int kStemMaxCout = 64;                   // output channels (two 32-wide blocks)
struct StemArgs {
  const uint16_t* x;     // [n][1][D][H][W], w contiguous, rows 16-byte aligned
  const uint16_t* w;     // [Cout][27] (OIDHW with one input channel)
  const uint16_t* b;     // fwd: [Cout] or null
  uint16_t* y;           // fwd: output
  const uint16_t* dy;    // dW: output gradient, ow contiguous, rows 16-byte aligned
  float* part;           // dW: [nsplit][Cout][27] partial sums
  float* dbpart;         // dW: [nsplit][Cout] or null
  int64_t xs0, xs2, xs3;              // x strides (n, d, h) in elements
  int64_t ys0, ys1, ys2, ys3, ys4;    // y / dy strides (n, c, d, h, w)
  int32_t D, H, W, OD, OH, OW, pd, ph, pw;
  int32_t Cout;
  int32_t P;             // LDS row pitch (elements, multiple of 8)
  int32_t nrb;           // row blocks per output plane
  int32_t njobs;         // n * OD * nrb
  int32_t nsplit;        // dW: workgroups (one partial each)
  int32_t yvec4;         // fwd: 1 = channels contiguous, 4 channels per 8-byte store
  int32_t yvec8;         // fwd: 1 = positions contiguous and 16-byte aligned rows, OW % 8 == 0:
                         //      8 positions per 16-byte store (through LDS)
};

// Conv3d with stride > 1 (r3c_strided.hip).  Forward: source x, destination
// y; dX: source dY, destination dX, tiles over residue classes of w.
struct StridedArgs {
  const uint16_t* src;
  const uint16_t* wpk;   // [nc16][taps][nbt][64][8]
  const uint16_t* b;     // forward bias or null
  uint16_t* dst;
  int64_t ss[5];         // source strides (n, c, d, h, w)
  int64_t sd5[5];        // destination strides
  int32_t Cs, Cd;        // source (K) channels, destination channels
  int32_t Sd, Sh, Sw;    // source spatial dims
  int32_t Rd, Rh, Rw;    // destination spatial dims
  int32_t k, taps;
  int32_t pd, ph, pw;    // padding
  int32_t sd, sh, sw;    // stride
  int32_t dx;            // 0 forward, 1 dX
  int32_t nc16, nbt, n_ctiles;
  int32_t nwb;           // 32-position blocks along w per row (dX: per residue class)
  int32_t scl;           // 1: source channel-contiguous, 16-byte aligned, Cs % 8 == 0
  int32_t dvec4;         // 1: destination channel-contiguous, Cd % 4 == 0, 8-byte aligned
  int32_t mb;            // blocks of 32 destination positions per wave (1, or 2 with scl)
  int32_t chan_first;    // row-segment forward on an NCDHW source: its 8-channel groups (1 .. 4), else 0
  int32_t dtile;         // 1: forward, one column tile, destination channel-contiguous with positions Cd
                         // apart, Cd % 8 == 0, 16-byte aligned: a tile is one contiguous run, stored
                         // through LDS as 16-byte chunks
  int64_t ntiles;        // wave tiles
};
struct StridedPackArgs {
  const uint16_t* w;     // OIDHW [cout][cin][taps]
  uint16_t* out;
  int32_t cin, cout, taps, nbt, dx;
  int64_t total;         // fragments (16 bytes each)
};
// Direct strided dW (stride along w 1 or 2): workgroup (split, channel-block
// pair) of 9 waves, wave = (kd, kh) with the 3 kw taps; K blocks of 16 output
// positions of one row.
struct StridedDwArgs {
  const uint16_t* x;     // [n][Cin][D][H][W], w contiguous
  const uint16_t* dy;    // [n][Cout][OD][OH][OW], ow contiguous
  float* part;           // [nsplit][Cout][27][Cin]
  float* dbpart;         // [nsplit][Cout] or null
  int64_t xs0, xs1, xs2, xs3;   // x strides (n, c, d, h)
  int64_t ys0, ys1, ys2, ys3;   // dY strides (n, c, d, h)
  int32_t Cin, Cout, D, H, W, OD, OH, OW;
  int32_t pd, ph, pw, sd, sh;   // padding; d / h stride (w stride is the template's)
  int32_t ncg, ngb;      // Cout groups (NCB blocks of 32), Cin blocks of 32; tile = Cout group * ngb + Cin block
  int64_t nkb;           // K blocks: n * OD * OH * (OW / 16)
  int32_t nsplit;
};
struct DilateArgs {
  const uint16_t* src;   // strided dY, any strides
  uint16_t* dst;         // NCDHW [n][C][D1][H1][W1p], 16-byte aligned
  int64_t ys[5];
  int32_t C, D1, H1, W1, W1p, sd, sh, sw;  // W1p: row pitch, a multiple of 8 >= W1
  int64_t rows;          // n * C * D1 * H1
};

struct PoolArgs {
  const void* x;          // forward input
  void* y;                // forward output
  const void* dy;         // backward: gradient of y
  void* dx;               // backward: gradient of x (every element written)
  uint8_t* idx;           // [n][c][od][oh][ow]: kd * 4 + kh * 2 + kw of the window maximum
  const void* add;        // backward: null, or a tensor shaped like x added to dx (may be dx itself)
  int64_t as0, as1;       // its sample and channel strides (planes dense)
  int64_t xs0, xs1;       // x / dx sample and channel strides (elements; planes dense)
  int64_t ys0, ys1;       // y / dy sample and channel strides
  int32_t n, c, d, h, w, od, oh, ow;
};

// Host launchers (return false when no instantiation matches).
// `cus`: compute units of the device; the grid is cus x resident workgroups per CU.
bool launch_row(int dtype, int mode, int nb, int cl, int wf, const RowArgs& a, int cus, size_t lds_bytes,
                hipStream_t stream);
// cl: G (and, with fl 0, F) staged by 16-byte channel vectors; fl 1: F staged
// channel-major from a w-contiguous source; fl 2 (k=1, no padding): F and G both.
bool launch_wgrad(int dtype, int mode, int cbw, int cl, int fl, const WgArgs& a, size_t lds_bytes, hipStream_t stream);
void launch_pack(int dtype, const PackArgs& a, hipStream_t stream);
void launch_to_channels_last(const LayoutArgs& a, hipStream_t stream);
void launch_to_channels_first(const LayoutArgs& a, hipStream_t stream);  // NDHWC -> NCDHW
// One launch: a thread per element (few splits) or a fixed-shape tree over the splits.
void launch_wgrad_reduce(const ReduceArgs& a, hipStream_t stream);
// Row-walking k=3 weight gradient (r3c_wgrow.h); false if no instantiation for (gcw, W).
bool launch_wgrow(int dtype, int gcw, int w, const WgArgs& a, hipStream_t stream);
// Register-direct single-tap weight gradient (mode MODE_K1 with nj 4, or
// MODE_T2DW with nj 1 / 2); false if no instantiation matches.
bool launch_pwdw(int dtype, int mode, int tr, int tc, int nj, const PwdwArgs& a, hipStream_t stream);
// Register-direct ConvTranspose dX (rb 1 or 2 row blocks per workgroup).
bool launch_t2dx(int dtype, int rb, const T2dxArgs& a, size_t lds, hipStream_t stream);
void launch_t2dx_pack(const T2dxPackArgs& a, hipStream_t stream);
// BatchNorm + ReLU: forward (statistics or running statistics, then z) and
// backward (sums, then dy); dtype 0 fp16, 1 bf16, 2 fp32 (the C ABI's codes).
void launch_bn_relu_fwd(int dtype, const BnArgs& a, hipStream_t stream);
void launch_bn_relu_bwd(int dtype, const BnArgs& a, hipStream_t stream);
// MaxPool3d(2): forward (y, idx) and backward (dx); dtype as the C ABI's codes.
// MFMA shape probe (r3c_probe.hip): shape 0 32x32x16, 1 16x16x32 (bf16).
void launch_mfma_probe(int shape, int blocks, int iters, float* out, hipStream_t stream);
// pass 0 fwd, 1 dX, 2 dW partials; false if O is not 1..4.
bool launch_skinny(int dtype, int pass, const SkinnyArgs& a, hipStream_t stream);
// pass 0 = forward, 2 = dW + db; false when Cout has no instantiation.
bool launch_stem(int dtype, int pass, const StemArgs& a, size_t lds, hipStream_t stream);
// Strided Conv3d: weight pack, forward / dX kernel (nb column blocks per wave
// tile, 1..4), and the dY scatter onto the stride-1 grid for dW.
void launch_strided_pack(const StridedPackArgs& a, hipStream_t stream);
bool launch_strided(int dtype, int nb, const StridedArgs& a, hipStream_t stream);
// Forward, k = 3, w stride 1 or 2, channel-contiguous source with at most 32 channels, nb <= 2:
// the x operand through per-wave LDS row segments.
bool launch_strided_fwd_rs(int dtype, int nb, const StridedArgs& a, hipStream_t stream);
// dX, k = 3, w stride 1 or 2, channel-contiguous dY with at most 64 channels, nb <= 2: the dY
// operand through per-wave LDS row segments.
bool launch_strided_dx_rs(int dtype, int nb, const StridedArgs& a, hipStream_t stream);
void launch_dilate(const DilateArgs& a, hipStream_t stream);
// Direct strided dW + db (sw 1 or 2); false for other w strides.
bool launch_strided_dw(int dtype, int sw, int ncb, const StridedDwArgs& a, hipStream_t stream);  // ncb: Cout blocks per wave (1, 2)
void launch_maxpool2_fwd(int dtype, const PoolArgs& a, hipStream_t stream);
void launch_maxpool2_bwd(int dtype, const PoolArgs& a, hipStream_t stream);

}  // namespace r3c
