// r3c_capi.hip -- the extern "C" boundary: argument validation, tile planning
// and kernel launches.  Every entry point is asynchronous on the caller's
// stream and allocates nothing (the caller passes the workspace it sized with
// the matching *_workspace query).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <initializer_list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "r3c_kernels.h"
#include "rdna4_conv3d.h"

namespace r3c {

#define R3C_DECL_ROW(m)                                                                       \
  bool launch_row_##m##_bf16(int nb, int cl, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s); \
  bool launch_row_##m##_f16(int nb, int cl, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s);
R3C_DECL_ROW(k1)
R3C_DECL_ROW(t2dx)
R3C_DECL_ROW(t2fwd)
#undef R3C_DECL_ROW
#define R3C_DECL_TAP(t)                                                                                     \
  bool launch_tap_##t(int nb, int mb, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s);
R3C_DECL_TAP(bf16_w32_s0)
R3C_DECL_TAP(bf16_w32_s1)
R3C_DECL_TAP(bf16_w16_s0)
R3C_DECL_TAP(bf16_w16_s1)
R3C_DECL_TAP(f16_w32_s0)
R3C_DECL_TAP(f16_w32_s1)
R3C_DECL_TAP(f16_w16_s0)
R3C_DECL_TAP(f16_w16_s1)
R3C_DECL_TAP(bf16_w32_s3)
R3C_DECL_TAP(bf16_w16_s3)
R3C_DECL_TAP(f16_w32_s3)
R3C_DECL_TAP(f16_w16_s3)
#undef R3C_DECL_TAP

bool launch_tap(int dtype, int nb, int mb, int src, int wf, int lw, const RowArgs& a, int cus, size_t lds,
                hipStream_t s) {
  const bool bf = dtype == R3C_BF16;
  if (src == 3) {
    if (lw == 32) return bf ? launch_tap_bf16_w32_s3(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w32_s3(nb, mb, wf, a, cus, lds, s);
    return bf ? launch_tap_bf16_w16_s3(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w16_s3(nb, mb, wf, a, cus, lds, s);
  }
  if (lw == 32) {
    if (src == 1) return bf ? launch_tap_bf16_w32_s1(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w32_s1(nb, mb, wf, a, cus, lds, s);
    return bf ? launch_tap_bf16_w32_s0(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w32_s0(nb, mb, wf, a, cus, lds, s);
  }
  if (src == 1) return bf ? launch_tap_bf16_w16_s1(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w16_s1(nb, mb, wf, a, cus, lds, s);
  return bf ? launch_tap_bf16_w16_s0(nb, mb, wf, a, cus, lds, s) : launch_tap_f16_w16_s0(nb, mb, wf, a, cus, lds, s);
}

#define R3C_DECL_WG(m)                                                                    \
  bool launch_wgrad_##m##_bf16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s); \
  bool launch_wgrad_##m##_f16(int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s);
R3C_DECL_WG(k3)
R3C_DECL_WG(k1)
R3C_DECL_WG(t2dw)
#undef R3C_DECL_WG

bool launch_row(int dtype, int mode, int nb, int cl, int wf, const RowArgs& a, int cus, size_t lds, hipStream_t s) {
  const bool bf = dtype == R3C_BF16;
  switch (mode) {
    case MODE_K1:
      return bf ? launch_row_k1_bf16(nb, cl, wf, a, cus, lds, s) : launch_row_k1_f16(nb, cl, wf, a, cus, lds, s);
    case MODE_T2DX:
      return bf ? launch_row_t2dx_bf16(nb, cl, wf, a, cus, lds, s) : launch_row_t2dx_f16(nb, cl, wf, a, cus, lds, s);
    case MODE_T2FWD:
      return bf ? launch_row_t2fwd_bf16(nb, cl, wf, a, cus, lds, s)
                : launch_row_t2fwd_f16(nb, cl, wf, a, cus, lds, s);
    default: return false;
  }
}

bool launch_wgrad(int dtype, int mode, int cbw, int cl, int fl, const WgArgs& a, size_t lds, hipStream_t s) {
  const bool bf = dtype == R3C_BF16;
  switch (mode) {
    case MODE_K3:
      return bf ? launch_wgrad_k3_bf16(cbw, cl, fl, a, lds, s) : launch_wgrad_k3_f16(cbw, cl, fl, a, lds, s);
    case MODE_K1:
      return bf ? launch_wgrad_k1_bf16(cbw, cl, fl, a, lds, s) : launch_wgrad_k1_f16(cbw, cl, fl, a, lds, s);
    case MODE_T2DW:
      return bf ? launch_wgrad_t2dw_bf16(cbw, cl, fl, a, lds, s) : launch_wgrad_t2dw_f16(cbw, cl, fl, a, lds, s);
    default: return false;
  }
}

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return R3C_OK;
}

// ---------------------------------------------------------------------------
// Kernel timing hook (measurement only).  While enabled, each kernel launch is
// bracketed by a pair of HIP events on its own launch stream, tagged with the
// caller's current tag and the kernel family; collect() waits for them and
// returns the per-launch durations.
// ---------------------------------------------------------------------------
enum KernelKind {
  KIND_PACK = 0, KIND_ROW = 1, KIND_WGRAD = 2, KIND_REDUCE = 3, KIND_LAYOUT = 4, KIND_SPLIT_EPI = 5, KIND_BN = 6,
  KIND_POOL = 7
};

struct TimingRec {
  int tag, kind;
  hipEvent_t e0, e1;
};

struct TimingState {
  std::mutex mu;
  bool on = false;
  int filter_tag = -1, filter_kind = -1;  // record only matching launches (-1 = any)
  std::vector<TimingRec> recs;
  std::vector<hipEvent_t> pool;
};

TimingState& timing() {
  static TimingState* st = new TimingState();  // lives for the process
  return *st;
}

thread_local int g_tag = 0;

hipEvent_t pool_event(TimingState& st) {
  if (!st.pool.empty()) {
    hipEvent_t e = st.pool.back();
    st.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

struct TimedLaunch {
  TimingState& st;
  hipStream_t s;
  int kind;
  hipEvent_t e0 = nullptr;
  bool active = false;
  TimedLaunch(int k, hipStream_t stream) : st(timing()), s(stream), kind(k) {
    std::lock_guard<std::mutex> lk(st.mu);
    if (!st.on) return;
    if ((st.filter_tag >= 0 && st.filter_tag != g_tag) || (st.filter_kind >= 0 && st.filter_kind != k)) return;
    e0 = pool_event(st);
    if (e0 && hipEventRecord(e0, s) == hipSuccess) active = true;
  }
  void end() {
    if (!active) return;
    std::lock_guard<std::mutex> lk(st.mu);
    hipEvent_t e1 = pool_event(st);
    if (e1 && hipEventRecord(e1, s) == hipSuccess) st.recs.push_back({g_tag, kind, e0, e1});
    active = false;
  }
};

constexpr int64_t kMaxLds = 160 * 1024;
constexpr int64_t kSplitTarget = 512;          // row-kernel jobs to aim for (two workgroups per CU)
constexpr int kNumCUs = 256;                   // MI355X compute units
constexpr int64_t kMaxPartialBytes = 96ll << 20;

// Row-walking k=3 weight gradient on (R3C_WGROW=0 turns it off).
bool wgrow_enabled() {
  static const bool v = [] {
    const char* e = getenv("R3C_WGROW");
    return !(e && e[0] == '0');
  }();
  return v;
}

int64_t align256(int64_t v) { return (v + 255) & ~int64_t(255); }
int cdiv(int64_t a, int64_t b) { return (int)((a + b - 1) / b); }

enum Op { OP_CONV_FWD, OP_CONV_DX, OP_T2_FWD, OP_T2_DX };

// ---------------------------------------------------------------------------
// Descriptor validation
// ---------------------------------------------------------------------------
int check_strides(const int64_t* s, const int32_t* dims, const char* what) {
  for (int i = 0; i < 5; ++i) {
    if (s[i] < 0) return fail(R3C_INVALID, "%s stride[%d] = %lld is negative", what, i, (long long)s[i]);
    if (dims[i] > 1 && s[i] == 0) return fail(R3C_INVALID, "%s stride[%d] is 0 for a dimension of size %d", what, i, dims[i]);
  }
  return R3C_OK;
}

// `st`: Conv3d stride (d, h, w) for the strided entry points; null = 1.
int validate(const r3c_conv_desc* d, bool transpose, const int32_t* st = nullptr) {
  if (!d) return fail(R3C_INVALID, "descriptor is NULL");
  if (d->dtype != R3C_F16 && d->dtype != R3C_BF16)
    return fail(R3C_UNSUPPORTED, "dtype %d is not fp16 or bf16", d->dtype);
  if (d->n < 1 || d->cin < 1 || d->cout < 1 || d->d < 1 || d->h < 1 || d->w < 1 || d->od < 1 || d->oh < 1 ||
      d->ow < 1)
    return fail(R3C_INVALID, "every dimension must be >= 1 (empty tensors are handled by the caller)");
  const int32_t lim = 1 << 15;
  if (d->d >= lim || d->h >= lim || d->w >= lim || d->od >= lim || d->oh >= lim || d->ow >= lim || d->cin > 65535 ||
      d->cout > 65535)
    return fail(R3C_UNSUPPORTED, "dimension too large (spatial < 32768, channels <= 65535)");
  if (transpose) {
    if (d->kernel != 2) return fail(R3C_UNSUPPORTED, "ConvTranspose3d: kernel %d (only k=2, s=2)", d->kernel);
    if (d->pad_d || d->pad_h || d->pad_w) return fail(R3C_UNSUPPORTED, "ConvTranspose3d: padding must be 0");
    if (d->od != 2 * d->d || d->oh != 2 * d->h || d->ow != 2 * d->w)
      return fail(R3C_INVALID, "ConvTranspose3d k2s2: output dims must be twice the input dims");
  } else {
    if (d->kernel != 1 && d->kernel != 3) return fail(R3C_UNSUPPORTED, "Conv3d: kernel %d (only 1 or 3)", d->kernel);
    const int k = d->kernel;
    if (d->pad_d < 0 || d->pad_h < 0 || d->pad_w < 0 || d->pad_d > 64 || d->pad_h > 64 || d->pad_w > 64)
      return fail(R3C_UNSUPPORTED, "Conv3d: padding must be in [0, 64]");
    const int32_t s1[3] = {1, 1, 1};
    const int32_t* s = st ? st : s1;
    for (int i = 0; i < 3; ++i)
      if (s[i] < 1 || s[i] > 8) return fail(R3C_UNSUPPORTED, "Conv3d: stride %d (only 1 .. 8)", s[i]);
    const int32_t in[3] = {d->d, d->h, d->w}, pad[3] = {d->pad_d, d->pad_h, d->pad_w}, out[3] = {d->od, d->oh, d->ow};
    for (int i = 0; i < 3; ++i)
      if (in[i] + 2 * pad[i] < k || out[i] != (in[i] + 2 * pad[i] - k) / s[i] + 1)
        return fail(R3C_INVALID, "Conv3d: output dims do not match (input + 2*pad - k) / stride + 1");
  }
  const int32_t xd[5] = {d->n, d->cin, d->d, d->h, d->w};
  const int32_t yd[5] = {d->n, d->cout, d->od, d->oh, d->ow};
  int rc = check_strides(d->x_strides, xd, "x");
  if (rc) return rc;
  return check_strides(d->y_strides, yd, "y");
}

// Compute units of the current device (set by check_device, per thread).
thread_local int t_cus = kNumCUs;

int check_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(R3C_HIP_ERROR, "hipGetDevice failed");
  if (!r3c_device_supported(dev)) return fail(R3C_UNSUPPORTED, "device %d is not gfx950", dev);
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1)
    cus = kNumCUs;
  t_cus = cus;
  return R3C_OK;
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(R3C_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

bool vec16_ok(const void* p, const int64_t* s) {
  if (s[1] != 1) return false;
  if ((reinterpret_cast<uintptr_t>(p) & 15) != 0) return false;
  return (s[0] % 8 == 0) && (s[2] % 8 == 0) && (s[3] % 8 == 0) && (s[4] % 8 == 0);
}

// A fully contiguous NCDHW tensor that the NDHWC copy kernel accepts.
bool ncdhw_copyable(const int64_t* st, int c, int d, int h, int w) {
  const int64_t S = (int64_t)d * h * w;
  return c % 8 == 0 && S % 8 == 0 && st[4] == 1 && st[3] == w && st[2] == (int64_t)h * w && st[1] == S &&
         st[0] == (int64_t)c * S;
}

// Dense NDHWC (channels_last_3d) with C and D H W multiples of 8: the layout
// the NCDHW copy (to_channels_first_kernel) reads.
bool ndhwc_copyable(const int64_t* st, int c, int d, int h, int w) {
  const int64_t S = (int64_t)d * h * w;
  return c % 8 == 0 && S % 8 == 0 && st[1] == 1 && st[4] == c && st[3] == (int64_t)w * c &&
         st[2] == (int64_t)h * w * c && st[0] == S * c;
}

// Element strides (n, c, d, h, w) of the dense NCDHW copy.
void channels_first_strides(int64_t* st, int c, int d, int h, int w) {
  st[4] = 1;
  st[3] = w;
  st[2] = (int64_t)h * w;
  st[1] = (int64_t)d * h * w;
  st[0] = (int64_t)c * d * h * w;
}

// Element strides (n, c, d, h, w) of the NDHWC copy.
void channels_last_strides(int64_t* st, int c, int d, int h, int w) {
  st[1] = 1;
  st[4] = c;
  st[3] = (int64_t)w * c;
  st[2] = (int64_t)h * w * c;
  st[0] = (int64_t)d * h * w * c;
}

int64_t tensor_bytes(int n, int c, int d, int h, int w) { return (int64_t)n * c * d * h * w * 2; }

int copy_to_channels_last(const void* src, void* dst, int n, int c, int d, int h, int w, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(src) & 15) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15) != 0)
    return fail(R3C_INVALID, "layout copy needs 16-byte aligned tensors");
  LayoutArgs la;
  la.src = static_cast<const uint16_t*>(src);
  la.dst = static_cast<uint16_t*>(dst);
  la.S = (int64_t)d * h * w;
  la.C = c;
  la.N = n;
  {
    TimedLaunch tl(KIND_LAYOUT, s);
    launch_to_channels_last(la, s);
    tl.end();
  }
  return check_launch("layout copy");
}

int copy_to_channels_first(const void* src, void* dst, int n, int c, int d, int h, int w, hipStream_t s) {
  if ((reinterpret_cast<uintptr_t>(src) & 15) != 0 || (reinterpret_cast<uintptr_t>(dst) & 15) != 0)
    return fail(R3C_INVALID, "layout copy needs 16-byte aligned tensors");
  LayoutArgs la;
  la.src = static_cast<const uint16_t*>(src);
  la.dst = static_cast<uint16_t*>(dst);
  la.S = (int64_t)d * h * w;
  la.C = c;
  la.N = n;
  {
    TimedLaunch tl(KIND_LAYOUT, s);
    launch_to_channels_first(la, s);
    tl.end();
  }
  return check_launch("layout copy to NCDHW");
}

// Bytes of one sample reachable from its base through `strides` (0 if too large
// for 32-bit buffer offsets).
uint32_t sample_bytes(const int64_t* st, int c, int d, int h, int w) {
  const int64_t last = (int64_t)(c - 1) * st[1] + (int64_t)(d - 1) * st[2] + (int64_t)(h - 1) * st[3] +
                       (int64_t)(w - 1) * st[4];
  const int64_t bytes = (last + 8) * 2;  // round up so a 16-byte load at the last element stays in range
  if (bytes >= (int64_t)0x3fffffff) return 0;
  return (uint32_t)bytes;
}

// ---------------------------------------------------------------------------
// Row-kernel plan (Conv3d fwd / dX, ConvTranspose fwd / dX)
// ---------------------------------------------------------------------------
struct RowPlan {
  int mode, ck, nb, cl;
  int tap;             // 1: Conv3d k=3 through the tap kernel (mb, lw below)
  int mb, lw;
  RowArgs a;
  PackArgs pk;
  size_t lds;
  int64_t wpk_bytes;
  int64_t copy_bytes;  // > 0: the source is first copied to NDHWC in the workspace
  int64_t part_bytes;  // split-K partial tiles (0 without split)
  int64_t ntiles;      // output tiles (box, column tile)
};

int pick_blocks(int nbt, const int* opts, int nopt) {
  int best = opts[0], best_waste = 1 << 30;
  for (int i = 0; i < nopt; ++i) {
    const int nb = opts[i];
    const int waste = cdiv(nbt, nb) * nb - nbt;
    if (waste < best_waste || (waste == best_waste && nb > best)) {
      best = nb;
      best_waste = waste;
    }
  }
  return best;
}

// Box of `rows` 32-wide lines: TD x TH = rows, TD in [td_min, td_max], minimising
// the padded, halo'd volume.
void pick_box(int rows, int Rd, int Rh, int halo, int td_min, int td_max, int& TD, int& TH) {
  int64_t best = -1;
  for (int td = td_min; td <= td_max && td <= rows; td *= 2) {
    const int th = rows / td;
    const int64_t cost = (int64_t)cdiv(Rd, td) * cdiv(Rh, th) * (td + halo) * (th + halo);
    if (best < 0 || cost < best || (cost == best && td == th)) {
      best = cost;
      TD = td;
      TH = th;
    }
  }
}

// Weight packing into the kernel's fragment order ([chunk][step][colblock][lane][8]).
void plan_pack(const r3c_conv_desc* d, int op, RowPlan& p, int taps, int nstep) {
  RowArgs& a = p.a;
  PackArgs& pk = p.pk;
  memset(&pk, 0, sizeof pk);
  pk.cs = a.Cs;
  pk.ncols = a.ncols;
  pk.taps = taps;
  pk.ck = p.ck;
  pk.nchunks = a.nchunks;
  pk.nstep = nstep;
  pk.nbt_pad = a.nbt_pad;
  pk.w_cin = d->cin;
  pk.w_cout = d->cout;
  pk.mode = p.mode | (op == OP_CONV_DX ? 16 : 0);
  // ConvTranspose into a w-contiguous output orders its columns kw-fastest so
  // the epilogue can interleave kw pairs into 16-byte stores.
  a.t2kw = (p.mode == MODE_T2FWD && a.sd[4] == 1) ? 1 : 0;
  pk.t2kw = a.t2kw;
  pk.total = (int64_t)a.nchunks * nstep * a.nbt_pad * 64 * 8;
  p.wpk_bytes = pk.total * 2;
}

// Tap-kernel geometry (mirrors TapGeom in r3c_tap.h): TD x TH lines of `lw`
// positions (a line spans 32 / lw h rows), a one-voxel halo on every side.
struct TapBox {
  int TD, TH, HR, HD, HH, HW, HPOS, HPAD;
};
TapBox tap_box(int mb, int lw) {
  TapBox b;
  b.TD = mb == 1 ? 2 : 4;
  b.TH = mb == 4 ? 8 : 4;
  b.HR = 32 / lw;
  b.HD = b.TD + 2;
  b.HH = b.TH * b.HR + 2;
  b.HW = lw + 2;
  b.HPOS = b.HD * b.HH * b.HW;
  b.HPAD = (b.HPOS + 15) / 16 * 16;
  return b;
}
constexpr int64_t kTapScratch = 512 * 16;        // one 16-byte trash slot per thread (NCDHW staging)
constexpr int kTapStep = 14;                      // MFMA steps per 8-channel chunk (27 taps)

// Conv3d k=3 plan on the tap kernel; `a` already holds the source/destination
// geometry, strides, padding and channel counts.
void plan_tap(const r3c_conv_desc* d, RowPlan& p) {
  RowArgs& a = p.a;
  p.tap = 1;
  p.ck = 8;
  p.lw = a.Rw <= 16 ? 16 : 32;
  const int nbt = cdiv(a.ncols, 32);
  static const int opts[] = {3, 2, 1};
  p.nb = pick_blocks(nbt, opts, 3);
  a.n_ctiles = cdiv(nbt, p.nb);
  a.nbt_pad = a.n_ctiles * p.nb;
  a.nchunks = cdiv(a.Cs, 8);
  const int64_t wfrag = (int64_t)kTapStep * p.nb * 64 * 16;  // bytes of one chunk's fragments
  const int64_t fixed = kTapScratch + (int64_t)a.nbt_pad * 32 * 4;
  // Largest row block per wave (MB lines) that still gives every CU a tile
  // and fits the LDS; MB = 4 only for a single column block.
  static const int mbs[] = {4, 2, 1};
  int chosen = -1;
  for (int mb : mbs) {
    if (mb == 4 && p.nb != 1) continue;
    const TapBox b = tap_box(mb, p.lw);
    const int64_t tiles = (int64_t)d->n * cdiv(a.Rd, b.TD) * cdiv(a.Rh, b.TH * b.HR) * cdiv(a.Rw, p.lw) * a.n_ctiles;
    const int64_t lds = fixed + 2 * (int64_t)b.HPAD * 16 + 2 * wfrag;
    if (lds > kMaxLds) continue;
    chosen = mb;
    if (tiles >= kNumCUs) break;
  }
  if (chosen < 0) chosen = 1;
  p.mb = chosen;
  const TapBox b = tap_box(p.mb, p.lw);
  a.TD = b.TD;
  a.TH = b.TH;
  a.HD = b.HD;
  a.HH = b.HH;
  a.CGS = b.HPAD;
  a.nbd = cdiv(a.Rd, b.TD);
  a.nbh = cdiv(a.Rh, b.TH * b.HR);
  a.nbw = cdiv(a.Rw, p.lw);
  const int64_t act = 2 * (int64_t)b.HPAD * 16;
  a.wfull = (p.nb == 1 && a.n_ctiles == 1 && fixed + act + wfrag * a.nchunks <= kMaxLds) ? 1 : 0;
  a.nbuf = 2;
  p.lds = (size_t)(fixed + act + (a.wfull ? wfrag * a.nchunks : 2 * wfrag));
  // Deterministic split K over the source-channel chunks when there are fewer
  // output tiles than CUs: the largest divisor of nchunks with at most one
  // job per CU.
  p.ntiles = (int64_t)d->n * a.nbd * a.nbh * a.nbw * a.n_ctiles;
  int split = 1;
  if (p.ntiles < kNumCUs) {
    const int64_t want = kNumCUs / p.ntiles;
    for (int sp = 2; sp <= a.nchunks && sp <= want; ++sp)
      if (a.nchunks % sp == 0) split = sp;
  }
  a.nsplit = split;
  a.cps = a.nchunks / split;
  p.part_bytes = split > 1 ? align256(p.ntiles * split * 8 * p.mb * p.nb * 16 * 64 * 4) : 0;
}

// allow_copy false: never copy the source to NDHWC (its 16-byte copy kernel
// needs an aligned source).
void plan_row(const r3c_conv_desc* d, int op, RowPlan& p, bool allow_copy = true) {
  RowArgs& a = p.a;
  memset(&a, 0, sizeof a);
  const int k = d->kernel;
  int cs = 0, sc = 0, sdd = 0, sh = 0, sw = 0;
  if (op == OP_CONV_FWD || op == OP_CONV_DX) p.mode = k == 3 ? MODE_K3 : MODE_K1;
  else p.mode = op == OP_T2_FWD ? MODE_T2FWD : MODE_T2DX;
  switch (op) {
    case OP_CONV_FWD:
      cs = d->cin; sdd = d->d; sh = d->h; sw = d->w;
      a.Rd = d->od; a.Rh = d->oh; a.Rw = d->ow;
      a.pd = d->pad_d; a.ph = d->pad_h; a.pw = d->pad_w;
      a.ncols = d->cout;
      memcpy(a.ss, d->x_strides, sizeof a.ss);
      memcpy(a.sd, d->y_strides, sizeof a.sd);
      break;
    case OP_CONV_DX:
      cs = d->cout; sdd = d->od; sh = d->oh; sw = d->ow;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.pd = k - 1 - d->pad_d; a.ph = k - 1 - d->pad_h; a.pw = k - 1 - d->pad_w;
      a.ncols = d->cin;
      memcpy(a.ss, d->y_strides, sizeof a.ss);
      memcpy(a.sd, d->x_strides, sizeof a.sd);
      break;
    case OP_T2_FWD:
      cs = d->cin; sdd = d->d; sh = d->h; sw = d->w;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.ncols = 8 * d->cout;
      a.cout_t2 = d->cout;
      memcpy(a.ss, d->x_strides, sizeof a.ss);
      memcpy(a.sd, d->y_strides, sizeof a.sd);
      break;
    default:  // OP_T2_DX
      cs = d->cout; sdd = d->od; sh = d->oh; sw = d->ow;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.ncols = d->cin;
      memcpy(a.ss, d->y_strides, sizeof a.ss);
      memcpy(a.sd, d->x_strides, sizeof a.sd);
      break;
  }
  (void)sc;
  // An unpadded k=1 pass maps each position to itself, so positions can be
  // walked in any order.  When source and destination both hold each
  // channel's D*H*W positions contiguously (NCDHW), view them as [S/256][8][32]:
  // a box of 8 lines x 32 is then 256 consecutive positions, one 512-byte run
  // per channel, instead of 8 runs of 64 bytes (w = 32 of a wider row).
  if (p.mode == MODE_K1 && a.pd == 0 && a.ph == 0 && a.pw == 0) {
    const int64_t S = (int64_t)sdd * sh * sw;
    const bool dense = a.ss[4] == 1 && a.ss[3] == sw && a.ss[2] == (int64_t)sh * sw && a.sd[4] == 1 &&
                       a.sd[3] == a.Rw && a.sd[2] == (int64_t)a.Rh * a.Rw && a.Rd == sdd && a.Rh == sh &&
                       a.Rw == sw;
    if (dense && S % 256 == 0 && S / 256 < (1ll << 30)) {
      a.Rd = sdd = (int)(S / 256);
      a.Rh = sh = 8;
      a.Rw = sw = 32;
      a.ss[2] = a.sd[2] = 256;
      a.ss[3] = a.sd[3] = 32;
    }
  }
  a.Cs = cs;
  a.Sd = sdd; a.Sh = sh; a.Sw = sw;
  // A low-channel NCDHW source of a k=3 pass is copied to NDHWC first: its
  // channel-contiguous staging is faster than strided staging by more than the
  // copy costs (two bytes read and written per element).
  p.copy_bytes = 0;
  // A w-contiguous k=3 source (NCDHW) is staged by 16-byte loads of 8
  // positions per channel and a register transpose (tap kernel staging mode 3).
  // The channel planes must be outermost in a sample (a plane's positions, up
  // to the end of its last 8-position load, below the channel stride): the
  // kernel's buffer range then ends at channel cs.
  const bool k3_wvec = p.mode == MODE_K3 && a.ss[4] == 1 && a.ss[1] != 1 && sw % 8 == 0 && a.ss[0] % 8 == 0 &&
                       a.ss[1] % 8 == 0 && a.ss[2] % 8 == 0 && a.ss[3] % 8 == 0 && a.pw >= -6 && a.pw <= 8 &&
                       a.ss[2] > 0 && a.ss[3] > 0 &&
                       a.ss[1] >= (int64_t)(sdd - 1) * a.ss[2] + (int64_t)(sh - 1) * a.ss[3] + sw &&
                       2 * (int64_t)(cs + 8) * a.ss[1] < (1ll << 30);  // no 32-bit wrap past the last chunk
  if (allow_copy && !k3_wvec && p.mode == MODE_K3 && cs <= 32 && ncdhw_copyable(a.ss, cs, sdd, sh, sw)) {
    p.copy_bytes = align256(tensor_bytes(d->n, cs, sdd, sh, sw));
    channels_last_strides(a.ss, cs, sdd, sh, sw);
  }
  a.src_bytes = sample_bytes(a.ss, cs, sdd, sh, sw);
  a.dst_bytes = sample_bytes(a.sd, a.ncols, a.Rd, a.Rh, a.Rw);
  // NCDHW k=3 staging: the buffer range ends exactly at channel cs, so loads
  // of the channels past it need no gating.
  a.chan_outer = k3_wvec ? 1 : 0;
  if (k3_wvec) a.src_bytes = (uint32_t)(2 * (int64_t)cs * a.ss[1]);
  // Channel-contiguous sources are staged by direct-to-LDS 16-byte loads;
  // others by 8 scalar loads per slot through registers.
  p.cl = (a.ss[1] == 1 && cs % 8 == 0 && a.ss[0] % 8 == 0 && a.ss[2] % 8 == 0 && a.ss[3] % 8 == 0 &&
          a.ss[4] % 8 == 0) ? 1 : 0;
  // A w-contiguous source of a single-tap pass (k=1 without w padding, or
  // ConvTranspose forward) is staged channel-major by 16-byte loads of 8
  // positions (cl 2) instead of 8 scalar loads per slot.
  if (!p.cl && (p.mode == MODE_T2FWD || (p.mode == MODE_K1 && a.pw == 0)) && a.ss[4] == 1 && sw % 8 == 0 &&
      a.ss[0] % 8 == 0 && a.ss[1] % 8 == 0 && a.ss[2] % 8 == 0 && a.ss[3] % 8 == 0)
    p.cl = 2;
  if (k3_wvec) p.cl = 3;
  p.tap = 0;
  p.mb = 2;
  p.lw = 32;
  if (p.mode == MODE_K3) {
    plan_tap(d, p);
    plan_pack(d, op, p, 27, kTapStep);
    return;
  }
  const int taps_k = p.mode == MODE_K3 ? 27 : (p.mode == MODE_T2DX ? 8 : 1);
  const int g8 = taps_k == 1 ? 4 : 1;  // the kernel's RowGeom::G8
  p.ck = 8 * g8;
  const int nbt = cdiv(a.ncols, 32);
  static const int opts[] = {3, 2, 1};
  static const int opts_t2[] = {6, 3, 2, 1};  // ConvTranspose fwd: one row block per wave
  p.nb = p.mode == MODE_T2FWD ? pick_blocks(nbt, opts_t2, 4) : pick_blocks(nbt, opts, 3);
  const bool mb1 = p.mode == MODE_T2DX || p.mode == MODE_T2FWD;  // the kernel's RowGeom::MB == 1
  const int rows = mb1 ? 4 : 8;  // 4 waves x MB row blocks
  if (p.mode == MODE_K3) pick_box(rows, a.Rd, a.Rh, 2, 2, 4, a.TD, a.TH);
  else pick_box(rows, a.Rd, a.Rh, 0, 1, rows, a.TD, a.TH);
  a.nbd = cdiv(a.Rd, a.TD);
  a.nbh = cdiv(a.Rh, a.TH);
  a.nbw = cdiv(a.Rw, 32);
  a.n_ctiles = cdiv(nbt, p.nb);
  a.nbt_pad = a.n_ctiles * p.nb;
  a.nchunks = cdiv(cs, p.ck);
  int hw;
  if (p.mode == MODE_K3) {
    a.HD = a.TD + 2; a.HH = a.TH + 2; hw = 34;
  } else if (p.mode == MODE_T2DX) {
    a.HD = 2 * a.TD; a.HH = 2 * a.TH; hw = 64;
  } else {
    a.HD = a.TD; a.HH = a.TH; hw = 32;
  }
  const int hpos = a.HD * a.HH * hw;
  a.CGS = (hpos + 15) / 16 * 16;  // 256-byte aligned channel-group planes
  // Channel-major rows: a pitch of 32 (mod 128) halves puts the rows a
  // transposing read touches on distinct banks.
  if (p.cl == 2) a.CGS = (hpos + 127) / 128 * 128 + 32;
  const int taps = taps_k;
  const int nstep = cdiv(taps * g8, 2);
  const int64_t wchunk = (int64_t)nstep * p.nb * 1024;  // bytes of one chunk's fragments
  // Buffering options in order of preference; take the first that leaves room
  // for two workgroups per CU (8 waves), else the one with the most room.
  //   wfull: every chunk's weights resident (only with a single column tile)
  //   nbuf 2: double-buffered stages, one barrier per stage; 1: two barriers
  const int64_t fixed = 4 * 2048 + (int64_t)a.nbt_pad * 32 * 4 + 16;
  const int64_t act1 = (int64_t)g8 * a.CGS * 16;
  struct Opt { int wfull, nbuf; };
  static const Opt opts2[] = {{1, 2}, {0, 2}, {1, 1}, {0, 1}};
  int best = -1;
  int64_t best_lds = 0;
  for (const Opt& o : opts2) {
    if (o.wfull && a.n_ctiles != 1) continue;
    const int64_t l = fixed + o.nbuf * act1 + (o.wfull ? wchunk * a.nchunks : o.nbuf * wchunk);
    if (l > kMaxLds) continue;
    if (best < 0 || kMaxLds / l > kMaxLds / best_lds) {
      best = (int)(&o - opts2);
      best_lds = l;
    }
    if (kMaxLds / l >= 2) break;
  }
  if (best < 0) best = 3, best_lds = fixed + act1 + wchunk;  // rejected by the LDS check
  a.wfull = opts2[best].wfull;
  a.nbuf = opts2[best].nbuf;
  p.lds = (size_t)best_lds;
  plan_pack(d, op, p, taps, nstep);

  // Split K over the source-channel chunks when there are fewer output tiles
  // than CUs: the largest divisor of nchunks that keeps jobs <= kSplitTarget
  // (two workgroups per CU).  With a tile per CU already, the partial-sum
  // traffic and the epilogue pass cost more than the extra parallelism gains
  // (measured).  Only the Conv3d modes, whose K is long.
  p.ntiles = (int64_t)d->n * a.nbd * a.nbh * a.nbw * a.n_ctiles;
  int split = 1;
  if ((p.mode == MODE_K3 || p.mode == MODE_K1) && p.ntiles < kNumCUs) {
    const int64_t want = (kSplitTarget + p.ntiles - 1) / p.ntiles;
    for (int sp = 2; sp <= a.nchunks && sp <= want; ++sp)
      if (a.nchunks % sp == 0) split = sp;
  }
  a.nsplit = split;
  a.cps = a.nchunks / split;
  const int mb = mb1 ? 1 : 2;
  p.part_bytes = split > 1 ? align256(p.ntiles * split * 4 * mb * p.nb * 16 * 64 * 4) : 0;
}

// ---------------------------------------------------------------------------
// Register-direct ConvTranspose dX (r3c_t2dx.h)
// ---------------------------------------------------------------------------
struct T2dxPlan {
  int rb;
  T2dxArgs a;
  T2dxPackArgs pk;
  size_t lds;
  int64_t wpk_bytes;
};

// w-contiguous dY with even strides (4-byte pair loads), dX with dense planes
// (positions addressed directly), S % 32 == 0 and N * S < 2^31.
bool plan_t2dx(const r3c_conv_desc* d, T2dxPlan& p) {
  memset(&p, 0, sizeof p);
  T2dxArgs& a = p.a;
  const int64_t* ys = d->y_strides;
  const int64_t* xs = d->x_strides;
  const int64_t D = d->d, H = d->h, W = d->w;
  if (ys[4] != 1 || ys[3] % 2 || ys[2] % 2 || ys[1] % 2 || ys[0] % 2) return false;
  if (xs[4] != 1 || xs[3] != W || xs[2] != H * W || xs[1] <= 0 || xs[0] <= 0) return false;
  const int64_t S = D * H * W;
  if (S % 32 != 0 || S * d->n >= (1ll << 31)) return false;
  a.dy_bytes = sample_bytes(ys, d->cout, 2 * D, 2 * H, 2 * W);
  a.dx_bytes = sample_bytes(xs, d->cin, D, H, W);
  if (a.dy_bytes == 0 || a.dx_bytes == 0) return false;
  a.ys0 = ys[0];
  a.ys1 = ys[1];
  a.ys2 = (int32_t)ys[2];
  a.ys3 = (int32_t)ys[3];
  a.xs0 = xs[0];
  a.xs1 = xs[1];
  a.Cin = d->cin;
  a.Cout = d->cout;
  a.nks = cdiv(8 * d->cout, 16);
  if (a.nks > 64) return false;  // A fragments of a row block beyond 64 KB of LDS
  // Two row blocks per workgroup where they fit 64 KB of LDS (more spill).
  const int nrb = cdiv(d->cin, 32);
  const int rb = (nrb >= 2 && 2 * a.nks <= 64) ? 2 : 1;
  a.nrg = cdiv(nrb, rb);
  p.rb = cdiv(nrb, a.nrg);
  a.S = (int32_t)S;
  a.W = (int32_t)W;
  a.HW = (int32_t)(H * W);
  a.ncb = (int32_t)(S * d->n / 32);
  // About two workgroups per CU over all row groups, each wave with at least
  // one column block.
  a.ncw = (int32_t)std::max<int64_t>(1, std::min<int64_t>(cdiv((int64_t)a.ncb, 8), cdiv((int64_t)2 * kNumCUs, a.nrg)));
  p.lds = (size_t)p.rb * a.nks * 1024;
  p.pk.cin = d->cin;
  p.pk.cout = d->cout;
  p.pk.nks = a.nks;
  p.pk.total = a.nrg * p.rb * a.nks * 64;
  p.wpk_bytes = (int64_t)p.pk.total * 16;
  return true;
}

int run_t2dx(const r3c_conv_desc* d, const T2dxPlan& p, const void* dy, const void* w, void* dx, void* ws,
             int64_t ws_bytes, hipStream_t s) {
  if (ws_bytes < p.wpk_bytes)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)p.wpk_bytes);
  if (!dy || !w || !dx || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  int rc = check_device();
  if (rc) return rc;
  T2dxPackArgs pk = p.pk;
  pk.w = static_cast<const uint16_t*>(w);
  pk.out = static_cast<uint16_t*>(ws);
  {
    TimedLaunch tl(KIND_PACK, s);
    launch_t2dx_pack(pk, s);
    tl.end();
  }
  rc = check_launch("ConvTranspose dX weight pack");
  if (rc) return rc;
  T2dxArgs a = p.a;
  a.dy = static_cast<const uint16_t*>(dy);
  a.apk = static_cast<const uint16_t*>(ws);
  a.dx = static_cast<uint16_t*>(dx);
  TimedLaunch tl(KIND_ROW, s);
  const bool launched = launch_t2dx(d->dtype, p.rb, a, p.lds, s);
  tl.end();
  if (!launched) return fail(R3C_UNSUPPORTED, "no ConvTranspose dX instantiation for rb %d", p.rb);
  return check_launch("ConvTranspose dX kernel");
}

// Why a row plan cannot run (nullptr: it can).  The workspace query applies
// the same checks, so a descriptor it accepts never fails on these grounds.
const char* row_plan_reject(const RowPlan& p) {
  if ((int64_t)p.lds > kMaxLds) return "the tile needs more LDS than a compute unit has";
  if (p.a.src_bytes == 0) return "one input sample exceeds 1 GiB (32-bit buffer offsets)";
  if (p.tap && p.a.dst_bytes == 0) return "one output sample exceeds 1 GiB (32-bit buffer offsets)";
  if (p.ntiles * p.a.nsplit >= (1ll << 31)) return "grid too large";
  return nullptr;
}

int64_t row_plan_ws(const RowPlan& p) { return align256(p.wpk_bytes) + p.copy_bytes + p.part_bytes; }

// The register-direct ConvTranspose dX loads 4-byte pairs; other alignments
// take the row kernel (mode T2DX), which stages any alignment.
bool t2dx_aligned(const void* dy, const void* dx) {
  return ((reinterpret_cast<uintptr_t>(dy) | reinterpret_cast<uintptr_t>(dx)) & 3) == 0;
}

// k=1 without padding, at most 4 output channels, dense NCDHW planes of a
// multiple of 8 positions: the streaming kernels of r3c_skinny.hip.
bool skinny_ok(const r3c_conv_desc* d) {
  if (d->kernel != 1 || d->pad_d || d->pad_h || d->pad_w || d->cout > 4 || d->cin > kSkinnyMaxC) return false;
  const int64_t P = (int64_t)d->d * d->h * d->w;
  if (P % 8 != 0 || (int64_t)d->n * (P / 8) >= (1ll << 31)) return false;
  const int64_t* st[2] = {d->x_strides, d->y_strides};
  for (const int64_t* t : st)
    if (!(t[4] == 1 && t[3] == d->w && t[2] == (int64_t)d->h * d->w && t[1] % 8 == 0 && t[0] % 8 == 0 &&
          t[1] >= P && t[0] > 0))
      return false;
  return true;
}

SkinnyArgs skinny_args(const r3c_conv_desc* d) {
  SkinnyArgs a;
  memset(&a, 0, sizeof a);
  a.xs0 = d->x_strides[0];
  a.xs1 = d->x_strides[1];
  a.ys0 = d->y_strides[0];
  a.ys1 = d->y_strides[1];
  a.P = (int64_t)d->d * d->h * d->w;
  a.ngroups = (int64_t)d->n * (a.P / 8);
  a.C = d->cin;
  a.O = d->cout;
  return a;
}

// Conv3d k=3 with one input channel (r3c_stem.hip): input rows w-contiguous
// and 16-byte aligned (W % 8 == 0, at most kStemMaxW), padding at most 2, at
// most kStemMaxCout output channels.  dW also reads dY rows as 16-byte
// vectors (ow-contiguous, aligned, OW % 16 == 0).  Pointer alignment is
// checked by the caller.
bool stem_ok(const r3c_conv_desc* d, bool dw) {
  if (d->kernel != 3 || d->cin != 1 || d->cout > kStemMaxCout) return false;
  if (d->pad_d > 2 || d->pad_h > 2 || d->pad_w > 2) return false;
  if (d->w % 8 || d->w > kStemMaxW || d->ow > kStemMaxW) return false;
  const int64_t* xs = d->x_strides;
  if (xs[4] != 1 || xs[3] % 8 || xs[2] % 8 || xs[0] % 8) return false;
  if ((int64_t)d->n * d->od * cdiv(d->oh, kStemRows) >= (1ll << 31)) return false;
  if (dw) {
    const int64_t* ys = d->y_strides;
    if (ys[4] != 1 || ys[3] % 8 || ys[2] % 8 || ys[1] % 8 || ys[0] % 8 || d->ow % 16) return false;
  }
  return true;
}

constexpr int kStemSplits = 1024;  // dW partials (workgroups), at most

StemArgs stem_args(const r3c_conv_desc* d) {
  StemArgs a;
  memset(&a, 0, sizeof a);
  a.xs0 = d->x_strides[0];
  a.xs2 = d->x_strides[2];
  a.xs3 = d->x_strides[3];
  for (int i = 0; i < 5; ++i) (&a.ys0)[i] = d->y_strides[i];
  a.D = d->d;
  a.H = d->h;
  a.W = d->w;
  a.OD = d->od;
  a.OH = d->oh;
  a.OW = d->ow;
  a.pd = d->pad_d;
  a.ph = d->pad_h;
  a.pw = d->pad_w;
  a.Cout = d->cout;
  // Row pitch: data at [8, 8 + W), zeros around it, and room for the reads of
  // the last 32-position tile (up to 2 past the row, plus the kw shifts).
  a.P = (int32_t)((std::max<int64_t>(d->w, cdiv(d->ow, 32) * 32) + 18 + 7) / 8 * 8);
  a.nrb = (int32_t)cdiv(d->oh, kStemRows);
  a.njobs = d->n * d->od * a.nrb;
  a.nsplit = std::min(a.njobs, kStemSplits);
  return a;
}

// Dynamic LDS: the staged input rows; dW reuses them for the 4 waves'
// accumulators, the forward appends each wave's output block (32 channels x
// 72 positions per channel block) when it stores positions 8 at a time.
size_t stem_lds(const StemArgs& a, bool dw) {
  const int nb = a.Cout <= 32 ? 1 : 2;
  const size_t tile = (size_t)kStemXRows * a.P * 2;
  if (dw) return std::max(tile, (size_t)kStemRows * nb * 16 * 64 * 4);
  return tile + (a.yvec8 ? (size_t)kStemRows * nb * 32 * 72 * 2 : 0);
}

bool aligned16_all(std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (reinterpret_cast<uintptr_t>(p) & 15) return false;
  return true;
}

// Descriptor checks of a channel concatenation (see CatSpec): k=3, NCDHW
// planes dense in (d, h, w), the split a positive multiple of 8 below cin, and
// sample strides that hold each tensor's channel planes.
int cat_check(const r3c_conv_desc* d, int32_t ca, int64_t xb_s0) {
  int rc = validate(d, false);
  if (rc) return rc;
  const int64_t* st = d->x_strides;
  if (d->kernel != 3) return fail(R3C_UNSUPPORTED, "channel concatenation: kernel must be 3");
  if (ca <= 0 || ca >= d->cin || ca % 8) return fail(R3C_UNSUPPORTED, "channel concatenation: split %d", ca);
  if (!(st[4] == 1 && st[3] == d->w && st[2] == (int64_t)d->h * d->w && st[1] % 8 == 0 && st[0] % 8 == 0 &&
        st[1] >= (int64_t)d->d * d->h * d->w && st[0] >= (int64_t)ca * st[1] && xb_s0 % 8 == 0 &&
        xb_s0 >= (int64_t)(d->cin - ca) * st[1]))
    return fail(R3C_UNSUPPORTED, "channel concatenation: tensors must be NCDHW with dense (d, h, w) planes");
  return R3C_OK;
}

// Channel concatenation [A, B] as the x of a k=3 Conv3d (the r3c_conv3d_cat_*
// entry points): A has `ca` channels and the descriptor's x strides, B the
// same channel and spatial strides and its own sample stride.
struct CatSpec {
  int32_t ca;
  const void* xb;   // forward and dW: B
  void* dxb;        // dX: B's gradient
  int64_t xb_s0;
};

int run_row(const r3c_conv_desc* d, int op, const void* src, const void* w, const void* bias, void* dst, void* ws,
            int64_t ws_bytes, void* stream, const CatSpec* cat = nullptr) {
  if (!cat && op == OP_CONV_FWD && stem_ok(d, false) && aligned16_all({src}) && src && dst && w) {
    int rc = check_device();
    if (rc) return rc;
    StemArgs a = stem_args(d);
    a.x = static_cast<const uint16_t*>(src);
    a.w = static_cast<const uint16_t*>(w);
    a.b = static_cast<const uint16_t*>(bias);
    a.y = static_cast<uint16_t*>(dst);
    a.yvec4 = a.ys1 == 1 && a.Cout % 4 == 0 && a.ys0 % 4 == 0 && a.ys2 % 4 == 0 && a.ys3 % 4 == 0 &&
              a.ys4 % 4 == 0 && (reinterpret_cast<uintptr_t>(dst) & 7) == 0;
    a.yvec8 = a.ys4 == 1 && a.OW % 8 == 0 && a.ys0 % 8 == 0 && a.ys1 % 8 == 0 && a.ys2 % 8 == 0 &&
              a.ys3 % 8 == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    TimedLaunch tl(KIND_ROW, s);
    const bool launched = launch_stem(d->dtype, 0, a, stem_lds(a, false), s);
    tl.end();
    if (!launched) return fail(R3C_UNSUPPORTED, "no one-channel k=3 instantiation for %d output channels", a.Cout);
    return check_launch("one-channel k=3 forward");
  }
  if (!cat && (op == OP_CONV_FWD || op == OP_CONV_DX) && skinny_ok(d) && aligned16_all({src, dst}) && src && dst && w) {
    int rc = check_device();
    if (rc) return rc;
    SkinnyArgs a = skinny_args(d);
    a.w = static_cast<const uint16_t*>(w);
    if (op == OP_CONV_FWD) {
      a.x = const_cast<uint16_t*>(static_cast<const uint16_t*>(src));
      a.y = static_cast<uint16_t*>(dst);
      a.b = static_cast<const uint16_t*>(bias);
    } else {
      a.y = const_cast<uint16_t*>(static_cast<const uint16_t*>(src));
      a.x = static_cast<uint16_t*>(dst);
    }
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    TimedLaunch tl(KIND_ROW, s);
    const bool launched = launch_skinny(d->dtype, op == OP_CONV_FWD ? 0 : 1, a, s);
    tl.end();
    if (!launched) return fail(R3C_UNSUPPORTED, "no k=1 skinny instantiation for %d output channels", a.O);
    return check_launch(op == OP_CONV_FWD ? "k=1 skinny forward" : "k=1 skinny dX");
  }
  if (op == OP_T2_DX && t2dx_aligned(src, dst)) {
    T2dxPlan tp;
    if (plan_t2dx(d, tp)) return run_t2dx(d, tp, src, w, dst, ws, ws_bytes, reinterpret_cast<hipStream_t>(stream));
  }
  RowPlan p;
  plan_row(d, op, p);
  if (p.copy_bytes && (reinterpret_cast<uintptr_t>(src) & 15)) plan_row(d, op, p, false);  // same or less workspace
  if (cat) {
    // The concatenation is read by the w-contiguous staging (forward) or
    // written by the NCDHW epilogue (dX) of the tap kernel, from 16-byte
    // aligned tensors; anything else has no plan here.
    if (!p.tap || p.copy_bytes || (op == OP_CONV_FWD && p.cl != 3) ||
        !aligned16_all({src, dst, op == OP_CONV_FWD ? cat->xb : static_cast<const void*>(cat->dxb)}))
      return fail(R3C_UNSUPPORTED, "no plan for this channel concatenation");
  }
  if (const char* why = row_plan_reject(p)) return fail(R3C_UNSUPPORTED, "%s", why);
  const int64_t need = row_plan_ws(p);
  if (ws_bytes < need)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
  if (!src || !w || !dst || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  int rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  char* wsb = static_cast<char*>(ws);
  float* part = p.part_bytes ? reinterpret_cast<float*>(wsb + align256(p.wpk_bytes) + p.copy_bytes) : nullptr;
  PackArgs pk = p.pk;
  pk.w = static_cast<const uint16_t*>(w);
  pk.out = static_cast<uint16_t*>(ws);
  {
    TimedLaunch tl(KIND_PACK, s);
    launch_pack(d->dtype, pk, s);
    tl.end();
  }
  rc = check_launch("weight pack");
  if (rc) return rc;
  if (p.copy_bytes) {
    void* copy = static_cast<char*>(ws) + align256(p.wpk_bytes);
    rc = copy_to_channels_last(src, copy, d->n, p.a.Cs, p.a.Sd, p.a.Sh, p.a.Sw, s);
    if (rc) return rc;
    src = copy;
  }
  RowArgs a = p.a;
  a.src = static_cast<const uint16_t*>(src);
  a.wpk = static_cast<const uint16_t*>(ws);
  a.bias = static_cast<const uint16_t*>(bias);
  a.dst = static_cast<uint16_t*>(dst);
  if (cat && op == OP_CONV_FWD) {
    a.src2 = static_cast<const uint16_t*>(cat->xb);
    a.ss0_2 = cat->xb_s0;
    a.csplit = cat->ca;
    a.src_bytes = (uint32_t)(2 * (int64_t)cat->ca * a.ss[1]);
    a.src2_bytes = (uint32_t)(2 * (int64_t)(d->cin - cat->ca) * a.ss[1]);
  } else if (cat) {
    a.dst2 = static_cast<uint16_t*>(cat->dxb);
    a.sd0_2 = cat->xb_s0;
    a.dsplit = cat->ca;
    a.dst_bytes = (uint32_t)(2 * (int64_t)cat->ca * a.sd[1]);
    a.dst2_bytes = (uint32_t)(2 * (int64_t)(d->cin - cat->ca) * a.sd[1]);
  }
  // 16-byte staging needs a 16-byte aligned source; otherwise stage by scalars.
  const int cl = (reinterpret_cast<uintptr_t>(src) & 15) == 0 ? p.cl : 0;
  a.src_cl = cl;
  a.part = part;
  a.ntiles = (int32_t)p.ntiles;
  {
    const int64_t span = (int64_t)a.ncols * std::llabs(a.sd[1]) + 64 * std::llabs(a.sd[4]) + 64;
    a.off32 = span < (1ll << 31) ? 1 : 0;
  }
  a.phase = 0;
  a.njobs = (int32_t)(p.ntiles * a.nsplit);  // below 2^31 (row_plan_reject)
  // The launcher sizes the grid to the resident capacity (CUs x workgroups
  // per CU from the occupancy query); workgroups take contiguous job ranges.
  TimedLaunch tl(KIND_ROW, s);
  const bool launched = p.tap ? launch_tap(d->dtype, p.nb, p.mb, cl, a.wfull, p.lw, a, t_cus, p.lds, s)
                              : launch_row(d->dtype, p.mode, p.nb, cl, a.wfull, a, t_cus, p.lds, s);
  tl.end();
  if (!launched)
    return fail(R3C_UNSUPPORTED, "no row-kernel instantiation for mode %d ck %d nb %d cl %d", p.mode, p.ck, p.nb,
                p.cl);
  rc = check_launch("row kernel");
  if (rc || a.nsplit == 1) return rc;
  // Split K: the epilogue pass adds each tile's split partial sums in split order.
  a.phase = 1;
  TimedLaunch te(KIND_SPLIT_EPI, s);
  if (p.tap) launch_tap(d->dtype, p.nb, p.mb, cl, a.wfull, p.lw, a, t_cus, p.lds, s);
  else launch_row(d->dtype, p.mode, p.nb, cl, a.wfull, a, t_cus, p.lds, s);
  te.end();
  return check_launch("row kernel epilogue pass");
}

// ---------------------------------------------------------------------------
// Weight-gradient plan (Conv3d dW k1/k3, ConvTranspose dW)
// ---------------------------------------------------------------------------
struct WgPlan {
  int mode, cbw, taps;
  int pw;              // 1: register-direct single-tap kernel (r3c_pwdw.h), fields below
  int tr, tc, nj;
  PwdwArgs pa;
  int fl;  // 1: F staged channel-major from its w-contiguous source; 2: G too (k=1, no padding);
           // 3: k=3, G transposed from w-contiguous in the kernel; 5: k=3 row-walking kernel (r3c_wgrow.h)
  WgArgs a;
  size_t lds;
  int64_t part_bytes, dbpart_bytes;
  int64_t fcopy_bytes, gcopy_bytes;  // > 0: that operand is first copied to NDHWC
};

// Dense w-contiguous planes (NCDHW-like: channel and sample strides free).
bool dense_planes(const int64_t* st, int64_t h, int64_t w) {
  return st[4] == 1 && st[3] == w && st[2] == h * w && st[1] % 8 == 0 && st[0] % 8 == 0 && st[0] > 0 && st[1] > 0;
}

// Register-direct plan for the single-tap weight gradients (Conv3d k=1 without
// padding, ConvTranspose k2s2) when both operands have dense w-contiguous
// planes: K blocks of 64 positions (k=1, S % 64 == 0) or of 16 / 32 positions
// within one w row (ConvTranspose, W % 16 == 0).  The GEMM always reserves the
// bias gradient's ones row / column, so the plan does not depend on db.
bool plan_pwdw(const r3c_conv_desc* d, bool transpose, WgPlan& p) {
  WgArgs& w = p.a;
  PwdwArgs& a = p.pa;
  memset(&a, 0, sizeof a);
  int64_t S;
  if (transpose) {
    if (!dense_planes(w.fs, w.Rh, w.Rw) || !dense_planes(w.gs, 2ll * w.Rh, 2ll * w.Rw)) return false;
    if (w.Gd != 2 * w.Rd || w.Gh != 2 * w.Rh || w.Gw != 2 * w.Rw || w.Rw % 16 != 0) return false;
    p.nj = w.Rw % 32 == 0 ? 2 : 1;
    S = (int64_t)w.Rd * w.Rh * w.Rw;
  } else {
    // k=1: with at most 32 output channels (one row block) the LDS-staged
    // kernel streams faster (measured 168 vs 196 us at [4,48,64,128,128] -> 24;
    // 338 vs 404 us the other way at -> 96).
    if (d->kernel != 1 || w.pd || w.ph || w.pw || w.Fc <= 32) return false;
    if (!dense_planes(w.fs, w.Rh, w.Rw) || !dense_planes(w.gs, w.Gh, w.Gw)) return false;
    if (w.Gd != w.Rd || w.Gh != w.Rh || w.Gw != w.Rw) return false;
    p.nj = 4;
    S = (int64_t)w.Rd * w.Rh * w.Rw;
    if (S % 64 != 0) return false;
  }
  if (S * d->n >= (1ll << 31)) return false;
  a.f_bytes = sample_bytes(w.fs, w.Fc, w.Rd, w.Rh, w.Rw);
  a.g_bytes = sample_bytes(w.gs, w.Gc, w.Gd, w.Gh, w.Gw);
  if (a.f_bytes == 0 || a.g_bytes == 0) return false;
  a.fs0 = w.fs[0];
  a.fs1 = w.fs[1];
  a.gs0 = w.gs[0];
  a.gs1 = w.gs[1];
  a.Fc = w.Fc;
  a.Gc = w.Gc;
  a.taps = p.taps;
  a.S = (int32_t)S;
  a.W = w.Rw;
  a.HW = w.Rh * w.Rw;
  a.M = w.Fc + (transpose ? 1 : 0);
  a.ncols = p.taps * w.Gc + (transpose ? 0 : 1);
  // Tiles per workgroup (TR x TC blocks of 32): the instantiated shapes that
  // fit the register file -- TR * TC <= 3 for k=1 (64-position K blocks), and
  // up to 2 x 2 for ConvTranspose.
  const int nrb = cdiv(a.M, 32), ncb = cdiv(a.ncols, 32);
  if (transpose) {
    p.tr = std::min(nrb, 2);
    p.tc = std::min(ncb, p.tr == 1 ? 3 : 2);
    if (nrb >= 3 && ncb == 1) p.tr = 3;
  } else {
    p.tr = std::min(nrb, 3);
    p.tc = std::min(ncb, 3 / p.tr);
  }
  a.ngr = cdiv(nrb, p.tr);
  a.ngc = cdiv(ncb, p.tc);
  const int kbpos = 16 * p.nj;
  a.nkb = (int32_t)(S * d->n / kbpos);
  // About two workgroups per CU, at least 8 K blocks (one per wave) each, and
  // at most kMaxPartialBytes of partials.
  const int ntg = a.ngr * a.ngc;
  const int64_t per_split = (int64_t)w.Fc * p.taps * w.Gc * 4;
  int64_t nsplit = cdiv((int64_t)2 * kNumCUs, ntg);
  nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, a.nkb / 8));
  nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, kMaxPartialBytes / per_split));
  if (nsplit >= 8) nsplit -= nsplit % 8;  // a grid of whole XCD eighths (the kernel's renumbering)
  a.nsplit = (int32_t)std::max<int64_t>(1, nsplit);
  a.kil = transpose ? 1 : 0;  // K-block order per split (measured per mode)
  p.pw = 1;
  p.mode = transpose ? MODE_T2DW : MODE_K1;
  p.part_bytes = align256(a.nsplit * per_split);
  p.dbpart_bytes = align256((int64_t)a.nsplit * std::max(w.Fc, 8 * w.Gc) * 4);
  p.fcopy_bytes = p.gcopy_bytes = 0;
  p.lds = 0;
  return true;
}

// allow_pw false: no register-direct plan (it needs 16-byte aligned sources);
// allow_copy false: no NDHWC copy of an operand (likewise).
// gcw_div > 0: G tiles must not straddle channel gcw_div (a channel concatenation's split).
void plan_wgrad(const r3c_conv_desc* d, bool transpose, WgPlan& p, bool allow_pw = true, bool allow_copy = true,
                int gcw_div = 0) {
  WgArgs& a = p.a;
  memset(&a, 0, sizeof a);
  if (transpose) {
    p.mode = MODE_T2DW;
    p.taps = 8;
    a.Fc = d->cin; a.Gc = d->cout;
    a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
    a.Gd = d->od; a.Gh = d->oh; a.Gw = d->ow;
    memcpy(a.fs, d->x_strides, sizeof a.fs);
    memcpy(a.gs, d->y_strides, sizeof a.gs);
  } else {
    p.mode = d->kernel == 3 ? MODE_K3 : MODE_K1;
    p.taps = d->kernel == 3 ? 27 : 1;
    a.Fc = d->cout; a.Gc = d->cin;
    a.Rd = d->od; a.Rh = d->oh; a.Rw = d->ow;
    a.Gd = d->d; a.Gh = d->h; a.Gw = d->w;
    a.pd = d->pad_d; a.ph = d->pad_h; a.pw = d->pad_w;
    memcpy(a.fs, d->y_strides, sizeof a.fs);
    memcpy(a.gs, d->x_strides, sizeof a.gs);
  }
  p.pw = 0;
  if (allow_pw && plan_pwdw(d, transpose, p)) return;
  // NCDHW operands of the k=3 pass are copied to NDHWC first: the tiles are
  // [position][channel], which strided staging fills slowly, and the pass does
  // enough arithmetic per byte to pay for the copy.  The memory-bound k=1 and
  // ConvTranspose passes stage strided operands directly.
  p.fcopy_bytes = p.gcopy_bytes = 0;
  const bool copy_ok = p.mode == MODE_K3 && allow_copy;
  // F needs no tap halo: a w-contiguous F (NCDHW) is staged channel-major
  // straight from the source (fl 1), with no copy.
  p.fl = (a.fs[4] == 1 && a.Rw % 8 == 0 && a.fs[0] % 8 == 0 && a.fs[1] % 8 == 0 && a.fs[2] % 8 == 0 &&
          a.fs[3] % 8 == 0) ? 1 : 0;
  // A k=1 pass without padding has no tap shift: G sits on F's grid and a
  // w-contiguous G is staged channel-major the same way (fl 2).
  if (p.fl && p.mode == MODE_K1 && a.pd == 0 && a.ph == 0 && a.pw == 0 && a.gs[4] == 1 && a.Gw % 8 == 0 &&
      a.gs[0] % 8 == 0 && a.gs[1] % 8 == 0 && a.gs[2] % 8 == 0 && a.gs[3] % 8 == 0)
    p.fl = 2;
  // With no tap shift the positions can be walked in any order.  When both
  // operands hold each channel's D*H*W positions contiguously, view them as
  // [S/64][4][16]: a box of 4 x 4 x 16 is then 256 consecutive positions, so a
  // channel's slice of a box is one 512-byte run instead of 16 runs of 32 bytes.
  if (p.fl == 2) {
    const int64_t S = (int64_t)a.Rd * a.Rh * a.Rw;
    const bool dense = a.fs[2] == (int64_t)a.Rh * a.Rw && a.fs[3] == a.Rw && a.gs[2] == a.fs[2] &&
                       a.gs[3] == a.fs[3] && a.Gd == a.Rd && a.Gh == a.Rh && a.Gw == a.Rw;
    if (dense && S % 64 == 0 && S / 64 < (1ll << 30)) {
      a.Rd = a.Gd = (int32_t)(S / 64);
      a.Rh = a.Gh = 4;
      a.Rw = a.Gw = 16;
      a.fs[2] = a.gs[2] = 64;
      a.fs[3] = a.gs[3] = 16;
    }
  }
  // k=3 with G w-contiguous too (both NCDHW): G is staged straight from its
  // source with a register transpose (fl 3) instead of being copied to NDHWC.
  // Its 8-aligned w segments [r0w - 8, r0w + 24) cover the halo row for pw <= 6.
  // It loads 1.8x the bytes of NDHWC staging plus the transposes, which costs
  // more than the copy saves above 64 G channels (measured: 24 and 48 channels
  // gain 52 and 22 us per trunk pass, 96 loses 15, 192 breaks even; with the
  // halved splits below, 96 loses 3.5 us and 192 gains 2).
  // The channel planes must be outermost in a sample: G's buffer range then
  // ends at channel Gc and the kernel gates no channel.
  const bool g_wcontig =
      p.fl == 1 && p.mode == MODE_K3 && a.gs[4] == 1 && a.Gw % 8 == 0 && a.gs[0] % 8 == 0 && a.gs[1] % 8 == 0 &&
      a.gs[2] % 8 == 0 && a.gs[3] % 8 == 0 && a.pw >= 0 && a.pw <= 6 && a.gs[2] > 0 && a.gs[3] > 0 &&
      a.gs[1] >= (int64_t)(a.Gd - 1) * a.gs[2] + (int64_t)(a.Gh - 1) * a.gs[3] + a.Gw &&
      2 * (int64_t)(a.Gc + 8) * a.gs[1] < (1ll << 30);  // no 32-bit wrap past the last channel group
  // k=3 with pad_w 1, the same w-contiguous sources 16-byte aligned (the
  // caller's allow_copy) and rows of 32, 64 or 128 positions: the row-walking
  // kernel (fl 5, r3c_wgrow.h) fetches whole lines with no w halo, each x row
  // once per column of output rows, and feeds the three kw taps of a (kd, kh)
  // from one LDS read.
  if (g_wcontig && allow_copy && a.pw == 1 && a.Rw == a.Gw &&
      (a.Rw == 32 || a.Rw == 64 || a.Rw == 128) && wgrow_enabled())
    p.fl = 5;
  else if (g_wcontig && a.Gc <= 64) p.fl = 3;
  if (!p.fl && copy_ok && ncdhw_copyable(a.fs, a.Fc, a.Rd, a.Rh, a.Rw)) {
    p.fcopy_bytes = align256(tensor_bytes(d->n, a.Fc, a.Rd, a.Rh, a.Rw));
    channels_last_strides(a.fs, a.Fc, a.Rd, a.Rh, a.Rw);
  }
  if (copy_ok && p.fl < 3 && ncdhw_copyable(a.gs, a.Gc, a.Gd, a.Gh, a.Gw)) {
    p.gcopy_bytes = align256(tensor_bytes(d->n, a.Gc, a.Gd, a.Gh, a.Gw));
    channels_last_strides(a.gs, a.Gc, a.Gd, a.Gh, a.Gw);
  }
  a.f_bytes = sample_bytes(a.fs, a.Fc, a.Rd, a.Rh, a.Rw);
  a.g_bytes = p.fl == 3 ? (uint32_t)(2 * (int64_t)a.Gc * a.gs[1]) : sample_bytes(a.gs, a.Gc, a.Gd, a.Gh, a.Gw);
  // G channel range per tile: a multiple of 8 (16-byte staging) and of 4 (quads).
  if (p.fl == 5) {
    // 8, 16 or 24 channels (9 GCW columns in blocks of 32, one block per
    // wave): the width with the fewest column blocks over all G tiles.
    int best = 0;
    for (int gcw : {24, 16, 8}) {
      if (gcw_div > 0 && gcw_div % gcw != 0) continue;
      const int64_t cost = cdiv(a.Gc, gcw) * cdiv(9 * gcw, 32);
      if (!best || cost < cdiv(a.Gc, best) * cdiv(9 * best, 32)) best = gcw;
    }
    a.GCW = best;
  } else if (a.Gc <= 32) a.GCW = (a.Gc + 7) / 8 * 8;
  else if (a.Gc % 32 == 0) a.GCW = 32;
  else if (a.Gc % 24 == 0) a.GCW = 24;
  else a.GCW = 32;
  a.n_ftiles = cdiv(a.Fc, 32);
  a.n_gtiles = cdiv(a.Gc, a.GCW);
  a.Fpad = a.n_ftiles * 32;
  a.Gpad = a.n_gtiles * a.GCW;
  const int ncb = cdiv((int64_t)p.taps * (a.GCW / 4), 8);  // 32-column blocks
  p.cbw = cdiv(ncb, 8);                                      // per wave, 8 waves
  const int cbw_max = p.mode == MODE_K3 ? 4 : (p.mode == MODE_K1 ? 1 : 2);
  if (p.cbw > cbw_max) p.cbw = cbw_max;  // cannot happen with GCW <= 32
  // Box geometry is fixed per mode (WgGeom).
  int TD, TH, lds;
  if (p.mode == MODE_K3) TD = WgGeom<MODE_K3>::TD, TH = WgGeom<MODE_K3>::TH, lds = WgGeom<MODE_K3>::LDS_BYTES;
  else if (p.mode == MODE_K1) TD = WgGeom<MODE_K1>::TD, TH = WgGeom<MODE_K1>::TH, lds = WgGeom<MODE_K1>::LDS_BYTES;
  else TD = WgGeom<MODE_T2DW>::TD, TH = WgGeom<MODE_T2DW>::TH, lds = WgGeom<MODE_T2DW>::LDS_BYTES;
  if (p.fl == 3) lds += WgGeom<MODE_K3>::TRASH_BYTES;
  if (p.fl == 5) {
#define R3C_WR_LDS(WL_) (a.GCW == 8 ? WrGeom<8, WL_>::LDS_BYTES : a.GCW == 16 ? WrGeom<16, WL_>::LDS_BYTES \
                                                               : WrGeom<24, WL_>::LDS_BYTES)
    lds = a.Rw == 32 ? R3C_WR_LDS(2) : a.Rw == 64 ? R3C_WR_LDS(4) : R3C_WR_LDS(8);
#undef R3C_WR_LDS
  }
  a.nbd = cdiv(a.Rd, TD);
  a.nbh = cdiv(a.Rh, TH);
  a.nbw = cdiv(a.Rw, 16);
  int64_t nbox = (int64_t)d->n * a.nbd * a.nbh * a.nbw;
  const int tiles = a.n_ftiles * a.n_gtiles;
  if (p.fl == 5) {
    // Jobs (n, d, h range): enough h ranges per (n, d) column to give every CU
    // a workgroup, each range at least 8 rows long.
    const int64_t cols = (int64_t)d->n * a.Rd;
    int64_t hs = std::max<int64_t>(1, cdiv(kNumCUs, cols * tiles));
    hs = std::min<int64_t>(hs, std::max(1, a.Rh / 8));
    a.nbd = a.Rd;
    a.nbh = (int32_t)hs;
    a.nbw = 1;
    nbox = cols * hs;
  }
  a.nbox = (int32_t)std::min<int64_t>(nbox, (1ll << 31) - 1);
  const int64_t per_split = (int64_t)a.Fpad * p.taps * a.Gpad * 4;
  // Enough workgroups to fill every CU at the LDS-limited occupancy, no more:
  // each extra split costs partial traffic.
  const int64_t wg_target = (int64_t)kNumCUs * std::max<int64_t>(1, kMaxLds / lds);
  int64_t nsplit = cdiv(wg_target, tiles);
  // Each split writes its fp32 partial sums and the reduce reads them back.
  // Where those would outweigh the operands (many channels over few
  // positions), half the splits is faster: fewer partial bytes, and each
  // workgroup's prologue and partial write-out cover twice the boxes
  // (measured: 96->96 dW pass 101 -> 90 us, 192->192 73 -> 62 us; a quarter
  // is slower again, 133 and 79 us).
  const int64_t op_bytes =
      2 * (int64_t)d->n * ((int64_t)a.Fc * a.Rd * a.Rh * a.Rw + (int64_t)a.Gc * a.Gd * a.Gh * a.Gw);
  if (nsplit * per_split > op_bytes && p.fl != 5) nsplit = std::max<int64_t>(1, nsplit / 2);
  // Row-walking jobs: one per workgroup while the partial sums stay below the
  // operand bytes, else as many as fill every CU once (a workgroup then walks
  // several columns).
  if (p.fl == 5) nsplit = std::min<int64_t>(nbox, std::max<int64_t>(cdiv(kNumCUs, tiles), op_bytes / per_split));
  nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, kMaxPartialBytes / per_split));
  nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, nbox));
  a.nsplit = (int32_t)nsplit;
  a.nblocks = (int32_t)(nsplit * tiles);
  p.lds = (size_t)lds;
  p.part_bytes = align256(nsplit * per_split);
  p.dbpart_bytes = align256(nsplit * (int64_t)std::max(a.Fpad, p.taps * a.Gpad) * 4);
}

// Register-direct single-tap weight gradient, then the shared fixed-order reduce.
int run_pwdw(const r3c_conv_desc* d, bool transpose, const WgPlan& p, const void* x, const void* dy, void* dw,
             int dw_dtype, void* db, int db_dtype, void* ws, hipStream_t s) {
  PwdwArgs a = p.pa;
  a.fsrc = static_cast<const uint16_t*>(transpose ? x : dy);
  a.gsrc = static_cast<const uint16_t*>(transpose ? dy : x);
  a.part = static_cast<float*>(ws);
  a.dbpart = reinterpret_cast<float*>(static_cast<char*>(ws) + p.part_bytes);
  a.db_mode = db ? (transpose ? 2 : 1) : 0;
  TimedLaunch tl(KIND_WGRAD, s);
  const bool launched = launch_pwdw(d->dtype, p.mode, p.tr, p.tc, p.nj, a, s);
  tl.end();
  if (!launched)
    return fail(R3C_UNSUPPORTED, "no single-tap weight-gradient instantiation for tiles %dx%d nj %d", p.tr, p.tc, p.nj);
  int rc = check_launch("single-tap weight-gradient kernel");
  if (rc) return rc;
  ReduceArgs r;
  memset(&r, 0, sizeof r);
  r.part = a.part;
  r.dbpart = a.dbpart;
  r.dw = dw;
  r.db = db;
  r.nsplit = a.nsplit;
  r.Fc = a.Fc;
  r.Gc = a.Gc;
  r.taps = p.taps;
  r.Fpad = a.Fc;
  r.Gpad = a.Gc;
  r.dw_dtype = dw_dtype;
  r.db_dtype = db_dtype;
  r.db_mode = a.db_mode;
  {
    TimedLaunch tr(KIND_REDUCE, s);
    launch_wgrad_reduce(r, s);
    tr.end();
  }
  return check_launch("weight-gradient reduce");
}

// Why a weight-gradient plan cannot run (nullptr: it can); shared with the
// workspace query.
// dW partials of the k=1 skinny kernel: one split per 512 position groups
// (two per thread, loaded together), at most 4096.
void plan_skinny_dw(const r3c_conv_desc* d, WgPlan& p) {
  const SkinnyArgs s = skinny_args(d);
  const int64_t nsplit = std::max<int64_t>(1, std::min<int64_t>(4096, cdiv(s.ngroups, 512)));
  p.a.nsplit = (int32_t)nsplit;
  p.taps = 1;
  p.part_bytes = align256(nsplit * (int64_t)s.O * s.C * 4);
  p.dbpart_bytes = align256(nsplit * (int64_t)s.O * 4);
  p.fcopy_bytes = p.gcopy_bytes = 0;
}

// dW partials of the one-channel k=3 kernel: one per workgroup.
void plan_stem_dw(const r3c_conv_desc* d, WgPlan& p) {
  const StemArgs s = stem_args(d);
  p.a.nsplit = s.nsplit;
  p.taps = 27;
  p.part_bytes = align256((int64_t)s.nsplit * s.Cout * 27 * 4);
  p.dbpart_bytes = align256((int64_t)s.nsplit * s.Cout * 4);
  p.fcopy_bytes = p.gcopy_bytes = 0;
}

const char* wgrad_plan_reject(const WgPlan& p) {
  if ((int64_t)p.lds > kMaxLds) return "the tile needs more LDS than a compute unit has";
  if (!p.pw && (p.a.f_bytes == 0 || p.a.g_bytes == 0))  // the register-direct plan checks its own
    return "one sample exceeds 1 GiB (32-bit buffer offsets)";
  return nullptr;
}

int64_t wgrad_plan_ws(const WgPlan& p) {
  return p.part_bytes + p.dbpart_bytes + p.fcopy_bytes + p.gcopy_bytes;
}

int run_wgrad(const r3c_conv_desc* d, bool transpose, const void* x, const void* dy, void* dw, int dw_dtype, void* db,
              int db_dtype, void* ws, int64_t ws_bytes, void* stream, const CatSpec* cat = nullptr) {
  // The register-direct single-tap kernel loads 16-byte vectors; other
  // alignments take the LDS-staged kernel, which stages any alignment.
  const bool al16 = ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(dy)) & 15) == 0;
  // Dedicated kernels: k=1 with at most 4 output channels (skinny), k=3 with
  // one input channel (stem).  Both write fp32 partials [split][Cout][taps][Cin]
  // (+ db partials [split][Cout]) for the split-ordered reduce.
  const bool skinny = !cat && !transpose && skinny_ok(d) && al16;
  const bool stem = !cat && !transpose && !skinny && stem_ok(d, true) && al16;
  if ((skinny || stem) && x && dy && dw && ws) {
    WgPlan p;
    if (stem) plan_stem_dw(d, p);
    else plan_skinny_dw(d, p);
    const int64_t need = wgrad_plan_ws(p);
    if (ws_bytes < need)
      return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
    if (dw_dtype != R3C_F32 && dw_dtype != d->dtype) return fail(R3C_INVALID, "dw_dtype must be fp32 or the input dtype");
    if (db && db_dtype != R3C_F32 && db_dtype != R3C_F16 && db_dtype != R3C_BF16)
      return fail(R3C_INVALID, "db_dtype must be fp32, fp16 or bf16");
    int rc = check_device();
    if (rc) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    float* part = static_cast<float*>(ws);
    float* dbpart = reinterpret_cast<float*>(static_cast<char*>(ws) + p.part_bytes);
    {
      TimedLaunch tl(KIND_WGRAD, s);
      bool launched;
      if (stem) {
        StemArgs a = stem_args(d);
        a.x = static_cast<const uint16_t*>(x);
        a.dy = static_cast<const uint16_t*>(dy);
        a.part = part;
        a.dbpart = db ? dbpart : nullptr;
        a.nsplit = p.a.nsplit;
        launched = launch_stem(d->dtype, 2, a, stem_lds(a, true), s);
      } else {
        SkinnyArgs a = skinny_args(d);
        a.x = const_cast<uint16_t*>(static_cast<const uint16_t*>(x));
        a.y = const_cast<uint16_t*>(static_cast<const uint16_t*>(dy));
        a.part = part;
        a.dbpart = db ? dbpart : nullptr;
        a.nsplit = p.a.nsplit;
        launched = launch_skinny(d->dtype, 2, a, s);
      }
      tl.end();
      if (!launched) return fail(R3C_UNSUPPORTED, "no dedicated dW instantiation for %d output channels", d->cout);
    }
    rc = check_launch(stem ? "one-channel k=3 dW" : "k=1 skinny dW");
    if (rc) return rc;
    ReduceArgs r;
    memset(&r, 0, sizeof r);
    r.part = part;
    r.dbpart = dbpart;
    r.dw = dw;
    r.db = db;
    r.nsplit = p.a.nsplit;
    r.Fc = d->cout;
    r.Gc = d->cin;
    r.taps = p.taps;
    r.Fpad = d->cout;
    r.Gpad = d->cin;
    r.dw_dtype = dw_dtype;
    r.db_dtype = db_dtype;
    r.db_mode = db ? 1 : 0;
    {
      TimedLaunch tr(KIND_REDUCE, s);
      launch_wgrad_reduce(r, s);
      tr.end();
    }
    return check_launch("weight-gradient reduce");
  }
  WgPlan p;
  plan_wgrad(d, transpose, p, al16, al16, cat ? cat->ca : 0);  // unaligned: no copies either (same or less workspace)
  if (cat && (p.fl != 5 || !aligned16_all({x, dy, cat->xb})))
    return fail(R3C_UNSUPPORTED, "no weight-gradient plan for this channel concatenation");
  if (const char* why = wgrad_plan_reject(p)) return fail(R3C_UNSUPPORTED, "%s", why);
  const int64_t need = wgrad_plan_ws(p);
  if (ws_bytes < need)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
  if (!x || !dy || !dw || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  if (dw_dtype != R3C_F32 && dw_dtype != d->dtype) return fail(R3C_INVALID, "dw_dtype must be fp32 or the input dtype");
  if (db && db_dtype != R3C_F32 && db_dtype != R3C_F16 && db_dtype != R3C_BF16)
    return fail(R3C_INVALID, "db_dtype must be fp32, fp16 or bf16");
  int rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.pw) return run_pwdw(d, transpose, p, x, dy, dw, dw_dtype, db, db_dtype, ws, s);
  WgArgs a = p.a;
  a.fsrc = static_cast<const uint16_t*>(transpose ? x : dy);
  a.gsrc = static_cast<const uint16_t*>(transpose ? dy : x);
  if (cat) {
    a.gsrc2 = static_cast<const uint16_t*>(cat->xb);
    a.gs0_2 = cat->xb_s0;
    a.gsplit = cat->ca;
    a.g_bytes = (uint32_t)(2 * (int64_t)cat->ca * a.gs[1]);
    a.g2_bytes = (uint32_t)(2 * (int64_t)(d->cin - cat->ca) * a.gs[1]);
  }
  {
    char* copies = static_cast<char*>(ws) + p.part_bytes + p.dbpart_bytes;
    if (p.fcopy_bytes) {
      rc = copy_to_channels_last(a.fsrc, copies, d->n, a.Fc, a.Rd, a.Rh, a.Rw, s);
      if (rc) return rc;
      a.fsrc = reinterpret_cast<const uint16_t*>(copies);
    }
    if (p.gcopy_bytes) {
      rc = copy_to_channels_last(a.gsrc, copies + p.fcopy_bytes, d->n, a.Gc, a.Gd, a.Gh, a.Gw, s);
      if (rc) return rc;
      a.gsrc = reinterpret_cast<const uint16_t*>(copies + p.fcopy_bytes);
    }
  }
  a.part = static_cast<float*>(ws);
  a.dbpart = reinterpret_cast<float*>(static_cast<char*>(ws) + p.part_bytes);
  // Channel-major staging needs 16-byte aligned sources; G (and F when not
  // channel-major) use 16-byte channel vectors when both allow, else 8 scalar
  // loads per slot.
  const bool f16b = (reinterpret_cast<uintptr_t>(a.fsrc) & 15) == 0;
  const bool g16b = (reinterpret_cast<uintptr_t>(a.gsrc) & 15) == 0;
  // fl 3 needs both sources 16-byte aligned; otherwise G falls back to scalar
  // staging (correct for any strides, slower).
  if (p.fl == 5) {
    // Planned only for 16-byte aligned sources (allow_copy).
    if (!f16b || !g16b) return fail(R3C_INVALID, "internal: row-walking weight gradient planned for unaligned sources");
    a.db_mode = db ? 1 : 0;
    TimedLaunch tl(KIND_WGRAD, s);
    const bool launched = launch_wgrow(d->dtype, a.GCW, a.Rw, a, s);
    tl.end();
    if (!launched) return fail(R3C_UNSUPPORTED, "no row-walking weight-gradient instantiation for %d channels", a.GCW);
  } else {
  const int fl = (p.fl == 3 && f16b && g16b) ? 3 : (p.fl == 2 && f16b && g16b) ? 2 : ((p.fl && f16b) ? 1 : 0);
  const bool g_ok = vec16_ok(a.gsrc, a.gs) && a.Gc % 8 == 0;
  const int cl = fl == 3 ? 0 : fl == 2 ? 1 : ((g_ok && (fl || (vec16_ok(a.fsrc, a.fs) && a.Fc % 8 == 0))) ? 1 : 0);
  // fl 3 stages 18 * GCW G items per box: one per thread, plus 64 more in one
  // wave when CBW = 4.
  if (fl == 3 && 18 * a.GCW > WgGeom<MODE_K3>::THREADS + (p.cbw == 4 ? 64 : 0))
    return fail(R3C_INVALID, "internal: %d G staging items exceed the kernel's capacity", 18 * a.GCW);
  a.db_mode = db ? (transpose ? 2 : 1) : 0;
  TimedLaunch tl(KIND_WGRAD, s);
  const bool launched = launch_wgrad(d->dtype, p.mode, p.cbw, cl, fl, a, p.lds, s);
  tl.end();
  if (!launched) return fail(R3C_UNSUPPORTED, "no weight-gradient instantiation for mode %d cbw %d", p.mode, p.cbw);
  }
  rc = check_launch("weight-gradient kernel");
  if (rc) return rc;
  ReduceArgs r;
  memset(&r, 0, sizeof r);
  r.part = a.part;
  r.dbpart = a.dbpart;
  r.dw = dw;
  r.db = db;
  r.nsplit = a.nsplit;
  r.Fc = a.Fc;
  r.Gc = a.Gc;
  r.taps = p.taps;
  r.Fpad = a.Fpad;
  r.Gpad = a.Gpad;
  r.dw_dtype = dw_dtype;
  r.db_dtype = db_dtype;
  r.db_mode = a.db_mode;
  {
    TimedLaunch tr(KIND_REDUCE, s);
    launch_wgrad_reduce(r, s);
    tr.end();
  }
  return check_launch("weight-gradient reduce");
}

// Workspace queries: -1 when the descriptor is invalid or no plan can run it
// (the caller then falls back).  The size covers every plan the launch may
// take for this descriptor, whatever the pointers' alignment.
// ---------------------------------------------------------------------------
// BatchNorm + ReLU
// ---------------------------------------------------------------------------
int bn_validate(const r3c_bn_desc* d) {
  if (!d) return fail(R3C_INVALID, "descriptor is NULL");
  if (d->dtype != R3C_F16 && d->dtype != R3C_BF16 && d->dtype != R3C_F32)
    return fail(R3C_UNSUPPORTED, "BatchNorm: dtype %d is not fp16, bf16 or fp32", d->dtype);
  if (d->n < 1 || d->c < 1 || d->s < 1) return fail(R3C_INVALID, "BatchNorm: every dimension must be >= 1");
  if (d->n > 65535 || d->c > 65535) return fail(R3C_UNSUPPORTED, "BatchNorm: n and c must be <= 65535");
  const int vec = d->dtype == R3C_F32 ? 4 : 8;
  if (d->s % vec) return fail(R3C_UNSUPPORTED, "BatchNorm: positions per plane must be a multiple of %d", vec);
  const int64_t* st[3] = {d->y_strides, d->g_strides, d->o_strides};
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 2; ++j)
      if (st[i][j] < 0 || st[i][j] % vec) return fail(R3C_UNSUPPORTED, "BatchNorm: strides must be multiples of %d", vec);
  if ((d->s + kBnChunk - 1) / kBnChunk >= (1ll << 31)) return fail(R3C_UNSUPPORTED, "BatchNorm: plane too large");
  return R3C_OK;
}

int64_t bn_ws(const r3c_bn_desc* d) {
  const int64_t nchunk = (d->s + kBnChunk - 1) / kBnChunk;
  return align256((int64_t)d->n * nchunk * d->c * 2 * 4) + align256((int64_t)d->c * 4 * 4);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

BnArgs bn_args(const r3c_bn_desc* d, void* ws) {
  BnArgs a;
  memset(&a, 0, sizeof a);
  a.S = d->s;
  a.N = d->n;
  a.C = d->c;
  a.nchunk = (int32_t)((d->s + kBnChunk - 1) / kBnChunk);
  a.training = d->training ? 1 : 0;
  a.eps = d->eps;
  a.momentum = d->momentum;
  a.sn = d->y_strides[0];
  a.sc = d->y_strides[1];
  a.gn = d->g_strides[0];
  a.gc = d->g_strides[1];
  a.on = d->o_strides[0];
  a.oc = d->o_strides[1];
  a.part = static_cast<float*>(ws);
  a.coef = reinterpret_cast<float*>(static_cast<char*>(ws) + align256((int64_t)d->n * a.nchunk * d->c * 2 * 4));
  return a;
}

// ---------------------------------------------------------------------------
// MaxPool3d(2)
// ---------------------------------------------------------------------------
int pool_setup(const r3c_pool_desc* d, PoolArgs& a) {
  if (!d) return fail(R3C_INVALID, "descriptor is NULL");
  if (d->dtype != R3C_F16 && d->dtype != R3C_BF16 && d->dtype != R3C_F32)
    return fail(R3C_UNSUPPORTED, "MaxPool3d: dtype %d is not fp16, bf16 or fp32", d->dtype);
  if (d->n < 1 || d->c < 1 || d->d < 2 || d->h < 2 || d->w < 8) return fail(R3C_UNSUPPORTED, "MaxPool3d: too small");
  if (d->d % 2 || d->h % 2 || d->w % 8) return fail(R3C_UNSUPPORTED, "MaxPool3d: d, h must be even and w a multiple of 8");
  // x / dx move as 16-byte vectors of 8 (fp32: 4) elements, y / dy as 4 elements.
  const int vec = d->dtype == R3C_F32 ? 4 : 8;
  for (int j = 0; j < 2; ++j) {
    if (d->x_strides[j] < 0 || d->x_strides[j] % vec)
      return fail(R3C_UNSUPPORTED, "MaxPool3d: x strides must be multiples of %d", vec);
    if (d->y_strides[j] < 0 || d->y_strides[j] % 4)
      return fail(R3C_UNSUPPORTED, "MaxPool3d: y strides must be multiples of 4");
  }
  memset(&a, 0, sizeof a);
  a.n = d->n;
  a.c = d->c;
  a.d = d->d;
  a.h = d->h;
  a.w = d->w;
  a.od = d->d / 2;
  a.oh = d->h / 2;
  a.ow = d->w / 2;
  a.xs0 = d->x_strides[0];
  a.xs1 = d->x_strides[1];
  a.ys0 = d->y_strides[0];
  a.ys1 = d->y_strides[1];
  if ((int64_t)a.n * a.c * a.od * a.oh * (a.ow / 4) >= (1ll << 31))
    return fail(R3C_UNSUPPORTED, "MaxPool3d: more than 2^31 threads");
  return R3C_OK;
}

int64_t fwd_ws(const r3c_conv_desc* d, int op, bool transpose) {
  if (validate(d, transpose) != R3C_OK) return -1;
  RowPlan p;
  plan_row(d, op, p);
  if (row_plan_reject(p)) return -1;
  int64_t need = row_plan_ws(p);
  if (op == OP_T2_DX) {
    T2dxPlan tp;
    if (plan_t2dx(d, tp)) need = std::max<int64_t>(need, align256(tp.wpk_bytes));
  }
  return need;
}

int64_t wgrad_ws(const r3c_conv_desc* d, bool transpose) {
  if (validate(d, transpose) != R3C_OK) return -1;
  WgPlan p;
  plan_wgrad(d, transpose, p, false);
  if (wgrad_plan_reject(p)) return -1;
  int64_t need = wgrad_plan_ws(p);
  WgPlan q;
  plan_wgrad(d, transpose, q, true);
  if (q.pw) need = std::max<int64_t>(need, wgrad_plan_ws(q));
  if (!transpose && skinny_ok(d)) {
    WgPlan k;
    plan_skinny_dw(d, k);
    need = std::max<int64_t>(need, wgrad_plan_ws(k));
  }
  if (!transpose && stem_ok(d, true)) {
    WgPlan k;
    plan_stem_dw(d, k);
    need = std::max<int64_t>(need, wgrad_plan_ws(k));
  }
  // Unaligned sources take the plan without copies or the kw-shift kernel.
  WgPlan u;
  plan_wgrad(d, transpose, u, false, false);
  if (!wgrad_plan_reject(u)) need = std::max<int64_t>(need, wgrad_plan_ws(u));
  return need;
}

// ---------------------------------------------------------------------------
// Conv3d with stride > 1 (r3c_strided.hip)
// ---------------------------------------------------------------------------
struct StridedPlan {
  StridedArgs a;
  StridedPackArgs pk;
  int nb;
  int64_t wpk_bytes;
  int64_t copy_bytes;  // > 0: the NCDHW source is first copied to NDHWC (16-byte fragment loads)
};

// Forward (dx false) or dX of a strided Conv3d: wave tiles of 32 destination
// positions along w (dX: of one residue class of w modulo the stride) and up
// to 4 column blocks of 32 destination channels.
void plan_strided(const r3c_conv_desc* d, const int32_t* st, bool dx, StridedPlan& p) {
  StridedArgs& a = p.a;
  memset(&a, 0, sizeof a);
  a.k = d->kernel;
  a.taps = d->kernel == 3 ? 27 : 1;
  a.pd = d->pad_d;
  a.ph = d->pad_h;
  a.pw = d->pad_w;
  a.sd = st[0];
  a.sh = st[1];
  a.sw = st[2];
  a.dx = dx ? 1 : 0;
  const int64_t* ss = dx ? d->y_strides : d->x_strides;
  const int64_t* sdst = dx ? d->x_strides : d->y_strides;
  for (int i = 0; i < 5; ++i) {
    a.ss[i] = ss[i];
    a.sd5[i] = sdst[i];
  }
  a.Cs = dx ? d->cout : d->cin;
  a.Cd = dx ? d->cin : d->cout;
  a.Sd = dx ? d->od : d->d;
  a.Sh = dx ? d->oh : d->h;
  a.Sw = dx ? d->ow : d->w;
  a.Rd = dx ? d->d : d->od;
  a.Rh = dx ? d->h : d->oh;
  a.Rw = dx ? d->w : d->ow;
  const int ncb = cdiv(a.Cd, 32);
  p.nb = std::min(ncb, 4);
  a.n_ctiles = cdiv(ncb, p.nb);
  a.nbt = a.n_ctiles * p.nb;
  a.nc16 = cdiv(a.Cs, 16);
  a.mb = 1;
  a.nwb = dx ? cdiv(cdiv(a.Rw, a.sw), 32) : cdiv(a.Rw, 32);
  a.ntiles = (int64_t)d->n * a.Rd * a.Rh * (dx ? a.sw : 1) * a.nwb * a.n_ctiles;
  a.scl = ss[1] == 1 && a.Cs % 8 == 0 && ss[0] % 8 == 0 && ss[2] % 8 == 0 && ss[3] % 8 == 0 && ss[4] % 8 == 0;
  a.dvec4 = sdst[1] == 1 && a.Cd % 4 == 0 && sdst[0] % 4 == 0 && sdst[2] % 4 == 0 && sdst[3] % 4 == 0 &&
            sdst[4] % 4 == 0;
  StridedPackArgs& k = p.pk;
  memset(&k, 0, sizeof k);
  k.cin = d->cin;
  k.cout = d->cout;
  k.taps = a.taps;
  k.nbt = a.nbt;
  k.dx = a.dx;
  k.total = (int64_t)a.nc16 * a.taps * a.nbt * 64;
  p.wpk_bytes = align256(k.total * 16);
  p.copy_bytes = !a.scl && ncdhw_copyable(ss, a.Cs, a.Sd, a.Sh, a.Sw)
                     ? align256(tensor_bytes(d->n, a.Cs, a.Sd, a.Sh, a.Sw))
                     : 0;
  // Forward, k = 3, w stride 1 or 2, an NCDHW source (w-contiguous rows of a
  // multiple of 8, at most 32 channels) and at most two column blocks: the
  // row-segment kernel reads the source in place, no NDHWC copy (with an
  // unaligned source the run falls back to 2-byte gathers, also without it).
  if (!dx && a.k == 3 && !a.scl && (a.sw == 1 || a.sw == 2) && p.nb <= 2 && a.Cs % 8 == 0 && a.Cs <= 32 &&
      ss[4] == 1 && a.Sw % 8 == 0 && ss[3] % 8 == 0 && ss[2] % 8 == 0 && ss[1] % 8 == 0 && ss[0] % 8 == 0 &&
      (int64_t)(a.Cs - 1) * ss[1] + a.Sw < (1ll << 31)) {
    a.chan_first = a.Cs / 8;
    p.copy_bytes = 0;
  }
}

int run_strided(const r3c_conv_desc* d, const int32_t* st, bool dx, const void* src, const void* w, const void* bias,
                void* dst, void* ws, int64_t ws_bytes, void* stream) {
  int rc = validate(d, false, st);
  if (rc) return rc;
  StridedPlan p;
  plan_strided(d, st, dx, p);
  if (p.a.ntiles / 4 >= (1ll << 31)) return fail(R3C_UNSUPPORTED, "strided Conv3d: too many output tiles");
  if (p.copy_bytes && (reinterpret_cast<uintptr_t>(src) & 15)) p.copy_bytes = 0;  // unaligned: 2-byte loads
  if (p.a.chan_first && (reinterpret_cast<uintptr_t>(src) & 15)) p.a.chan_first = 0;  // unaligned: 2-byte loads
  const int64_t need = p.wpk_bytes + p.copy_bytes;
  if (ws_bytes < need)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
  if (!src || !w || !dst || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  p.pk.w = static_cast<const uint16_t*>(w);
  p.pk.out = static_cast<uint16_t*>(ws);
  {
    TimedLaunch tl(KIND_PACK, s);
    launch_strided_pack(p.pk, s);
    tl.end();
  }
  rc = check_launch("strided Conv3d weight pack");
  if (rc) return rc;
  StridedArgs& a = p.a;
  a.src = static_cast<const uint16_t*>(src);
  if (p.copy_bytes) {
    void* cl = static_cast<char*>(ws) + p.wpk_bytes;
    rc = copy_to_channels_last(src, cl, d->n, a.Cs, a.Sd, a.Sh, a.Sw, s);
    if (rc) return rc;
    a.src = static_cast<const uint16_t*>(cl);
    channels_last_strides(a.ss, a.Cs, a.Sd, a.Sh, a.Sw);
    a.scl = 1;
  }
  a.wpk = static_cast<const uint16_t*>(ws);
  a.b = dx ? nullptr : static_cast<const uint16_t*>(bias);
  a.dst = static_cast<uint16_t*>(dst);
  a.scl = a.scl && (reinterpret_cast<uintptr_t>(src) & 15) == 0;
  a.dvec4 = a.dvec4 && (reinterpret_cast<uintptr_t>(dst) & 7) == 0;
  // Two blocks of 32 positions per wave (one weight fragment feeds two MFMAs)
  // when the fragments are 16-byte loads, at most 2 column blocks (3 waves per
  // SIMD; more blocks leave 1-2) and at least 8 workgroups per CU remain.
  {
    const int64_t per_w = (dx ? cdiv(a.Rw, a.sw) : a.Rw);
    const int nwb2 = (int)cdiv(per_w, 64);
    const int64_t nt2 = a.ntiles / a.nwb * nwb2;
    // (an NCDHW forward source of 4 channel groups with 2 column blocks keeps
    // one block: two would spill registers)
    const bool cf_spill = !dx && a.chan_first == 4 && p.nb == 2;
    if ((a.scl || a.chan_first) && p.nb <= 2 && !cf_spill && (nt2 + 3) / 4 >= 8ll * kNumCUs) {
      a.mb = 2;
      a.nwb = nwb2;
      a.ntiles = nt2;
    }
  }
  a.dtile = !dx && a.n_ctiles == 1 && a.sd5[1] == 1 && a.sd5[4] == a.Cd && a.Cd % 8 == 0 && a.sd5[0] % 8 == 0 &&
            a.sd5[2] % 8 == 0 && a.sd5[3] % 8 == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
  // Forward with k = 3, w stride 1 or 2, at most 32 source channels and two
  // column blocks: the x operand through per-wave LDS row segments.
  // dX likewise with dY row segments (at most 64 dY channels).
  const bool seg_ok = a.k == 3 && a.scl && (a.sw == 1 || a.sw == 2) && p.nb <= 2 &&
                      (int64_t)a.Sw * a.ss[4] < (1ll << 31);
  const bool rs = (seg_ok || a.chan_first) && !dx && a.nc16 <= 2;
  const bool dxrs = seg_ok && dx && a.nc16 <= 4;
  TimedLaunch tl(KIND_ROW, s);
  const bool launched = rs     ? launch_strided_fwd_rs(d->dtype, p.nb, a, s)
                        : dxrs ? launch_strided_dx_rs(d->dtype, p.nb, a, s)
                               : launch_strided(d->dtype, p.nb, a, s);
  tl.end();
  if (!launched) return fail(R3C_UNSUPPORTED, "strided Conv3d: no instantiation for %d column blocks", p.nb);
  return check_launch(dx ? "strided Conv3d dX" : "strided Conv3d forward");
}

// The stride-1 convolution whose output grid holds the strided one at
// multiples of the stride: same input, padding and kernel; dY NCDHW with rows
// padded to a multiple of 8 elements.
void stride1_desc(const r3c_conv_desc* d, r3c_conv_desc& d1) {
  d1 = *d;
  d1.od = d->d + 2 * d->pad_d - d->kernel + 1;
  d1.oh = d->h + 2 * d->pad_h - d->kernel + 1;
  d1.ow = d->w + 2 * d->pad_w - d->kernel + 1;
  // Rows padded to a multiple of 8 elements (16-byte stores of the scatter).
  const int64_t wp = (d1.ow + 7) / 8 * 8;
  const int64_t S1 = (int64_t)d1.od * d1.oh * wp;
  d1.y_strides[0] = (int64_t)d->cout * S1;
  d1.y_strides[1] = S1;
  d1.y_strides[2] = (int64_t)d1.oh * wp;
  d1.y_strides[3] = wp;
  d1.y_strides[4] = 1;
}

int64_t dilated_bytes(const r3c_conv_desc& d1) { return align256((int64_t)d1.n * d1.y_strides[0] * 2); }

// Direct strided dW (r3c_strided.hip, strided_dw_kernel): k = 3, w stride 1
// or 2 with w padding 1, w-contiguous x and dY with 16-byte aligned rows,
// W % 8 == 0 and OW % 16 == 0 (pointer alignment is the caller's check).
struct StridedDwPlan {
  StridedDwArgs a;
  int sw, ncb;
  int64_t part_bytes, dbpart_bytes;
};
bool plan_strided_dw(const r3c_conv_desc* d, const int32_t* st, StridedDwPlan& p) {
  const int64_t* xs = d->x_strides;
  const int64_t* ys = d->y_strides;
  if (d->kernel != 3 || (st[2] != 1 && st[2] != 2) || d->pad_w != 1 || d->w % 8 || d->ow % 16) return false;
  if (xs[4] != 1 || xs[3] % 8 || xs[2] % 8 || xs[1] % 8 || xs[0] % 8) return false;
  if (ys[4] != 1 || ys[3] % 8 || ys[2] % 8 || ys[1] % 8 || ys[0] % 8) return false;
  StridedDwArgs& a = p.a;
  memset(&a, 0, sizeof a);
  a.xs0 = xs[0];
  a.xs1 = xs[1];
  a.xs2 = xs[2];
  a.xs3 = xs[3];
  a.ys0 = ys[0];
  a.ys1 = ys[1];
  a.ys2 = ys[2];
  a.ys3 = ys[3];
  a.Cin = d->cin;
  a.Cout = d->cout;
  a.D = d->d;
  a.H = d->h;
  a.W = d->w;
  a.OD = d->od;
  a.OH = d->oh;
  a.OW = d->ow;
  a.pd = d->pad_d;
  a.ph = d->pad_h;
  a.pw = d->pad_w;
  a.sd = st[0];
  a.sh = st[1];
  p.sw = st[2];
  p.ncb = d->cout > 32 ? 2 : 1;  // Cout blocks per wave: x fragments serve two MFMAs
  a.ncg = cdiv(d->cout, 32 * p.ncb);
  a.ngb = cdiv(d->cin, 32);
  a.nkb = (int64_t)d->n * d->od * d->oh * (d->ow / 16);
  // One workgroup (9 waves of 100-152 VGPRs: one fits a CU) per CU, at
  // least 4 K blocks each, partials within kMaxPartialBytes.
  const int64_t tiles = (int64_t)a.ncg * a.ngb;
  const int64_t per_split = (int64_t)d->cout * 27 * d->cin * 4;
  int64_t ns = std::max<int64_t>(1, kNumCUs / tiles);
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, a.nkb / 4));
  ns = std::min<int64_t>(ns, std::max<int64_t>(1, kMaxPartialBytes / per_split));
  a.nsplit = (int32_t)ns;
  p.part_bytes = align256(ns * per_split);
  p.dbpart_bytes = align256(ns * d->cout * 4);
  return true;
}

// Dense NDHWC x and dY whose NCDHW copies the direct dW kernel takes: d2 is
// the descriptor of the copies, xc / yc their workspace bytes.
bool plan_strided_dw_copies(const r3c_conv_desc* d, const int32_t* st, r3c_conv_desc& d2, StridedDwPlan& p,
                            int64_t& xc, int64_t& yc) {
  if (!ndhwc_copyable(d->x_strides, d->cin, d->d, d->h, d->w) ||
      !ndhwc_copyable(d->y_strides, d->cout, d->od, d->oh, d->ow))
    return false;
  d2 = *d;
  channels_first_strides(d2.x_strides, d->cin, d->d, d->h, d->w);
  channels_first_strides(d2.y_strides, d->cout, d->od, d->oh, d->ow);
  if (!plan_strided_dw(&d2, st, p)) return false;
  xc = align256(tensor_bytes(d->n, d->cin, d->d, d->h, d->w));
  yc = align256(tensor_bytes(d->n, d->cout, d->od, d->oh, d->ow));
  return true;
}

int run_strided_dw(const r3c_conv_desc* d, const int32_t* st, const void* x, const void* dy, void* dw, int dw_dtype,
                   void* db, int db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  int rc = validate(d, false, st);
  if (rc) return rc;
  StridedDwPlan dp;
  r3c_conv_desc d2;
  int64_t xc = 0, yc = 0;
  const bool aligned = aligned16_all({x, dy});
  const bool direct = aligned && plan_strided_dw(d, st, dp);
  const bool copies = aligned && !direct && plan_strided_dw_copies(d, st, d2, dp, xc, yc);
  if (direct || copies) {
    const int64_t need = xc + yc + dp.part_bytes + dp.dbpart_bytes;
    if (ws_bytes < need)
      return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)need);
    if (!x || !dy || !dw || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
    if (dw_dtype != R3C_F32 && dw_dtype != d->dtype) return fail(R3C_INVALID, "dw_dtype must be fp32 or the input dtype");
    if (db && db_dtype != R3C_F32 && db_dtype != R3C_F16 && db_dtype != R3C_BF16)
      return fail(R3C_INVALID, "db_dtype must be fp32, fp16 or bf16");
    rc = check_device();
    if (rc) return rc;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    StridedDwArgs& a = dp.a;
    a.x = static_cast<const uint16_t*>(x);
    a.dy = static_cast<const uint16_t*>(dy);
    char* wsp = static_cast<char*>(ws);
    if (copies) {  // NDHWC operands: NCDHW copies in the workspace first
      rc = copy_to_channels_first(x, wsp, d->n, d->cin, d->d, d->h, d->w, s);
      if (rc) return rc;
      rc = copy_to_channels_first(dy, wsp + xc, d->n, d->cout, d->od, d->oh, d->ow, s);
      if (rc) return rc;
      a.x = reinterpret_cast<const uint16_t*>(wsp);
      a.dy = reinterpret_cast<const uint16_t*>(wsp + xc);
      wsp += xc + yc;
    }
    a.part = reinterpret_cast<float*>(wsp);
    float* dbpart = reinterpret_cast<float*>(wsp + dp.part_bytes);
    a.dbpart = db ? dbpart : nullptr;
    {
      TimedLaunch tl(KIND_WGRAD, s);
      const bool launched = launch_strided_dw(d->dtype, dp.sw, dp.ncb, a, s);
      tl.end();
      if (!launched) return fail(R3C_UNSUPPORTED, "strided dW: no kernel for w stride %d", dp.sw);
    }
    rc = check_launch("strided Conv3d dW");
    if (rc) return rc;
    ReduceArgs r;
    memset(&r, 0, sizeof r);
    r.part = a.part;
    r.dbpart = dbpart;
    r.dw = dw;
    r.db = db;
    r.nsplit = a.nsplit;
    r.Fc = d->cout;
    r.Gc = d->cin;
    r.taps = 27;
    r.Fpad = d->cout;
    r.Gpad = d->cin;
    r.dw_dtype = dw_dtype;
    r.db_dtype = db_dtype;
    r.db_mode = db ? 1 : 0;
    {
      TimedLaunch tr(KIND_REDUCE, s);
      launch_wgrad_reduce(r, s);
      tr.end();
    }
    return check_launch("weight-gradient reduce");
  }
  r3c_conv_desc d1;
  stride1_desc(d, d1);
  const int64_t dil = dilated_bytes(d1);
  if (ws_bytes < dil)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)dil);
  if (!x || !dy || !dw || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  DilateArgs a;
  memset(&a, 0, sizeof a);
  a.src = static_cast<const uint16_t*>(dy);
  a.dst = static_cast<uint16_t*>(ws);
  for (int i = 0; i < 5; ++i) a.ys[i] = d->y_strides[i];
  a.C = d->cout;
  a.D1 = d1.od;
  a.H1 = d1.oh;
  a.W1 = d1.ow;
  a.W1p = (int32_t)d1.y_strides[3];
  a.sd = st[0];
  a.sh = st[1];
  a.sw = st[2];
  a.rows = (int64_t)d1.n * d->cout * d1.od * d1.oh;
  {
    TimedLaunch tl(KIND_LAYOUT, s);
    launch_dilate(a, s);
    tl.end();
  }
  rc = check_launch("strided Conv3d dY scatter");
  if (rc) return rc;
  return run_wgrad(&d1, false, x, ws, dw, dw_dtype, db, db_dtype, static_cast<char*>(ws) + dil, ws_bytes - dil,
                   stream);
}

std::mutex g_dev_mu;
std::unordered_map<int, int> g_dev_ok;

// Device address of `scratch` (below) on each device, looked up once per
// device with that device current: every GPU holds its own copy of the array.
std::mutex g_scratch_mu;
std::unordered_map<int, void*> g_scratch_ptr;

}  // namespace

// Workspace of the allocation-free dW entry point r3c_conv3d_dw_static: a
// file-scope device array, resident on every GPU the library runs on until the
// process ends.  In host code `scratch` names a host-side stand-in, never a
// device address: only the pointer from hipGetSymbolAddress is passed on.
constexpr int64_t kStaticScratchBytes = 64ll << 20;
static __device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

namespace {

int static_scratch(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(R3C_HIP_ERROR, "hipGetDevice failed");
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  auto it = g_scratch_ptr.find(dev);
  if (it == g_scratch_ptr.end()) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return fail(R3C_HIP_ERROR, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    it = g_scratch_ptr.emplace(dev, ptr).first;
  }
  *out = it->second;
  return R3C_OK;
}

}  // namespace
}  // namespace r3c

using namespace r3c;

extern "C" {

int32_t r3c_abi_version(void) { return R3C_ABI_VERSION; }

const char* r3c_last_error(void) { return g_err.c_str(); }

int32_t r3c_device_supported(int32_t device) {
  std::lock_guard<std::mutex> lk(g_dev_mu);
  auto it = g_dev_ok.find(device);
  if (it != g_dev_ok.end()) return it->second;
  hipDeviceProp_t prop;
  int v = 0;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) v = strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  g_dev_ok[device] = v;
  return v;
}

int64_t r3c_conv3d_fwd_workspace(const r3c_conv_desc* d) { return fwd_ws(d, OP_CONV_FWD, false); }
int64_t r3c_conv3d_dx_workspace(const r3c_conv_desc* d) { return fwd_ws(d, OP_CONV_DX, false); }
int64_t r3c_conv3d_dw_workspace(const r3c_conv_desc* d) { return wgrad_ws(d, false); }
int64_t r3c_convt_k2s2_fwd_workspace(const r3c_conv_desc* d) { return fwd_ws(d, OP_T2_FWD, true); }
int64_t r3c_convt_k2s2_dx_workspace(const r3c_conv_desc* d) { return fwd_ws(d, OP_T2_DX, true); }
int64_t r3c_convt_k2s2_dw_workspace(const r3c_conv_desc* d) { return wgrad_ws(d, true); }

int32_t r3c_conv3d_fwd(const r3c_conv_desc* d, const void* x, const void* w, const void* bias, void* y, void* ws,
                       int64_t ws_bytes, void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  return run_row(d, OP_CONV_FWD, x, w, bias, y, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_dx(const r3c_conv_desc* d, const void* dy, const void* w, void* dx, void* ws, int64_t ws_bytes,
                      void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  return run_row(d, OP_CONV_DX, dy, w, nullptr, dx, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_dw(const r3c_conv_desc* d, const void* x, const void* dy, void* dw, int32_t dw_dtype, void* db,
                      int32_t db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  return run_wgrad(d, false, x, dy, dw, dw_dtype, db, db_dtype, ws, ws_bytes, stream);
}

int64_t r3c_conv3d_strided_workspace(const r3c_conv_desc* d, const int32_t* stride, int32_t pass) {
  if (!stride || validate(d, false, stride) != R3C_OK) return -1;
  if (pass == 0 || pass == 1) {
    StridedPlan p;
    plan_strided(d, stride, pass == 1, p);
    return p.wpk_bytes + p.copy_bytes;
  }
  if (pass == 2) {
    r3c_conv_desc d1;
    stride1_desc(d, d1);
    const int64_t inner = wgrad_ws(&d1, false);
    if (inner < 0) return -1;
    int64_t need = dilated_bytes(d1) + inner;
    StridedDwPlan dp;
    if (plan_strided_dw(d, stride, dp)) need = std::max(need, dp.part_bytes + dp.dbpart_bytes);
    r3c_conv_desc d2;
    int64_t xc = 0, yc = 0;
    if (plan_strided_dw_copies(d, stride, d2, dp, xc, yc))
      need = std::max(need, xc + yc + dp.part_bytes + dp.dbpart_bytes);
    return need;
  }
  return -1;
}

int32_t r3c_conv3d_strided_fwd(const r3c_conv_desc* d, const int32_t* stride, const void* x, const void* w,
                               const void* bias, void* y, void* ws, int64_t ws_bytes, void* stream) {
  if (!stride) return fail(R3C_INVALID, "stride is NULL");
  return run_strided(d, stride, false, x, w, bias, y, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_strided_dx(const r3c_conv_desc* d, const int32_t* stride, const void* dy, const void* w, void* dx,
                              void* ws, int64_t ws_bytes, void* stream) {
  if (!stride) return fail(R3C_INVALID, "stride is NULL");
  return run_strided(d, stride, true, dy, w, nullptr, dx, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_strided_dw(const r3c_conv_desc* d, const int32_t* stride, const void* x, const void* dy, void* dw,
                              int32_t dw_dtype, void* db, int32_t db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  if (!stride) return fail(R3C_INVALID, "stride is NULL");
  return run_strided_dw(d, stride, x, dy, dw, dw_dtype, db, db_dtype, ws, ws_bytes, stream);
}

int64_t r3c_conv3d_cat_workspace(const r3c_conv_desc* d, int32_t ca, int64_t xb_sample_stride, int32_t pass) {
  if (cat_check(d, ca, xb_sample_stride) != R3C_OK) return -1;
  if (pass == 0 || pass == 1) {
    RowPlan p;
    plan_row(d, pass == 0 ? OP_CONV_FWD : OP_CONV_DX, p);
    if (row_plan_reject(p) || !p.tap || p.copy_bytes || (pass == 0 && p.cl != 3)) return -1;
    return row_plan_ws(p);
  }
  if (pass == 2) {
    WgPlan p;
    plan_wgrad(d, false, p, true, true, ca);
    if (wgrad_plan_reject(p) || p.fl != 5) return -1;
    return wgrad_plan_ws(p);
  }
  return -1;
}

int32_t r3c_conv3d_cat_fwd(const r3c_conv_desc* d, int32_t ca, const void* xa, const void* xb,
                           int64_t xb_sample_stride, const void* w, const void* bias, void* y, void* ws,
                           int64_t ws_bytes, void* stream) {
  int rc = cat_check(d, ca, xb_sample_stride);
  if (rc) return rc;
  if (!xb) return fail(R3C_INVALID, "NULL tensor pointer");
  const CatSpec cs{ca, xb, nullptr, xb_sample_stride};
  return run_row(d, OP_CONV_FWD, xa, w, bias, y, ws, ws_bytes, stream, &cs);
}

int32_t r3c_conv3d_cat_dx(const r3c_conv_desc* d, int32_t ca, const void* dy, const void* w, void* dxa, void* dxb,
                          int64_t xb_sample_stride, void* ws, int64_t ws_bytes, void* stream) {
  int rc = cat_check(d, ca, xb_sample_stride);
  if (rc) return rc;
  if (!dxb) return fail(R3C_INVALID, "NULL tensor pointer");
  const CatSpec cs{ca, nullptr, dxb, xb_sample_stride};
  return run_row(d, OP_CONV_DX, dy, w, nullptr, dxa, ws, ws_bytes, stream, &cs);
}

int32_t r3c_conv3d_cat_dw(const r3c_conv_desc* d, int32_t ca, const void* xa, const void* xb,
                          int64_t xb_sample_stride, const void* dy, void* dw, int32_t dw_dtype, void* db,
                          int32_t db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  int rc = cat_check(d, ca, xb_sample_stride);
  if (rc) return rc;
  if (!xb) return fail(R3C_INVALID, "NULL tensor pointer");
  const CatSpec cs{ca, xb, nullptr, xb_sample_stride};
  return run_wgrad(d, false, xa, dy, dw, dw_dtype, db, db_dtype, ws, ws_bytes, stream, &cs);
}

int64_t r3c_bn_relu_workspace(const r3c_bn_desc* d) {
  if (bn_validate(d) != R3C_OK) return -1;
  return bn_ws(d);
}

int32_t r3c_bn_relu_fwd(const r3c_bn_desc* d, const void* y, const float* gamma, const float* beta,
                        float* running_mean, float* running_var, void* z, float* save_mean, float* save_invstd,
                        void* ws, int64_t ws_bytes, void* stream) {
  int rc = bn_validate(d);
  if (rc) return rc;
  if (!y || !z || !save_mean || !save_invstd || !ws) return fail(R3C_INVALID, "NULL pointer");
  if (!d->training && (!running_mean || !running_var))
    return fail(R3C_INVALID, "BatchNorm: evaluation needs the running statistics");
  if ((running_mean == nullptr) != (running_var == nullptr))
    return fail(R3C_INVALID, "BatchNorm: running_mean and running_var go together");
  if (ws_bytes < bn_ws(d))
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)bn_ws(d));
  if (!aligned16(y) || !aligned16(z)) return fail(R3C_UNSUPPORTED, "BatchNorm needs 16-byte aligned tensors");
  rc = check_device();
  if (rc) return rc;
  BnArgs a = bn_args(d, ws);
  a.y = y;
  a.out = z;
  a.gamma = gamma;
  a.beta = beta;
  a.running_mean = running_mean;
  a.running_var = running_var;
  a.save_mean = save_mean;
  a.save_invstd = save_invstd;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    TimedLaunch tl(KIND_BN, s);
    launch_bn_relu_fwd(d->dtype, a, s);
    tl.end();
  }
  return check_launch("BatchNorm + ReLU forward");
}

int32_t r3c_bn_relu_bwd(const r3c_bn_desc* d, const void* dz, const void* y, const float* gamma, const float* beta,
                        const float* save_mean, const float* save_invstd, void* dy, float* dgamma, float* dbeta,
                        void* ws, int64_t ws_bytes, void* stream) {
  int rc = bn_validate(d);
  if (rc) return rc;
  if (!dz || !y || !dy || !save_mean || !save_invstd || !ws) return fail(R3C_INVALID, "NULL pointer");
  if (ws_bytes < bn_ws(d))
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes, (long long)bn_ws(d));
  if (!aligned16(dz) || !aligned16(y) || !aligned16(dy))
    return fail(R3C_UNSUPPORTED, "BatchNorm needs 16-byte aligned tensors");
  rc = check_device();
  if (rc) return rc;
  BnArgs a = bn_args(d, ws);
  a.y = y;
  a.dz = dz;
  a.out = dy;
  a.gamma = gamma;
  a.beta = beta;
  a.save_mean = const_cast<float*>(save_mean);
  a.save_invstd = const_cast<float*>(save_invstd);
  a.dgamma = dgamma;
  a.dbeta = dbeta;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    TimedLaunch tl(KIND_BN, s);
    launch_bn_relu_bwd(d->dtype, a, s);
    tl.end();
  }
  return check_launch("BatchNorm + ReLU backward");
}

int32_t r3c_probe_mfma(int32_t shape, int32_t blocks, int32_t iters, float* out, void* stream) {
  if (shape != 0 && shape != 1) return fail(R3C_INVALID, "probe shape must be 0 (32x32x16) or 1 (16x16x32)");
  if (blocks < 1 || iters < 1 || !out) return fail(R3C_INVALID, "probe: blocks and iters >= 1, out non-null");
  int rc = check_device();
  if (rc) return rc;
  launch_mfma_probe(shape, blocks, iters, out, reinterpret_cast<hipStream_t>(stream));
  return check_launch("MFMA probe");
}

int32_t r3c_maxpool2_fwd(const r3c_pool_desc* d, const void* x, void* y, uint8_t* idx, void* stream) {
  PoolArgs a;
  int rc = pool_setup(d, a);
  if (rc) return rc;
  if (!x || !y || !idx) return fail(R3C_INVALID, "NULL pointer");
  if (!aligned16(x) || (reinterpret_cast<uintptr_t>(y) & 15) || (reinterpret_cast<uintptr_t>(idx) & 3))
    return fail(R3C_UNSUPPORTED, "MaxPool3d needs 16-byte aligned tensors");
  rc = check_device();
  if (rc) return rc;
  a.x = x;
  a.y = y;
  a.idx = idx;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    TimedLaunch tl(KIND_POOL, s);
    launch_maxpool2_fwd(d->dtype, a, s);
    tl.end();
  }
  return check_launch("MaxPool3d forward");
}

static int run_pool_bwd(const r3c_pool_desc* d, const void* dy, const uint8_t* idx, const void* add, const int64_t* add_strides,
                 void* dx, void* stream) {
  PoolArgs a;
  int rc = pool_setup(d, a);
  if (rc) return rc;
  if (!dy || !idx || !dx) return fail(R3C_INVALID, "NULL pointer");
  if (!aligned16(dx) || (reinterpret_cast<uintptr_t>(dy) & 15) || (reinterpret_cast<uintptr_t>(idx) & 3))
    return fail(R3C_UNSUPPORTED, "MaxPool3d needs 16-byte aligned tensors");
  if (add) {
    const int vec = d->dtype == R3C_F32 ? 4 : 8;
    if (!add_strides || !aligned16(add)) return fail(R3C_UNSUPPORTED, "MaxPool3d: the added gradient must be 16-byte aligned");
    for (int j = 0; j < 2; ++j)
      if (add_strides[j] < 0 || add_strides[j] % vec)
        return fail(R3C_UNSUPPORTED, "MaxPool3d: added gradient strides must be multiples of %d", vec);
    a.add = add;
    a.as0 = add_strides[0];
    a.as1 = add_strides[1];
  }
  rc = check_device();
  if (rc) return rc;
  a.dy = dy;
  a.dx = dx;
  a.idx = const_cast<uint8_t*>(idx);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  {
    TimedLaunch tl(KIND_POOL, s);
    launch_maxpool2_bwd(d->dtype, a, s);
    tl.end();
  }
  return check_launch("MaxPool3d backward");
}

int32_t r3c_maxpool2_bwd(const r3c_pool_desc* d, const void* dy, const uint8_t* idx, void* dx, void* stream) {
  return run_pool_bwd(d, dy, idx, nullptr, nullptr, dx, stream);
}

int32_t r3c_maxpool2_bwd_add(const r3c_pool_desc* d, const void* dy, const uint8_t* idx, const void* add,
                             const int64_t* add_strides, void* dx, void* stream) {
  if (!add) return fail(R3C_INVALID, "NULL pointer");
  return run_pool_bwd(d, dy, idx, add, add_strides, dx, stream);
}

int32_t r3c_conv3d_dw_static(const r3c_conv_desc* d, const void* x, const void* dy, void* dw, int32_t dw_dtype,
                             void* db, int32_t db_dtype, void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  const int64_t need = wgrad_ws(d, false);
  if (need < 0) return fail(R3C_UNSUPPORTED, "no weight-gradient plan for this descriptor");
  if (need > kStaticScratchBytes)
    return fail(R3C_UNSUPPORTED, "r3c_conv3d_dw_static: the pass needs %lld bytes of scratch, the static scratch holds %lld",
                (long long)need, (long long)kStaticScratchBytes);
  void* ws = nullptr;
  rc = static_scratch(&ws);
  if (rc) return rc;
  return run_wgrad(d, false, x, dy, dw, dw_dtype, db, db_dtype, ws, kStaticScratchBytes, stream);
}


int32_t r3c_convt_k2s2_fwd(const r3c_conv_desc* d, const void* x, const void* w, const void* bias, void* y, void* ws,
                           int64_t ws_bytes, void* stream) {
  int rc = validate(d, true);
  if (rc) return rc;
  return run_row(d, OP_T2_FWD, x, w, bias, y, ws, ws_bytes, stream);
}

int32_t r3c_convt_k2s2_dx(const r3c_conv_desc* d, const void* dy, const void* w, void* dx, void* ws,
                          int64_t ws_bytes, void* stream) {
  int rc = validate(d, true);
  if (rc) return rc;
  return run_row(d, OP_T2_DX, dy, w, nullptr, dx, ws, ws_bytes, stream);
}

int32_t r3c_convt_k2s2_dw(const r3c_conv_desc* d, const void* x, const void* dy, void* dw, int32_t dw_dtype,
                          void* db, int32_t db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  int rc = validate(d, true);
  if (rc) return rc;
  return run_wgrad(d, true, x, dy, dw, dw_dtype, db, db_dtype, ws, ws_bytes, stream);
}

int32_t r3c_timing_enable(int32_t on) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  st.on = on != 0;
  return R3C_OK;
}

void r3c_timing_set_tag(int32_t tag) { g_tag = tag; }

void r3c_timing_filter(int32_t tag, int32_t kind) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  st.filter_tag = tag;
  st.filter_kind = kind;
}

int32_t r3c_timing_collect(int32_t max_records, int32_t* tags, int32_t* kinds, float* ms) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  int32_t n = 0;
  for (const TimingRec& r : st.recs) {
    float t = -1.f;
    if (hipEventSynchronize(r.e1) == hipSuccess && hipEventElapsedTime(&t, r.e0, r.e1) != hipSuccess) t = -1.f;
    if (n < max_records) {
      if (tags) tags[n] = r.tag;
      if (kinds) kinds[n] = r.kind;
      if (ms) ms[n] = t;
    }
    ++n;
    st.pool.push_back(r.e0);
    st.pool.push_back(r.e1);
  }
  st.recs.clear();
  return n;
}

}  // extern "C"
