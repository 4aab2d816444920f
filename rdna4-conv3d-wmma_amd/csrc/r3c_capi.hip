// r3c_capi.hip -- the extern "C" boundary: argument validation, tile planning
// and kernel launches.  Every entry point is asynchronous on the caller's
// stream and allocates nothing (the caller passes the workspace it sized with
// the matching *_workspace query).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "r3c_kernels.h"
#include "rdna4_conv3d.h"

namespace r3c {

bool launch_fwd_k3(int dtype, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s);
bool launch_fwd_k1(int dtype, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s);
bool launch_fwd_t2dx(int dtype, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s);
bool launch_fwd_t2fwd(int dtype, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s);
bool launch_wgrad_k3(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s);
bool launch_wgrad_k1(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s);
bool launch_wgrad_t2(int dtype, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s);

bool launch_igemm_fwd(int dtype, int mode, int ck, int nb, const FwdArgs& a, size_t lds, hipStream_t s) {
  switch (mode) {
    case MODE_K3: return launch_fwd_k3(dtype, ck, nb, a, lds, s);
    case MODE_K1: return launch_fwd_k1(dtype, ck, nb, a, lds, s);
    case MODE_T2DX: return launch_fwd_t2dx(dtype, ck, nb, a, lds, s);
    case MODE_T2FWD: return launch_fwd_t2fwd(dtype, ck, nb, a, lds, s);
    default: return false;
  }
}

bool launch_igemm_wgrad(int dtype, int mode, int fb, int cbw, const WgradArgs& a, size_t lds, hipStream_t s) {
  switch (mode) {
    case MODE_K3: return launch_wgrad_k3(dtype, fb, cbw, a, lds, s);
    case MODE_K1: return launch_wgrad_k1(dtype, fb, cbw, a, lds, s);
    case MODE_T2DW: return launch_wgrad_t2(dtype, fb, cbw, a, lds, s);
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
enum KernelKind { KIND_PACK = 0, KIND_ROW = 1, KIND_WGRAD = 2, KIND_REDUCE = 3 };

struct TimingRec {
  int tag, kind;
  hipEvent_t e0, e1;
};

struct TimingState {
  std::mutex mu;
  bool on = false;
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
constexpr int kWgTarget = 512;                 // weight-gradient workgroups to aim for
constexpr int64_t kMaxPartialBytes = 96ll << 20;

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

int validate(const r3c_conv_desc* d, bool transpose) {
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
    if (d->od != d->d + 2 * d->pad_d - k + 1 || d->oh != d->h + 2 * d->pad_h - k + 1 ||
        d->ow != d->w + 2 * d->pad_w - k + 1)
      return fail(R3C_INVALID, "Conv3d: output dims do not match input + 2*pad - k + 1");
  }
  const int32_t xd[5] = {d->n, d->cin, d->d, d->h, d->w};
  const int32_t yd[5] = {d->n, d->cout, d->od, d->oh, d->ow};
  int rc = check_strides(d->x_strides, xd, "x");
  if (rc) return rc;
  return check_strides(d->y_strides, yd, "y");
}

int check_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return fail(R3C_HIP_ERROR, "hipGetDevice failed");
  if (!r3c_device_supported(dev)) return fail(R3C_UNSUPPORTED, "device %d is not gfx950", dev);
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

// ---------------------------------------------------------------------------
// Row-kernel plan (Conv3d fwd / dX, ConvTranspose fwd / dX)
// ---------------------------------------------------------------------------
struct FwdPlan {
  int mode, ck, nb, mb;
  FwdArgs a;
  PackArgs pk;
  size_t lds;
  int64_t wpk_bytes;
};

int pick_ck(int cs) { return cs <= 8 ? 8 : cs <= 16 ? 16 : cs <= 24 ? 24 : 32; }

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

void pick_box(int rows, int Rd, int Rh, int halo, int& TD, int& TH) {
  int64_t best = -1;
  for (int td = 1; td <= rows; td *= 2) {
    const int th = rows / td;
    const int64_t cost = (int64_t)cdiv(Rd, td) * cdiv(Rh, th) * (td + halo) * (th + halo);
    if (best < 0 || cost < best || (cost == best && td == 4)) {
      best = cost;
      TD = td;
      TH = th;
    }
  }
}

void plan_fwd(const r3c_conv_desc* d, int op, FwdPlan& p) {
  FwdArgs& a = p.a;
  memset(&a, 0, sizeof a);
  const int k = d->kernel;
  int cs = 0;
  if (op == OP_CONV_FWD || op == OP_CONV_DX) {
    p.mode = k == 3 ? MODE_K3 : MODE_K1;
  } else {
    p.mode = op == OP_T2_FWD ? MODE_T2FWD : MODE_T2DX;
  }
  switch (op) {
    case OP_CONV_FWD:
      cs = d->cin;
      a.Sd = d->d; a.Sh = d->h; a.Sw = d->w;
      a.Rd = d->od; a.Rh = d->oh; a.Rw = d->ow;
      a.Dd = d->od; a.Dh = d->oh; a.Dw = d->ow;
      a.pd = d->pad_d; a.ph = d->pad_h; a.pw = d->pad_w;
      a.ncols = d->cout;
      memcpy(a.ss, d->x_strides, sizeof a.ss);
      memcpy(a.sd, d->y_strides, sizeof a.sd);
      break;
    case OP_CONV_DX:
      cs = d->cout;
      a.Sd = d->od; a.Sh = d->oh; a.Sw = d->ow;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.Dd = d->d; a.Dh = d->h; a.Dw = d->w;
      a.pd = k - 1 - d->pad_d; a.ph = k - 1 - d->pad_h; a.pw = k - 1 - d->pad_w;
      a.ncols = d->cin;
      memcpy(a.ss, d->y_strides, sizeof a.ss);
      memcpy(a.sd, d->x_strides, sizeof a.sd);
      break;
    case OP_T2_FWD:
      cs = d->cin;
      a.Sd = d->d; a.Sh = d->h; a.Sw = d->w;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.Dd = d->od; a.Dh = d->oh; a.Dw = d->ow;
      a.ncols = 8 * d->cout;
      a.cout_t2 = d->cout;
      memcpy(a.ss, d->x_strides, sizeof a.ss);
      memcpy(a.sd, d->y_strides, sizeof a.sd);
      break;
    default:  // OP_T2_DX
      cs = d->cout;
      a.Sd = d->od; a.Sh = d->oh; a.Sw = d->ow;
      a.Rd = d->d; a.Rh = d->h; a.Rw = d->w;
      a.Dd = d->d; a.Dh = d->h; a.Dw = d->w;
      a.ncols = d->cin;
      memcpy(a.ss, d->y_strides, sizeof a.ss);
      memcpy(a.sd, d->x_strides, sizeof a.sd);
      break;
  }
  a.Cs = cs;
  p.ck = pick_ck(cs);
  const int nbt = cdiv(a.ncols, 16);
  if (p.mode == MODE_T2FWD) {
    static const int opts[] = {8, 4, 2};
    p.nb = pick_blocks(nbt, opts, 3);
  } else {
    static const int opts[] = {4, 3, 2, 1};
    p.nb = pick_blocks(nbt, opts, 4);
  }
  p.mb = p.mode == MODE_T2DX ? 2 : 4;
  const int rows = 4 * p.mb;
  const int halo = p.mode == MODE_K3 ? 2 : 0;
  pick_box(rows, a.Rd, a.Rh, halo, a.TD, a.TH);
  a.nbd = cdiv(a.Rd, a.TD);
  a.nbh = cdiv(a.Rh, a.TH);
  a.nbw = cdiv(a.Rw, 16);
  a.n_ctiles = cdiv(nbt, p.nb);
  a.nbt_pad = a.n_ctiles * p.nb;
  a.nchunks = cdiv(cs, p.ck);
  if (p.mode == MODE_K3) {
    a.HD = a.TD + 2; a.HH = a.TH + 2; a.HW = 18;
  } else if (p.mode == MODE_T2DX) {
    a.HD = 2 * a.TD; a.HH = 2 * a.TH; a.HW = 32;
  } else {
    a.HD = a.TD; a.HH = a.TH; a.HW = 16;
  }
  const int g8 = p.ck / 8;
  const int cp = (g8 & 1) ? p.ck : p.ck + 8;
  const int taps = p.mode == MODE_K3 ? 27 : (p.mode == MODE_T2DX ? 8 : 1);
  const int nstep = cdiv(taps * g8, 4);
  const int64_t hpos = (int64_t)a.HD * a.HH * a.HW;
  p.lds = (size_t)(hpos * cp * 2 + nstep * 4 * 4);
  a.nblocks = 0;  // filled with the batch at launch
  PackArgs& pk = p.pk;
  memset(&pk, 0, sizeof pk);
  pk.cs = cs;
  pk.ncols = a.ncols;
  pk.taps = taps;
  pk.ck = p.ck;
  pk.nchunks = a.nchunks;
  pk.nstep = nstep;
  pk.nbt_pad = a.nbt_pad;
  pk.w_cin = d->cin;
  pk.w_cout = d->cout;
  pk.mode = p.mode | (op == OP_CONV_DX ? 16 : 0);
  pk.total = (int64_t)a.nchunks * nstep * a.nbt_pad * 64 * 8;
  p.wpk_bytes = pk.total * 2;
}

int run_fwd(const r3c_conv_desc* d, int op, const void* src, const void* w, const void* bias, void* dst, void* ws,
            int64_t ws_bytes, void* stream) {
  FwdPlan p;
  plan_fwd(d, op, p);
  if ((int64_t)p.lds > kMaxLds) return fail(R3C_UNSUPPORTED, "tile needs %zu bytes of LDS", p.lds);
  if (ws_bytes < align256(p.wpk_bytes))
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes,
                (long long)align256(p.wpk_bytes));
  if (!src || !w || !dst || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  int rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
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
  FwdArgs a = p.a;
  a.src = static_cast<const uint16_t*>(src);
  a.wpk = static_cast<const uint16_t*>(ws);
  a.bias = static_cast<const uint16_t*>(bias);
  a.dst = static_cast<uint16_t*>(dst);
  a.src_cl = vec16_ok(src, a.ss) ? 1 : 0;
  const int64_t blocks = (int64_t)d->n * a.nbd * a.nbh * a.nbw * a.n_ctiles;
  if (blocks >= (1ll << 31)) return fail(R3C_UNSUPPORTED, "grid too large");
  a.nblocks = (int32_t)blocks;
  TimedLaunch tl(KIND_ROW, s);
  const bool launched = launch_igemm_fwd(d->dtype, p.mode, p.ck, p.nb, a, p.lds, s);
  tl.end();
  if (!launched)
    return fail(R3C_UNSUPPORTED, "no row-kernel instantiation for mode %d ck %d nb %d", p.mode, p.ck, p.nb);
  return check_launch("row kernel");
}

// ---------------------------------------------------------------------------
// Weight-gradient plan (Conv3d dW k1/k3, ConvTranspose dW)
// ---------------------------------------------------------------------------
struct WgPlan {
  int mode, fb, cbw, taps;
  WgradArgs a;
  size_t lds;
  int64_t part_bytes, dbpart_bytes;
};

int pad16(int c) { return (c / 16) % 2 == 0 ? c + 16 : c; }  // LDS row pitch: an odd number of 32-byte units

void plan_wgrad(const r3c_conv_desc* d, bool transpose, WgPlan& p) {
  WgradArgs& a = p.a;
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
  const int nfb = cdiv(a.Fc, 16), ngb = cdiv(a.Gc, 16);
  // F blocks per workgroup.
  {
    static const int opts[] = {3, 2, 1};
    p.fb = nfb <= 3 ? nfb : pick_blocks(nfb, opts, 3);
  }
  // Column tiling: (CBW, GCB) maximising useful MFMA slots.
  int cbw_opts[3];
  int ncbw = 0;
  if (p.mode == MODE_K3) {
    if (p.fb == 3) {
      cbw_opts[0] = 7;
      ncbw = 1;
    } else {
      cbw_opts[0] = 14;
      cbw_opts[1] = 7;
      ncbw = 2;
    }
  } else if (p.mode == MODE_K1) {
    cbw_opts[0] = 1;
    ncbw = 1;
  } else {
    cbw_opts[0] = 7;
    cbw_opts[1] = 4;
    cbw_opts[2] = 2;
    ncbw = 3;
  }
  double best_eff = -1.0;
  int best_tiles = 0;
  const int gcb_max = p.mode == MODE_K1 ? 4 : 3;
  for (int i = 0; i < ncbw; ++i) {
    for (int gcb = 1; gcb <= gcb_max; ++gcb) {
      const int slots = 4 * cbw_opts[i];
      if (gcb > slots) continue;
      const int tt = std::min(p.taps, slots / gcb);
      const int ntt = cdiv(p.taps, tt);
      const int ngt = cdiv(ngb, gcb);
      const double eff = (double)p.taps * ngb / ((double)ntt * ngt * slots);
      const int tiles = ntt * ngt;
      if (eff > best_eff + 1e-9 || (eff > best_eff - 1e-9 && tiles < best_tiles)) {
        best_eff = eff;
        best_tiles = tiles;
        p.cbw = cbw_opts[i];
        a.GCB = gcb;
        a.TT = tt;
      }
    }
  }
  a.n_ftiles = cdiv(nfb, p.fb);
  a.n_gtiles = cdiv(ngb, a.GCB);
  a.n_ttiles = cdiv(p.taps, a.TT);
  a.Fpad = a.n_ftiles * p.fb * 16;
  a.Gpad = a.n_gtiles * a.GCB * 16;
  a.cpf = pad16(p.fb * 16);
  a.cpg = pad16(a.GCB * 16);
  if (p.mode == MODE_K3) {
    a.TD = 2; a.TH = 4;
  } else if (p.mode == MODE_K1) {
    a.TD = 4; a.TH = 4;
  } else {
    a.TD = 2; a.TH = 2;
  }
  a.th_log2 = a.TH == 1 ? 0 : (a.TH == 2 ? 1 : (a.TH == 4 ? 2 : 3));
  if (p.mode == MODE_K3) {
    a.HD = a.TD + 2; a.HH = a.TH + 2; a.HW = 18;
  } else if (p.mode == MODE_T2DW) {
    a.HD = 2 * a.TD; a.HH = 2 * a.TH; a.HW = 32;
  } else {
    a.HD = a.TD; a.HH = a.TH; a.HW = 16;
  }
  a.nbd = cdiv(a.Rd, a.TD);
  a.nbh = cdiv(a.Rh, a.TH);
  a.nbw = cdiv(a.Rw, 16);
  const int64_t nbox = (int64_t)d->n * a.nbd * a.nbh * a.nbw;
  a.nbox = (int32_t)std::min<int64_t>(nbox, (1ll << 31) - 1);
  const int tiles = a.n_ftiles * a.n_gtiles * a.n_ttiles;
  const int64_t per_split = (int64_t)a.Fpad * p.taps * a.Gpad * 4;
  int64_t nsplit = cdiv(kWgTarget, tiles);
  nsplit = std::min<int64_t>(nsplit, std::max<int64_t>(1, kMaxPartialBytes / per_split));
  nsplit = std::max<int64_t>(1, std::min<int64_t>(nsplit, nbox));
  a.nsplit = (int32_t)nsplit;
  a.nblocks = (int32_t)(nsplit * tiles);
  const int64_t boxpos = (int64_t)a.TD * a.TH * 16;
  const int64_t hpos = (int64_t)a.HD * a.HH * a.HW;
  p.lds = (size_t)(boxpos * a.cpf * 2 + hpos * a.cpg * 2);
  p.part_bytes = align256(nsplit * per_split);
  p.dbpart_bytes = align256(nsplit * (int64_t)std::max(a.Fpad, p.taps * a.Gpad) * 4);
}

int run_wgrad(const r3c_conv_desc* d, bool transpose, const void* x, const void* dy, void* dw, int dw_dtype, void* db,
              int db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  WgPlan p;
  plan_wgrad(d, transpose, p);
  if ((int64_t)p.lds > kMaxLds) return fail(R3C_UNSUPPORTED, "tile needs %zu bytes of LDS", p.lds);
  if (ws_bytes < p.part_bytes + p.dbpart_bytes)
    return fail(R3C_INVALID, "workspace too small: %lld < %lld bytes", (long long)ws_bytes,
                (long long)(p.part_bytes + p.dbpart_bytes));
  if (!x || !dy || !dw || !ws) return fail(R3C_INVALID, "NULL tensor pointer");
  if (dw_dtype != R3C_F32 && dw_dtype != d->dtype) return fail(R3C_INVALID, "dw_dtype must be fp32 or the input dtype");
  if (db && db_dtype != R3C_F32 && db_dtype != R3C_F16 && db_dtype != R3C_BF16)
    return fail(R3C_INVALID, "db_dtype must be fp32, fp16 or bf16");
  int rc = check_device();
  if (rc) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  WgradArgs a = p.a;
  a.fsrc = static_cast<const uint16_t*>(transpose ? x : dy);
  a.gsrc = static_cast<const uint16_t*>(transpose ? dy : x);
  a.part = static_cast<float*>(ws);
  a.dbpart = reinterpret_cast<float*>(static_cast<char*>(ws) + p.part_bytes);
  a.f_cl = vec16_ok(a.fsrc, a.fs) ? 1 : 0;
  a.g_cl = vec16_ok(a.gsrc, a.gs) ? 1 : 0;
  a.db_mode = db ? (transpose ? 2 : 1) : 0;
  TimedLaunch tl(KIND_WGRAD, s);
  const bool launched = launch_igemm_wgrad(d->dtype, p.mode, p.fb, p.cbw, a, p.lds, s);
  tl.end();
  if (!launched)
    return fail(R3C_UNSUPPORTED, "no weight-gradient instantiation for mode %d fb %d cbw %d", p.mode, p.fb, p.cbw);
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

int64_t fwd_ws(const r3c_conv_desc* d, int op, bool transpose) {
  if (validate(d, transpose) != R3C_OK) return -1;
  FwdPlan p;
  plan_fwd(d, op, p);
  return align256(p.wpk_bytes);
}

int64_t wgrad_ws(const r3c_conv_desc* d, bool transpose) {
  if (validate(d, transpose) != R3C_OK) return -1;
  WgPlan p;
  plan_wgrad(d, transpose, p);
  return p.part_bytes + p.dbpart_bytes;
}

std::mutex g_dev_mu;
std::unordered_map<int, int> g_dev_ok;

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
  return run_fwd(d, OP_CONV_FWD, x, w, bias, y, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_dx(const r3c_conv_desc* d, const void* dy, const void* w, void* dx, void* ws, int64_t ws_bytes,
                      void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  return run_fwd(d, OP_CONV_DX, dy, w, nullptr, dx, ws, ws_bytes, stream);
}

int32_t r3c_conv3d_dw(const r3c_conv_desc* d, const void* x, const void* dy, void* dw, int32_t dw_dtype, void* db,
                      int32_t db_dtype, void* ws, int64_t ws_bytes, void* stream) {
  int rc = validate(d, false);
  if (rc) return rc;
  return run_wgrad(d, false, x, dy, dw, dw_dtype, db, db_dtype, ws, ws_bytes, stream);
}

int32_t r3c_convt_k2s2_fwd(const r3c_conv_desc* d, const void* x, const void* w, const void* bias, void* y, void* ws,
                           int64_t ws_bytes, void* stream) {
  int rc = validate(d, true);
  if (rc) return rc;
  return run_fwd(d, OP_T2_FWD, x, w, bias, y, ws, ws_bytes, stream);
}

int32_t r3c_convt_k2s2_dx(const r3c_conv_desc* d, const void* dy, const void* w, void* dx, void* ws,
                          int64_t ws_bytes, void* stream) {
  int rc = validate(d, true);
  if (rc) return rc;
  return run_fwd(d, OP_T2_DX, dy, w, nullptr, dx, ws, ws_bytes, stream);
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
