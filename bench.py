"""Benchmark of the Conv3d hot path on one MI355X (gfx950).

Metric: "Conv3d fwd/dW/dX TFLOP/s (% MFMA peak); UNet3D b4 ms/sample".

One step = forward, dX and dW (with the fused bias gradient) of the four UNet3D
trunk k=3 layers of BASELINE config 2, bf16 inputs, fp32 accumulation, inputs
already resident in HBM:
    [4,24,64,128,128]->24, [4,48,32,64,64]->48, [4,96,16,32,32]->96, [4,192,8,16,16]->192
value = algorithmic FLOPs of the step (3 passes x 2*N*D*H*W*Cin*Cout*27 per layer)
        / measured step time, in TFLOP/s.  Order: W warmup steps, --preheat
        seconds of further untimed steps (clocks at steady state; reported as
        preheat_s / preheat_steps), the per-pass profile steps, then exactly K
        timed steps.

Also reported on the same JSON line:
  roofline      the dominant kernel (largest share of the step): algorithmic FLOPs
                per launch / its average launch duration, measured live with HIP
                events on its launch stream (the library's timing hook) during the
                timed steps, against the 2.5 PFLOP/s dense bf16 MFMA peak.  Only
                that kernel's launches carry events in the timed steps, so the
                hook does not slow the step it measures.
  passes        per-pass kernel time and fraction of peak, from a few untimed
                steps before the timed region in which every launch carries events
                (these also pick the dominant kernel).
  hbm_passes    BASELINE configs 3 and 4 (k=1 fp16, ConvTranspose3d k2s2 bf16):
                per-pass time (all kernels of the pass, median of 20, MALL
                flushed before each by a 512 MB write and a 512 MB read) and
                compulsory HBM bytes / time vs 8 TB/s.
  strided_passes  the strided Conv3d (k=3 stride 2, [4,24,64,128,128] -> 48,
                bf16; outside the reference's stride-1 policy): native and stock
                (MIOpen) time per pass, TFLOP/s on the algorithmic FLOPs and the
                fraction of HBM peak on the compulsory activation bytes.
  cpu_baseline  the reference's CPU path (Conv3dWmma on CPU tensors ->
                nn.Conv3d.forward -> F.conv3d, oneDNN, fp32) on a bounded sample.

  unet3d        BASELINE config 5: ms per AMP training step (and per sample) of the
                base=24 UNet3D at batch 4 built with this package's layers, with its
                fused BatchNorm + ReLU too, and with stock nn.Conv3d /
                nn.ConvTranspose3d; the largest loss gaps over 40 steps against
                stock, and stock's own spread (the batch in reversed order);
                unet3d_base32 the same at base=32; with --unet-fp16, unet3d_fp16
                the same at base=24 under fp16 autocast (the reference's protocol).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--preheat SEC] [--layout ncdhw|ndhwc]
                       [--unet-steps S] [--unet-fp16]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "rdna4-conv3d-wmma_amd"))

MFMA_PEAK_TFLOPS = 2500.0   # dense bf16, MI355X
HBM_PEAK_GBS = 8000.0

TRUNK = [  # (N, Cin, Cout, D, H, W)
    (4, 24, 24, 64, 128, 128),
    (4, 48, 48, 32, 64, 64),
    (4, 96, 96, 16, 32, 32),
    (4, 192, 192, 8, 16, 16),
]
PASSES = ("fwd", "dx", "dw")
# BASELINE configs 3 (pointwise k=1, fp16) and 4 (ConvTranspose3d k=2 s=2, bf16):
# memory-bound passes, judged on compulsory HBM bytes per pass.
POINTWISE = [(4, 48, 24, 64, 128, 128), (4, 24, 96, 64, 128, 128)]   # (N, Cin, Cout, D, H, W)
CONVT = [(4, 192, 96, 8, 16, 16), (4, 48, 24, 32, 64, 64)]           # (N, Cin, Cout, D, H, W) of the input
FLUSH_BYTES = 512 << 20  # written, then another buffer of this size read, between repetitions (256 MB MALL)


def _flops(n, ci, co, d, h, w):
    return 2.0 * n * d * h * w * ci * co * 27


def _gen(shape, seed, dtype):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32).to(dtype)


def _kaiming(shape, fan_in, seed, dtype):
    import torch
    g = torch.Generator().manual_seed(seed)
    b = 1.0 / fan_in ** 0.5
    return ((torch.rand(*shape, generator=g) * 2 - 1) * b).to(dtype)


def cpu_baseline(budget_s: float = 20.0):
    """Reference CPU path on the host cores: F.conv3d fwd + dX + dW in fp32.

    Sample: batch 1 of each trunk shape (1/4 of the GPU step's work per shape),
    1 warmup, then repeated until the time budget is used (at least 1 rep).
    """
    import torch
    import torch.nn.functional as F
    torch.set_num_threads(os.cpu_count() or 1)
    layers = []
    for (n, ci, co, d, h, w) in TRUNK:
        x = _gen((1, ci, d, h, w), 0, torch.float32).requires_grad_(True)
        wt = _kaiming((co, ci, 3, 3, 3), ci * 27, 1, torch.float32).requires_grad_(True)
        go = _gen((1, co, d, h, w), 2, torch.float32)
        layers.append((x, wt, go, _flops(1, ci, co, d, h, w) * 3))

    def once():
        for x, wt, go, _ in layers:
            x.grad = None
            wt.grad = None
            y = F.conv3d(x, wt, None, 1, 1)
            y.backward(go)

    once()  # warmup
    reps, t0 = 0, time.perf_counter()
    while True:
        once()
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 500:
            break
    flops = sum(l[3] for l in layers) * reps
    return {
        "value": round(flops / el / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": torch.get_num_threads(),
        "kind": "reference",
        "sample": (f"reference CPU path (Conv3dWmma on CPU tensors -> nn.Conv3d.forward -> F.conv3d, "
                   f"oneDNN, fp32): fwd+dX+dW of the 4 trunk layers at batch 1, {reps} rep(s) in {el:.1f} s; "
                   f"os.cpu_count()={os.cpu_count()}, mkldnn={torch.backends.mkldnn.is_available()}"),
    }


def _unet_block(cin, cout, conv, bnrelu=None):
    """Two (3x3x3 conv, BatchNorm, ReLU); `bnrelu(c)` builds one fused
    BatchNorm + ReLU module in place of nn.BatchNorm3d(c), nn.ReLU().  Both
    forms create their parameters in the same order, so a seeded build gives
    the same initial weights either way."""
    import torch.nn as nn
    if bnrelu is None:
        return nn.Sequential(
            conv(cin, cout, 3, padding=1), nn.BatchNorm3d(cout), nn.ReLU(inplace=True),
            conv(cout, cout, 3, padding=1), nn.BatchNorm3d(cout), nn.ReLU(inplace=True),
        )
    return nn.Sequential(conv(cin, cout, 3, padding=1), bnrelu(cout), conv(cout, cout, 3, padding=1), bnrelu(cout))


def build_unet3d(conv, tr, base=24, cin=1, classes=2, bnrelu=None, pool=None, cat_free=False):
    """UNet3D of BASELINE config 5: 4 levels (base, 2, 4, 8 x base channels),
    two (3x3x3 conv + BatchNorm + ReLU) per block, MaxPool3d(2) down,
    ConvTranspose3d k2s2 up with skip concat, 1x1x1 head to `classes`.
    `conv` / `tr` are the Conv3d / ConvTranspose3d classes to build with (the
    reference's factory pattern, benches/unet_e2e.py:13-32); `bnrelu`, if
    given, builds the fused BatchNorm + ReLU modules, `pool` the MaxPool3d(2)
    module class (nn.MaxPool3d by default); `cat_free` feeds each decoder
    block's first conv the upsampled tensor and the skip tensor through its
    forward_cat (no torch.cat) when the conv class has one, and takes the
    pooled and skip tensors from the pool's forward_with_skip when it has one
    (the skip's gradient is added in the pooling backward's pass)."""
    import torch
    import torch.nn as nn

    ch = [base, 2 * base, 4 * base, 8 * base]

    class UNet3D(nn.Module):
        def __init__(self):
            super().__init__()
            self.enc = nn.ModuleList([_unet_block(cin, ch[0], conv, bnrelu), _unet_block(ch[0], ch[1], conv, bnrelu),
                                      _unet_block(ch[1], ch[2], conv, bnrelu), _unet_block(ch[2], ch[3], conv, bnrelu)])
            self.pool = (pool or nn.MaxPool3d)(2)
            self.up = nn.ModuleList([tr(ch[3], ch[2], 2, stride=2), tr(ch[2], ch[1], 2, stride=2),
                                     tr(ch[1], ch[0], 2, stride=2)])
            self.dec = nn.ModuleList([_unet_block(2 * ch[2], ch[2], conv, bnrelu),
                                      _unet_block(2 * ch[1], ch[1], conv, bnrelu),
                                      _unet_block(2 * ch[0], ch[0], conv, bnrelu)])
            self.head = conv(ch[0], classes, 1)

        def forward(self, x):
            skips = []
            for i, blk in enumerate(self.enc):
                x = blk(x)
                if i < 3:
                    if cat_free and hasattr(self.pool, "forward_with_skip"):
                        # one backward pass for the pooled path and the skip's gradient
                        x, skip = self.pool.forward_with_skip(x)
                        skips.append(skip)
                    else:
                        skips.append(x)
                        x = self.pool(x)
            for up, dec, skip in zip(self.up, self.dec, reversed(skips)):
                u = up(x)
                if cat_free and hasattr(dec[0], "forward_cat"):
                    x = dec[1:](dec[0].forward_cat(u, skip))
                else:
                    x = dec(torch.cat([u, skip], dim=1))
            return self.head(x)

    return UNet3D()


def _rounded_layers():
    """Conv3d / ConvTranspose3d whose arithmetic is fp32 on the autocast-dtype
    operands, with every result (y, dX, dW, db) rounded once to that dtype:
    a correctly rounded half-precision convolution.  Used as the second correct
    half-precision implementation in the loss-spread control (stock MIOpen is
    the first): the two differ only in how each convolution sums and rounds."""
    import torch
    import torch.nn as nn
    import torch.nn.functional as F

    def amp_cast(*ts):
        if not torch.is_autocast_enabled("cuda"):
            return ts
        dt = torch.get_autocast_dtype("cuda")
        return tuple(None if t is None else t.to(dt) for t in ts)

    class _Fn(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, w, b, transpose, stride, padding):
            ctx.save_for_backward(x, w)
            ctx.cfg = (transpose, stride, padding, b is not None, None if b is None else b.dtype)
            f = F.conv_transpose3d if transpose else F.conv3d
            with torch.autocast("cuda", enabled=False):
                y = f(x.float(), w.float(), None if b is None else b.float(), stride, padding)
            return y.to(x.dtype)

        @staticmethod
        def backward(ctx, go):
            x, w = ctx.saved_tensors
            transpose, stride, padding, has_b, b_dtype = ctx.cfg
            with torch.enable_grad(), torch.autocast("cuda", enabled=False):
                xf = x.detach().float().requires_grad_(True)
                wf = w.detach().float().requires_grad_(True)
                f = F.conv_transpose3d if transpose else F.conv3d
                y = f(xf, wf, None, stride, padding)
                gx, gw = torch.autograd.grad(y, (xf, wf), go.float())
            gb = go.float().sum((0, 2, 3, 4)).to(b_dtype) if has_b else None
            return gx.to(x.dtype), gw.to(w.dtype), gb, None, None, None

    class RoundedConv3d(nn.Conv3d):
        def forward(self, x):
            x, w, b = amp_cast(x, self.weight, self.bias)
            return _Fn.apply(x, w, b, False, self.stride, self.padding)

    class RoundedConvTranspose3d(nn.ConvTranspose3d):
        def forward(self, x, output_size=None):
            x, w, b = amp_cast(x, self.weight, self.bias)
            return _Fn.apply(x, w, b, True, self.stride, self.padding)

    return RoundedConv3d, RoundedConvTranspose3d


def _gpu_preheat(seconds: float) -> None:
    """Untimed bf16 matrix products for `seconds`: the GPU's clocks settle
    within about half a second of sustained load, and a timed loop that
    starts after host-side work (building a model) would otherwise start
    below them."""
    import torch
    a = torch.ones(4096, 4096, dtype=torch.bfloat16, device="cuda")
    t0 = time.perf_counter()
    n = 0
    while time.perf_counter() - t0 < seconds:
        torch.mm(a, a)
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    del a


def unet3d_train(conv, tr, base, x, labels, steps, warmup, amp_dtype=None, channels_last=False, bnrelu=None,
                 pool=None, cat_free=False):
    """AMP training of build_unet3d(conv, tr, base) on (x, labels):
    cross-entropy, Adam(lr=1e-3), autocast in `amp_dtype` (bf16 by default,
    BASELINE config 5; torch.float16 is the reference's protocol,
    benches/unet_e2e.py:47, whose torch.autocast("cuda") defaults to fp16), no
    gradient scaler (as in the reference).  channels_last runs model and input
    in channels_last_3d.  Weights are seeded (seed 1) before the build, so two
    calls with different layer classes start from identical weights.
    Returns (ms per timed step, losses of every step in order)."""
    import torch
    import torch.nn as nn
    amp_dtype = amp_dtype or torch.bfloat16
    torch.manual_seed(1)
    net = build_unet3d(conv, tr, base, bnrelu=bnrelu, pool=pool, cat_free=cat_free).to(x.device)
    if channels_last:
        net = net.to(memory_format=torch.channels_last_3d)
        x = x.contiguous(memory_format=torch.channels_last_3d)
    opt = torch.optim.Adam(net.parameters(), lr=1e-3)
    loss_fn = nn.CrossEntropyLoss()

    def step():
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=amp_dtype):
            y = net(x)
            loss = loss_fn(y, labels)
        loss.backward()
        opt.step()
        return loss.detach()

    losses = [step() for _ in range(warmup)]
    torch.cuda.synchronize()
    _gpu_preheat(0.5)  # clocks at steady state for every variant alike; the model is untouched
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        losses.append(step())
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / max(1, steps)
    del net, opt
    return ms, [float(v) for v in losses]


def hbm_passes(layout: str, reps: int = 20):
    """BASELINE configs 3 and 4: per-pass time (median over reps of the summed
    kernel durations of the pass, HIP events on the launch stream) and the
    compulsory HBM bytes over that time.  Before every repetition a 512 MB
    buffer is written and a second 512 MB buffer is read: the write evicts the
    working set from the 256 MB MALL, the read leaves the MALL holding clean
    lines, so the timed pass neither hits its operands there nor pays for
    writing back an unrelated kernel's dirty lines."""
    import torch
    from rdna4_conv3d import _native as nat
    dev = torch.device("cuda", 0)
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    flush_rd = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)

    def L(t):
        return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()

    def nbytes(*ts):
        return sum(t.numel() * t.element_size() for t in ts)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        tot = []
        for r in range(reps):
            flush.zero_()
            flush_rd.sum()
            nat.timing_enable(True)
            nat.timing_collect()
            fn()
            recs = nat.timing_collect()
            nat.timing_enable(False)
            tot.append(sum(ms for _, _, ms in recs))
        tot.sort()
        return tot[len(tot) // 2]

    out = {}
    for (n, ci, co, d, h, w) in POINTWISE:
        x = L(torch.relu(_gen((n, ci, d, h, w), 0, torch.float16)).to(dev))
        go = L(_gen((n, co, d, h, w), 2, torch.float16).to(dev))
        wt = _kaiming((co, ci, 1, 1, 1), ci, 1, torch.float16).to(dev)
        y = nat.conv3d_fwd(x, wt, None, (0, 0, 0))
        dw, _ = nat.conv3d_dw(x, go, wt.shape, (0, 0, 0), torch.float32)
        cases = {
            "fwd": (lambda: nat.conv3d_fwd(x, wt, None, (0, 0, 0)), nbytes(x, y, wt)),
            "dx": (lambda: nat.conv3d_dx(go, wt, x.shape, (0, 0, 0), like=x), nbytes(go, x, wt)),
            "dw": (lambda: nat.conv3d_dw(x, go, wt.shape, (0, 0, 0), torch.float32), nbytes(x, go, dw)),
        }
        for p, (fn, by) in cases.items():
            ms = timed(fn)
            out[f"k1_{ci}to{co}_{d}x{h}x{w}_fp16_{p}"] = {
                "us": round(ms * 1e3, 2), "bytes": by, "gbs": round(by / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del x, go, y, dw
    for (n, ci, co, d, h, w) in CONVT:
        x = L(_gen((n, ci, d, h, w), 0, torch.bfloat16).to(dev))
        go = L(_gen((n, co, 2 * d, 2 * h, 2 * w), 2, torch.bfloat16).to(dev))
        wt = _kaiming((ci, co, 2, 2, 2), co * 8, 1, torch.bfloat16).to(dev)
        b = _kaiming((co,), co * 8, 3, torch.bfloat16).to(dev)
        y = nat.convt_fwd(x, wt, b)
        dw, db = nat.convt_dw(x, go, wt.shape, torch.float32, want_db=True, db_dtype=torch.float32)
        cases = {
            "fwd": (lambda: nat.convt_fwd(x, wt, b), nbytes(x, y, wt, b)),
            "dx": (lambda: nat.convt_dx(go, wt, x.shape, like=x), nbytes(go, x, wt)),
            "dw": (lambda: nat.convt_dw(x, go, wt.shape, torch.float32, want_db=True, db_dtype=torch.float32),
                   nbytes(x, go, dw, db)),
        }
        for p, (fn, by) in cases.items():
            ms = timed(fn)
            out[f"convt_{ci}to{co}_{2 * d}x{2 * h}x{2 * w}_bf16_{p}"] = {
                "us": round(ms * 1e3, 2), "bytes": by, "gbs": round(by / (ms * 1e-3) / 1e9, 1),
                "frac_hbm": round(by / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del x, go, y, dw, db
    del flush, flush_rd
    torch.cuda.empty_cache()
    return out


# The strided pass: the downsampling convolution k=3 stride 2 pad 1,
# (n, cin, cout, d, h, w, stride, padding).
STRIDED = (4, 24, 48, 64, 128, 128, (2, 2, 2), (1, 1, 1))


def strided_passes(layout: str, reps: int = 10):
    """Strided Conv3d (the downsampling convolution, outside the reference's
    stride-1 policy): k=3 stride 2 pad 1, [4, 24, 64, 128, 128] -> 48 channels
    bf16.  Native: median of the summed kernel durations of each pass (HIP
    events on the launch stream, MALL flushed as in hbm_passes).  Stock:
    F.conv3d / torch.nn.grad on the same tensors, CUDA events around the call.
    TFLOP/s on the algorithmic 2 N OD OH OW Cout Cin 27; frac_hbm on the
    compulsory |x| + |y| bytes (the bound at this shape: 130 FLOP per byte)."""
    import torch
    import torch.nn.functional as F
    from rdna4_conv3d import _native as nat
    dev = torch.device("cuda", 0)
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    flush_rd = torch.ones(FLUSH_BYTES // 4, dtype=torch.float32, device=dev)

    def L(t):
        return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()

    def med(v):
        v = sorted(v)
        return v[len(v) // 2]

    def native_ms(fn):
        fn()
        torch.cuda.synchronize()
        tot = []
        for _ in range(reps):
            flush.zero_()
            flush_rd.sum()
            nat.timing_enable(True)
            nat.timing_collect()
            fn()
            recs = nat.timing_collect()
            nat.timing_enable(False)
            tot.append(sum(ms for _, _, ms in recs))
        return med(tot)

    def stock_ms(fn):
        fn()
        torch.cuda.synchronize()
        tot = []
        for _ in range(reps):
            flush.zero_()
            flush_rd.sum()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            fn()
            b.record()
            b.synchronize()
            tot.append(a.elapsed_time(b))
        return med(tot)

    n, ci, co, d, h, w, st, pd = STRIDED
    x = L(_gen((n, ci, d, h, w), 0, torch.bfloat16).to(dev))
    wt = _kaiming((co, ci, 3, 3, 3), ci * 27, 1, torch.bfloat16).to(dev)
    b = _kaiming((co,), ci * 27, 3, torch.bfloat16).to(dev)
    y_shape = nat.strided_out_shape(x.shape, wt.shape, st, pd)
    go = L(_gen(y_shape, 2, torch.bfloat16).to(dev))
    flops = 2.0 * n * y_shape[2] * y_shape[3] * y_shape[4] * co * ci * 27
    native = {
        "fwd": lambda: nat.conv3d_strided_fwd(x, wt, b, st, pd),
        "dx": lambda: nat.conv3d_strided_dx(go, wt, x.shape, st, pd, like=x),
        "dw": lambda: nat.conv3d_strided_dw(x, go, wt.shape, st, pd, torch.float32, want_db=True,
                                            db_dtype=torch.float32),
    }
    stock = {
        "fwd": lambda: F.conv3d(x, wt, b, st, pd),
        "dx": lambda: torch.nn.grad.conv3d_input(x.shape, wt, go, st, pd),
        "dw": lambda: torch.nn.grad.conv3d_weight(x, wt.shape, go, st, pd),
    }
    # compulsory HBM bytes: the pass's two activation tensors (the weight is 62 KB)
    act_bytes = (x.numel() + go.numel()) * 2
    out = {}
    for p in ("fwd", "dx", "dw"):
        ms_n, ms_s = native_ms(native[p]), stock_ms(stock[p])
        out[f"k3s2_{ci}to{co}_{d}x{h}x{w}_bf16_{p}"] = {
            "us": round(ms_n * 1e3, 2), "tflops": round(flops / (ms_n * 1e-3) / 1e12, 1),
            "frac_hbm": round(act_bytes / (ms_n * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "stock_us": round(ms_s * 1e3, 2), "stock_tflops": round(flops / (ms_s * 1e-3) / 1e12, 1)}
    del x, go, wt, flush, flush_rd
    torch.cuda.empty_cache()
    return out


def unet3d_bench(steps: int, warmup: int, base: int = 24, batch: int = 4, amp_dtype=None):
    """the UNet3D built with this package's layers (and, as
    a second variant, with its fused BatchNorm + ReLU, MaxPool3d(2) and
    concatenation-free decoder convs as well) against stock nn.Conv3d /
    nn.ConvTranspose3d, AMP bf16 (amp_dtype torch.float16: the reference's own
    protocol, torch.autocast("cuda") without a gradient scaler).

    Loss tracking is reported against the spread of stock itself: the same
    stock model trained on the same batch with the sample order reversed (a
    second correct bf16 computation of the same step: every sum over the batch
    runs in another order).  The north star's |dloss| <= 1e-3 over 40 steps
    sits below that spread."""
    import torch
    import torch.nn as nn
    from rdna4_conv3d import Conv3dWmma, ConvTranspose3dWmma
    from rdna4_conv3d.fused import BatchNormReLU3d, MaxPool3dWmma
    g = torch.Generator().manual_seed(0)
    x = torch.randn(batch, 1, 64, 128, 128, generator=g).cuda()
    labels = torch.randint(0, 2, (batch, 64, 128, 128), generator=torch.Generator().manual_seed(3)).cuda()
    amp = amp_dtype or torch.bfloat16
    ms_w, loss_w = unet3d_train(Conv3dWmma, ConvTranspose3dWmma, base, x, labels, steps, warmup, amp_dtype=amp)
    torch.cuda.empty_cache()
    ms_f, loss_f = unet3d_train(Conv3dWmma, ConvTranspose3dWmma, base, x, labels, steps, warmup, amp_dtype=amp,
                                bnrelu=BatchNormReLU3d, pool=MaxPool3dWmma, cat_free=True)
    torch.cuda.empty_cache()
    ms_s, loss_s = unet3d_train(nn.Conv3d, nn.ConvTranspose3d, base, x, labels, steps, warmup, amp_dtype=amp)
    torch.cuda.empty_cache()
    rev = torch.arange(batch - 1, -1, -1, device=x.device)
    _, loss_r = unet3d_train(nn.Conv3d, nn.ConvTranspose3d, base, x[rev].contiguous(), labels[rev].contiguous(),
                             steps, warmup, amp_dtype=amp)
    torch.cuda.empty_cache()
    n40 = min(40, len(loss_s))

    def gap(a, b):  # None when a loss is not finite (no NaN in the JSON line)
        d = [abs(u - v) for u, v in zip(a[:n40], b[:n40])]
        return round(max(d), 6) if all(math.isfinite(v) for v in d) else None

    def fin(v):
        return round(v, 6) if math.isfinite(v) else None

    amp_name = "fp16" if amp == torch.float16 else "bf16"
    return {
        "config": f"base={base} b{batch} x[{batch},1,64,128,128] AMP {amp_name}, CrossEntropy, Adam lr 1e-3, NCDHW",
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_w, 3),
        "ms_per_sample": round(ms_w / batch, 3),
        "stock_ms_per_step": round(ms_s, 3),
        "speedup_vs_stock": round(ms_s / ms_w, 3),
        "all_native_layers": "Conv3dWmma (decoder skip concatenation through forward_cat), ConvTranspose3dWmma, "
                             "BatchNormReLU3d, MaxPool3dWmma",
        "all_native_ms_per_step": round(ms_f, 3),
        "all_native_ms_per_sample": round(ms_f / batch, 3),
        "all_native_speedup_vs_stock": round(ms_s / ms_f, 3),
        "loss_steps_compared": n40,
        "max_abs_dloss": gap(loss_w, loss_s),
        "max_abs_dloss_all_native": gap(loss_f, loss_s),
        "max_abs_dloss_stock_vs_stock_batch_reversed": gap(loss_r, loss_s),
        "final_loss": fin(loss_w[-1]),
        "stock_final_loss": fin(loss_s[-1]),
    }


def unet_probe(name: str) -> int:
    """Kernels of UNet3D training steps for a kernel trace (rocprofv3
    --kernel-trace --stats): `unet<base>[_fused|_stock]` runs 3 warmup + 5 AMP
    bf16 steps of BASELINE config 5 built with this package's layers (with its
    BatchNorm + ReLU, MaxPool3d(2) and concatenation-free decoder convs as well
    for _fused, stock layers for _stock)."""
    import torch
    import torch.nn as nn
    from rdna4_conv3d import Conv3dWmma, ConvTranspose3dWmma
    from rdna4_conv3d.fused import BatchNormReLU3d, MaxPool3dWmma
    stem, _, kind = name.partition("_")
    base = int(stem[4:] or 24)
    g = torch.Generator().manual_seed(0)
    x = torch.randn(4, 1, 64, 128, 128, generator=g).cuda()
    labels = torch.randint(0, 2, (4, 64, 128, 128), generator=torch.Generator().manual_seed(3)).cuda()
    if kind == "stock":
        ms, _ = unet3d_train(nn.Conv3d, nn.ConvTranspose3d, base, x, labels, 5, 3)
    else:
        ms, _ = unet3d_train(Conv3dWmma, ConvTranspose3dWmma, base, x, labels, 5, 3,
                             bnrelu=BatchNormReLU3d if kind == "fused" else None,
                             pool=MaxPool3dWmma if kind == "fused" else None, cat_free=kind == "fused")
    print(f"probe {name}: {ms:.3f} ms/step", flush=True)
    return 0


def mfma_probe() -> int:
    """MFMA shape throughput on this GPU (bf16, dense): the library's probe
    kernel issues independent MFMAs of one shape from every wave; prints one
    JSON line per (shape, waves per SIMD) with TFLOP/s and the fraction of the
    published 2.5 PFLOP/s.  The basis for building every k=3 kernel on
    v_mfma_f32_32x32x16 rather than 16x16x32."""
    import torch
    from rdna4_conv3d import _native as nat
    dev = torch.device("cuda", 0)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 4096
    for shape, name, flops_per, per_round in ((0, "32x32x16", 32768, 4), (1, "16x16x32", 16384, 8)):
        for wps in (1, 2, 4):  # waves per SIMD: 4 SIMDs per CU, 4 waves per 256-thread workgroup
            blocks = cus * wps
            out = torch.empty(blocks * 256, device=dev, dtype=torch.float32)
            nat.probe_mfma(shape, blocks, 64, out)  # warm-up
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            nat.probe_mfma(shape, blocks, iters, out)
            e1.record()
            torch.cuda.synchronize()
            ms = e0.elapsed_time(e1)
            flops = blocks * 4 * iters * per_round * flops_per
            tf = flops / (ms * 1e-3) / 1e12
            print(json.dumps({"probe": "mfma", "shape": f"v_mfma_f32_{name}_bf16", "waves_per_simd": wps,
                              "cus": cus, "iters": iters, "ms": round(ms, 3), "tflops": round(tf, 1),
                              "frac_peak": round(tf / MFMA_PEAK_TFLOPS, 4)}), flush=True)
    return 0


def traffic_probe(name: str, layout: str) -> int:
    """Kernels for an HBM-traffic measurement (run under rocprofv3 --pmc): a
    256 MiB device copy three times (FETCH_SIZE / WRITE_SIZE calibration), then
    the trunk pass `name` (k3_<ci>to<co>_<fwd|dx|dw>) or the strided pass
    (k3s2_24to48_<fwd|dx|dw>, STRIDED) three times."""
    import torch
    from rdna4_conv3d import _native as nat
    dev = torch.device("cuda", 0)
    a = torch.empty(256 << 20, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b
    stem, p = name.rsplit("_", 1)
    n, ci, co, d, h, w, st, pd = STRIDED
    strided = stem == f"k3s2_{ci}to{co}"
    if not strided:
        for (n, ci, co, d, h, w) in TRUNK:
            if stem == f"k3_{ci}to{co}":
                break
        else:
            print(f"bench.py: unknown probe pass {name}", file=sys.stderr)
            return 2

    def L(t):
        return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()
    x = L(_gen((n, ci, d, h, w), 0, torch.bfloat16).to(dev))
    wt = _kaiming((co, ci, 3, 3, 3), ci * 27, 1, torch.bfloat16).to(dev)
    bias = _kaiming((co,), ci * 27, 3, torch.bfloat16).to(dev)
    y_shape = nat.strided_out_shape(x.shape, wt.shape, st, pd) if strided else (n, co, d, h, w)
    go = L(_gen(y_shape, 2, torch.bfloat16).to(dev))
    for _ in range(3):
        if strided and p == "fwd":
            nat.conv3d_strided_fwd(x, wt, bias, st, pd)
        elif strided and p == "dx":
            nat.conv3d_strided_dx(go, wt, x.shape, st, pd, like=x)
        elif strided:
            nat.conv3d_strided_dw(x, go, wt.shape, st, pd, torch.float32, want_db=True, db_dtype=torch.float32)
        elif p == "fwd":
            nat.conv3d_fwd(x, wt, bias, (1, 1, 1))
        elif p == "dx":
            nat.conv3d_dx(go, wt, x.shape, (1, 1, 1), like=x)
        else:
            nat.conv3d_dw(x, go, wt.shape, (1, 1, 1), torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    print(f"probe {name} {layout} done", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--preheat", type=float, default=1.0,
                    help="seconds of further untimed trunk steps after the warmup (clocks reach steady state)")
    ap.add_argument("--layout", choices=("ncdhw", "ndhwc"), default="ncdhw")
    ap.add_argument("--cpu-budget", type=float, default=12.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--unet-steps", type=int, default=40, help="UNet3D config-5 timed steps (0 skips it)")
    ap.add_argument("--no-hbm-passes", action="store_true", help="skip the k=1 / ConvTranspose3d passes")
    ap.add_argument("--unet-fp16", action="store_true",
                    help="also run config 5 under fp16 autocast (the reference's protocol; MIOpen's fp16 kernels "
                         "are built on first use, which adds minutes on a fresh box)")
    ap.add_argument("--probe", default=None, metavar="PASS",
                    help="traffic probe for rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE: a 256 MiB Tensor.copy_ (the "
                         "calibration) three times, then one trunk pass three times, e.g. k3_24to24_fwd, or the "
                         "strided pass, k3s2_24to48_dw; or "
                         "unet24[_fused|_stock]: 8 UNet3D training steps for a kernel trace; or mfma: "
                         "MFMA shape throughput (32x32x16 vs 16x16x32); exits")
    ap.add_argument("--no-kernel-timing", action="store_true",
                    help="diagnostic: time the step without the per-launch event hook (no roofline/passes)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (the hot path runs on a single MI355X; "
              "multi-GPU sharding is a design note, not a measured configuration). Use --gpus 1.",
              file=sys.stderr, flush=True)
        return 2

    import torch
    from rdna4_conv3d import _native as nat

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    nat.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    arch = torch.cuda.get_device_properties(0).gcnArchName
    if not nat.device_supported(0):
        print(f"bench.py: device {arch} is not gfx950", file=sys.stderr)
        return 1
    layout = args.layout

    def L(t):
        return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()

    if args.probe == "mfma":
        return mfma_probe()
    if args.probe and args.probe.startswith("unet"):
        return unet_probe(args.probe)
    if args.probe:
        return traffic_probe(args.probe, layout)

    layers = []
    for li, (n, ci, co, d, h, w) in enumerate(TRUNK):
        x = L(_gen((n, ci, d, h, w), 0, torch.bfloat16).to(dev))
        go = L(_gen((n, co, d, h, w), 2, torch.bfloat16).to(dev))
        wt = _kaiming((co, ci, 3, 3, 3), ci * 27, 1, torch.bfloat16).to(dev)
        b = _kaiming((co,), ci * 27, 3, torch.bfloat16).to(dev)
        layers.append((x, go, wt, b, _flops(n, ci, co, d, h, w)))
    pad = (1, 1, 1)

    def step():
        for li, (x, go, wt, b, _) in enumerate(layers):
            nat.timing_tag(li * 3 + 0)
            nat.conv3d_fwd(x, wt, b, pad)
            nat.timing_tag(li * 3 + 1)
            nat.conv3d_dx(go, wt, x.shape, pad, like=x)
            nat.timing_tag(li * 3 + 2)
            nat.conv3d_dw(x, go, wt.shape, pad, torch.float32, want_db=True, db_dtype=torch.float32)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # Steady state: the GPU's clocks settle within about half a second of
    # sustained load (measured: 1.204 ms/step right after 5 warmup steps,
    # 1.139-1.145 ms/step from 0.6 s on); keep stepping, untimed, for
    # --preheat seconds before the per-pass profile and the timed steps.
    pre_steps = 0
    t_pre = time.perf_counter()
    while time.perf_counter() - t_pre < args.preheat:
        step()
        pre_steps += 1
        if pre_steps % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()

    step_flops = 3 * sum(l[4] for l in layers)

    # Kernel profile: every launch of a few untimed steps is bracketed by HIP
    # events on its launch stream -> per-pass kernel times and the dominant
    # kernel (largest share of the step).
    passes = {}
    dominant = None
    if not args.no_kernel_timing:
        nat.timing_filter(-1, None)
        nat.timing_enable(True)
        nat.timing_collect()
        for _ in range(max(3, min(args.steps, 10))):
            step()
        torch.cuda.synchronize()
        recs = nat.timing_collect()
        nat.timing_enable(False)
        per = {}
        for tag, kind, ms in recs:
            per.setdefault((tag, kind), []).append(ms)
        for li, (n, ci, co, d, h, w) in enumerate(TRUNK):
            for pi, p in enumerate(PASSES):
                tag = li * 3 + pi
                main_kind = "wgrad" if p == "dw" else "row"
                main = per.get((tag, main_kind), [])
                aux = sum(sum(v) for (t, k), v in per.items() if t == tag and k != main_kind) / max(1, len(main))
                if not main:
                    continue
                avg = sum(main) / len(main)
                fl = layers[li][4]
                name = f"k3_{ci}to{co}_{d}x{h}x{w}_{p}"
                aux_kinds = {}
                for (t, k), v in per.items():
                    if t == tag and k != main_kind:
                        aux_kinds[k] = round(sum(v) / max(1, len(main)) * 1e3, 2)
                passes[name] = {
                    "kernel_us": round(avg * 1e3, 2),
                    "aux_us": round(aux * 1e3, 2),
                    "aux_by_kind_us": aux_kinds,
                    "tflops": round(fl / (avg * 1e-3) / 1e12, 1),
                    "frac_mfma": round(fl / (avg * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                    # the whole pass: main kernel plus its weight pack, reduce, copies, split epilogue
                    "frac_mfma_with_aux": round(fl / ((avg + aux) * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
                }
                share = avg * len(main)
                if dominant is None or share > dominant[0]:
                    dominant = (share, name, tag, main_kind, fl)
        # Timed region: only the dominant kernel's launches carry events, so
        # the hook does not slow the step it measures.
        nat.timing_filter(dominant[2], dominant[3])
        nat.timing_enable(True)
        nat.timing_collect()

    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(args.steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    drecs = nat.timing_collect() if not args.no_kernel_timing else []
    nat.timing_enable(False)
    nat.timing_filter(-1, None)
    ms_step = e0.elapsed_time(e1) / args.steps
    value = step_flops / (ms_step * 1e-3) / 1e12

    if dominant is None:  # --no-kernel-timing
        print(json.dumps({"metric": "step time without the kernel timing hook (diagnostic)",
                          "ms_per_step": round(ms_step, 4), "value": round(value, 2), "unit": "TFLOP/s"}), flush=True)
        return 0
    _, dname, _, _, dfl = dominant
    dms = [ms for _, _, ms in drecs if ms > 0]
    davg = sum(dms) / len(dms)
    achieved = dfl / (davg * 1e-3) / 1e12
    traffic = None
    tfile = ROOT / "profiles" / "traffic.json"
    if tfile.exists():
        try:
            traffic = json.loads(tfile.read_text()).get(dname)
        except (ValueError, OSError):
            traffic = None
    roofline = {
        "bound": "mfma",
        "kernel": dname,
        "achieved": round(achieved, 2),
        "peak": MFMA_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_PEAK_TFLOPS, 4),
        "traffic": traffic,
        "avg_launch_us": round(davg * 1e3, 2),
        "launches_timed": len(dms),
        "flops_per_launch": dfl,
    }

    del layers
    torch.cuda.empty_cache()
    hbm = None if args.no_hbm_passes else hbm_passes(layout)
    strided = None if args.no_hbm_passes else strided_passes(layout)
    unet = unet3d_bench(args.unet_steps, 3) if args.unet_steps > 0 else None
    unet32 = unet3d_bench(args.unet_steps, 3, base=32) if args.unet_steps > 0 else None
    unet16 = unet3d_bench(args.unet_steps, 3, amp_dtype=torch.float16) if args.unet_steps > 0 and args.unet_fp16 else None

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_budget)

    line = {
        "metric": "Conv3d fwd/dW/dX TFLOP/s (% MFMA peak); UNet3D b4 ms/sample",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "preheat_s": args.preheat,
        "preheat_steps": pre_steps,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "unet3d_trunk_k3_fwd_dx_dw",
            "shapes": ["[4,24,64,128,128]->24", "[4,48,32,64,64]->48", "[4,96,16,32,32]->96",
                       "[4,192,8,16,16]->192"],
            "layout": layout,
            "padding": 1,
            "step": "fwd + dX + dW(+db) per layer",
            "flops_per_step": step_flops,
            "device": arch,
            "wall_s": round(wall, 3),
        },
        "roofline": roofline,
        "passes": passes,
        "hbm_passes": hbm,
        "strided_passes": strided,
        "unet3d": unet,
        "unet3d_base32": unet32,
        "unet3d_fp16": unet16,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
