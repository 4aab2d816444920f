"""Drop-in Conv3d / ConvTranspose3d for MI355X (gfx950) on hand-written HIP MFMA kernels.

Public surface (names, signatures and semantics follow the reference module
src/rdna4_conv3d/conv3d_wmma.py):

  Conv3dWmma, ConvTranspose3dWmma          nn.Conv3d / nn.ConvTranspose3d subclasses
  conv3d_wmma(x, w, b, stride, padding, dilation, groups)
  wmma_fwd / wmma_dw / wmma_dx             isolated passes
  wmma_ok_fwd / wmma_ok_dw / wmma_ok_dx, conv3d_plan, swap_conv3d

Dispatch policy (reference conv3d_wmma.py:44-139):
  RDNA4_CONV3D_BACKEND (alias BIOHUB_CONV3D_BACKEND) = hybrid (default) | wmma | hip |
  miopen | torch.  hybrid/hip: native kernels on gfx950 for k=1 / k=3, stride 1,
  dilation 1, groups 1; everything else runs the stock PyTorch path
  (F.conv3d -> MIOpen on GPU, oneDNN on CPU).  wmma forces the native path for
  every supported geometry.  miopen / torch force the stock path.

The compute path is the C-ABI library librdna4_conv3d_hip.so (bound in
_native.py).  On a gfx950 GPU with a native backend selected, a missing library
is an error, not a silent fallback.

Deliberate differences from the reference (each one a reference quirk):
  * k=3 dX uses padding k-1-p (the reference reuses p, correct only for p=1).
  * dW is accumulated and returned in fp32 for fp32 parameters (the reference
    rounds it through the activation dtype first).
  * ConvTranspose3dWmma honours the backend variable, the arch gate, dilation
    and output_size (falling back when they do not fit k=2 s=2).
  * Conv3dWmma falls back for padding_mode != 'zeros' and string padding;
    swap_conv3d keeps device, dtype and padding_mode.
  * The arch check is cached once per device.
"""
from __future__ import annotations

import os
import warnings
from functools import lru_cache
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from rdna4_conv3d import _native

# ---------------------------------------------------------------------------
# Policy (reference conv3d_wmma.py:44-139)
# ---------------------------------------------------------------------------

_NATIVE_BACKENDS = ("hybrid", "wmma", "hip")
_STOCK_BACKENDS = ("miopen", "torch")


def _t3(v) -> Tuple[int, int, int]:
    if isinstance(v, int):
        return (v, v, v)
    return tuple(int(x) for x in v)


def _backend_name() -> str:
    return (
        os.environ.get("RDNA4_CONV3D_BACKEND")
        or os.environ.get("BIOHUB_CONV3D_BACKEND")
        or "hybrid"
    ).lower()


_BACKEND = _backend_name()


@lru_cache(maxsize=None)
def _arch_name(device_index: int) -> str:
    return getattr(torch.cuda.get_device_properties(device_index), "gcnArchName", "") or ""


def _is_gfx950(device_index: Optional[int] = None) -> bool:
    """Arch gate (the reference's _is_rdna4, conv3d_wmma.py:44-48), cached per device."""
    if not torch.cuda.is_available():
        return False
    idx = torch.cuda.current_device() if device_index is None else int(device_index)
    return _arch_name(idx).startswith("gfx950")


def _wmma_hw() -> bool:
    """True when the native kernels should run (reference conv3d_wmma.py:79-86)."""
    if _BACKEND in _STOCK_BACKENDS:
        return False
    if _BACKEND == "wmma":
        return True
    return _is_gfx950()


def _geom_ok(kernel_size, stride, dilation, groups) -> bool:
    """groups 1, stride 1, dilation 1, kernel 1x1x1 or 3x3x3 (conv3d_wmma.py:89-95)."""
    if int(groups) != 1:
        return False
    ks, st, dl = _t3(kernel_size), _t3(stride), _t3(dilation)
    if dl != (1, 1, 1) or st != (1, 1, 1):
        return False
    return ks in ((1, 1, 1), (3, 3, 3))


def wmma_ok_fwd(cin, cout, kernel_size, stride=1, dilation=1, groups=1) -> bool:
    return _wmma_hw() and _geom_ok(kernel_size, stride, dilation, groups)


def wmma_ok_dw(cin, cout, kernel_size, stride=1, dilation=1, groups=1) -> bool:
    return wmma_ok_fwd(cin, cout, kernel_size, stride, dilation, groups)


def wmma_ok_dx(cin, cout, kernel_size, stride=1, dilation=1, groups=1) -> bool:
    """Every supported dX geometry runs natively, skinny layers included.

    The reference settled this end-to-end (conv3d_wmma.py:106-128): per-layer
    isolated timings misjudge behaviour inside a training step.
    """
    return wmma_ok_fwd(cin, cout, kernel_size, stride, dilation, groups)


def conv3d_plan(cin, cout, kernel_size, stride=1, dilation=1, groups=1) -> dict:
    """Which backend runs each leg. Values are 'wmma' (native) or 'miopen' (stock)."""
    ks, st, dl, g = kernel_size, stride, dilation, groups
    return {
        "fwd": "wmma" if wmma_ok_fwd(cin, cout, ks, st, dl, g) else "miopen",
        "dw": "wmma" if wmma_ok_dw(cin, cout, ks, st, dl, g) else "miopen",
        "dx": "wmma" if wmma_ok_dx(cin, cout, ks, st, dl, g) else "miopen",
    }


def _out_size(L, k, stride, pad, dil):
    return (L + 2 * pad - dil * (k - 1) - 1) // stride + 1


_HALF = (torch.float16, torch.bfloat16)


def _native_tensors_ok(*ts) -> bool:
    """Tensors the native kernels accept: CUDA, 5-D where relevant, non-empty."""
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda or t.numel() == 0:
            return False
    return True


def _conv_native_ok(x, weight, stride, padding, dilation) -> bool:
    """Full native-path predicate for one Conv3d call (geometry, padding, tensors)."""
    if x.dim() != 5 or weight.dim() != 5:
        return False
    ks = (int(weight.shape[2]), int(weight.shape[3]), int(weight.shape[4]))
    cin, cout = int(x.shape[1]), int(weight.shape[0])
    if cin != int(weight.shape[1]):
        return False
    if not wmma_ok_fwd(cin, cout, ks, stride, dilation, 1):
        return False
    pd = _t3(padding)
    if any(p < 0 or p > 64 for p in pd):
        return False
    sp = tuple(int(s) for s in x.shape[2:])
    if any(_out_size(L, ks[0], 1, p, 1) < 1 for L, p in zip(sp, pd)):
        return False
    if not _native_tensors_ok(x, weight):
        return False
    # The library must have plans for all three passes (e.g. not for a sample
    # of 1 GiB or more); decided here, before the forward runs, so a native
    # forward is never followed by an unsupported backward.
    compute = x.dtype if x.dtype in _HALF else torch.float16
    return _native.conv_plans_ok(x, weight.shape, pd, compute)


_warned = set()


def _fallback_warning(what: str, err: Exception) -> None:
    """One warning per call site when the library declines a call it was
    expected to run (R3C_UNSUPPORTED); the stock PyTorch routine runs instead."""
    if what not in _warned:
        _warned.add(what)
        warnings.warn(f"rdna4_conv3d: {what} runs the stock PyTorch path: {err}", RuntimeWarning, stacklevel=3)


def _ensure_native(device: torch.device) -> None:
    """On the native path the library must exist and the device must be gfx950."""
    _native.load()
    if not _native.device_supported(device.index if device.index is not None else torch.cuda.current_device()):
        raise RuntimeError(
            f"rdna4_conv3d: native kernels need a gfx950 GPU, got {_arch_name(device.index or 0)!r} "
            f"(backend {_BACKEND!r}); set RDNA4_CONV3D_BACKEND=torch to use the stock path")


def _layout_of(x: torch.Tensor):
    if x.dim() == 5 and x.is_contiguous(memory_format=torch.channels_last_3d) and not x.is_contiguous():
        return torch.channels_last_3d
    return torch.contiguous_format


# ---------------------------------------------------------------------------
# Autograd Function: Conv3d (reference conv3d_wmma.py:1233-1319)
# ---------------------------------------------------------------------------
class Conv3dWmmaFn(torch.autograd.Function):
    """Conv3d on the native kernels.  Tensors are saved in setup_context (AMP-safe)."""

    @staticmethod
    def forward(x, weight, bias, stride, padding, dilation):
        if not _conv_native_ok(x, weight, stride, padding, dilation):
            return F.conv3d(x, weight, bias, stride, padding, dilation)
        _ensure_native(x.device)
        compute_dtype = x.dtype
        if compute_dtype not in _HALF:
            # fp32 without autocast computes in fp16 and returns fp32 (conv3d_wmma.py:1244-1248).
            x = x.to(torch.float16)
            weight = weight.to(torch.float16)
            bias = None if bias is None else bias.to(torch.float16)
        else:
            weight = weight.to(compute_dtype)
            bias = None if bias is None else bias.to(compute_dtype)
        try:
            with torch.cuda.device(x.device):
                y = _native.conv3d_fwd(x, weight, bias, _t3(padding))
        except _native.NativeUnsupported as e:
            _fallback_warning("Conv3d forward", e)
            y = F.conv3d(x, weight, bias, stride, padding, dilation)
        if compute_dtype not in _HALF:
            y = y.to(compute_dtype)
        return y

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, weight, bias, stride, padding, dilation = inputs
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.stride = stride
        ctx.padding = padding
        ctx.dilation = dilation
        ctx.native = _conv_native_ok(x, weight, stride, padding, dilation)

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        stride, padding, dilation = ctx.stride, ctx.padding, ctx.dilation
        need_x, need_w, need_b = ctx.needs_input_grad[0], ctx.needs_input_grad[1], ctx.needs_input_grad[2]
        need_b = need_b and ctx.has_bias
        gx = dw = db = None
        if not ctx.native:
            go = grad_out
            if need_x:
                gx = _stock_dx(x, weight, go, stride, padding, dilation)
            if need_w:
                dw = _stock_dw(x, weight, go, stride, padding, dilation)
            if need_b:
                db = go.sum(dim=(0, 2, 3, 4)).to(ctx.bias_dtype)
            return gx, dw, db, None, None, None

        _ensure_native(x.device)
        half = x.dtype if x.dtype in _HALF else torch.float16
        go = grad_out if grad_out.dtype == half else grad_out.to(half)
        pad3 = _t3(padding)
        with torch.cuda.device(x.device):
            if need_x:
                w_c = weight if weight.dtype == half else weight.to(half)
                try:
                    gx = _native.conv3d_dx(go, w_c, x.shape, pad3, like=x)
                except _native.NativeUnsupported as e:
                    _fallback_warning("Conv3d dX", e)
                    gx = _stock_dx(x, w_c, go, stride, padding, dilation)
                if gx.dtype != x.dtype:
                    gx = gx.to(x.dtype)
            if need_w:
                x_c = x if x.dtype == half else x.to(half)
                dw_dtype = weight.dtype if weight.dtype == half else torch.float32
                try:
                    dw, db = _native.conv3d_dw(x_c, go, weight.shape, pad3, dw_dtype, want_db=need_b,
                                               db_dtype=_db_dtype(ctx.bias_dtype, half))
                except _native.NativeUnsupported as e:
                    _fallback_warning("Conv3d dW", e)
                    dw, db = _stock_dw(x_c, weight, go, stride, padding, dilation), None
                if dw.dtype != weight.dtype:
                    dw = dw.to(weight.dtype)
            if need_b and db is None:
                db = go.float().sum(dim=(0, 2, 3, 4))
            if need_b and db is not None and db.dtype != ctx.bias_dtype:
                db = db.to(ctx.bias_dtype)
        return gx, dw, db, None, None, None


def _stock_dx(x, weight, go, stride, padding, dilation):
    """dX by PyTorch (MIOpen / oneDNN), in x's layout."""
    gx = torch.nn.grad.conv3d_input(x.shape, weight.to(go.dtype), go.contiguous(), stride, padding, dilation, 1)
    return _follow_layout(gx, x)


def _stock_dw(x, weight, go, stride, padding, dilation):
    """dW by PyTorch, in the weight's dtype."""
    return torch.nn.grad.conv3d_weight(x.to(go.dtype), weight.shape, go.contiguous(), stride, padding, dilation,
                                       1).to(weight.dtype)


def _db_dtype(bias_dtype, half):
    if bias_dtype in (torch.float32, torch.float16, torch.bfloat16):
        return bias_dtype
    return torch.float32


# ---------------------------------------------------------------------------
# Autocast (reference conv3d_wmma.py:1322-1358): cast OUTSIDE the Function, the
# way autocast treats nn.Conv3d, so the output stays in the autocast dtype.
# ---------------------------------------------------------------------------
def _autocast_dtype():
    try:
        if not torch.is_autocast_enabled("cuda"):
            return None
        dt = torch.get_autocast_dtype("cuda")
    except TypeError:  # older signature without device_type
        if not torch.is_autocast_enabled():
            return None
        dt = torch.get_autocast_gpu_dtype()
    return dt if dt in _HALF else None


def _autocast_args(x, weight, bias):
    """x in the autocast dtype; weight and bias stay in their parameter dtype.
    The autograd Functions cast them to the compute dtype for the kernels and
    return their gradients in that parameter dtype straight from the kernels
    (fp32 dW / db for fp32 master parameters), so the backward has no cast
    kernels (autocast's own weight cast would add a bf16 -> fp32 copy per
    gradient) and dW is not rounded to bf16 on the way."""
    dt = _autocast_dtype()
    if dt is None or not x.is_cuda:
        return x, weight, bias
    x = x.to(dt) if x.dtype != dt else x
    return x, weight, bias


def conv3d_wmma(x, weight, bias=None, stride=1, padding=0, dilation=1, groups=1):
    """Functional drop-in for F.conv3d (reference conv3d_wmma.py:1361-1365)."""
    if groups != 1 or isinstance(padding, str):
        return F.conv3d(x, weight, bias, stride, padding, dilation, groups)
    x, weight, bias = _autocast_args(x, weight, bias)
    return Conv3dWmmaFn.apply(x, weight, bias, _t3(stride), _t3(padding), _t3(dilation))


# ---------------------------------------------------------------------------
# Isolated passes (reference conv3d_wmma.py:1368-1409).  Unsupported
# geometries run the stock torch routine instead of raising.
# ---------------------------------------------------------------------------
def _follow_layout(t: torch.Tensor, like: torch.Tensor) -> torch.Tensor:
    if _layout_of(like) == torch.channels_last_3d:
        return t.contiguous(memory_format=torch.channels_last_3d)
    return t.contiguous()


def wmma_fwd(x, weight, bias=None, stride=1, padding=0, dilation=1):
    """Isolated forward. Returns NCDHW unless x is channels_last_3d."""
    st, pd, dl = _t3(stride), _t3(padding), _t3(dilation)
    if not _conv_native_ok(x, weight, st, pd, dl) or x.dtype not in _HALF:
        return _follow_layout(F.conv3d(x, weight, bias, st, pd, dl), x)
    _ensure_native(x.device)
    try:
        with torch.cuda.device(x.device):
            return _native.conv3d_fwd(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype), pd)
    except _native.NativeUnsupported as e:
        _fallback_warning("wmma_fwd", e)
        return _follow_layout(F.conv3d(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype), st, pd,
                                       dl), x)


def wmma_dw(x, weight, go, stride=1, padding=0, dilation=1):
    """Isolated dW. Returns OIDHW in go.dtype, like the reference's wmma_dw."""
    st, pd, dl = _t3(stride), _t3(padding), _t3(dilation)
    if not _conv_native_ok(x, weight, st, pd, dl) or go.dtype not in _HALF or x.dtype != go.dtype:
        return torch.nn.grad.conv3d_weight(x.to(go.dtype), weight.shape, go.contiguous(), st, pd, dl, 1)
    _ensure_native(x.device)
    try:
        with torch.cuda.device(x.device):
            dw, _ = _native.conv3d_dw(x, go, weight.shape, pd, go.dtype)
    except _native.NativeUnsupported as e:
        _fallback_warning("wmma_dw", e)
        dw = torch.nn.grad.conv3d_weight(x, weight.shape, go.contiguous(), st, pd, dl, 1)
    return dw


def wmma_dx(x, weight, go, stride=1, padding=0, dilation=1):
    """Isolated dX. Returns NCDHW unless x is channels_last_3d."""
    st, pd, dl = _t3(stride), _t3(padding), _t3(dilation)
    if not _conv_native_ok(x, weight, st, pd, dl) or go.dtype not in _HALF:
        w = weight if weight.dtype == go.dtype else weight.to(go.dtype)
        gx = torch.nn.grad.conv3d_input(x.shape, w, go.contiguous(), st, pd, dl, 1)
        return _follow_layout(gx, x)
    _ensure_native(x.device)
    try:
        with torch.cuda.device(x.device):
            return _native.conv3d_dx(go, weight.to(go.dtype), x.shape, pd, like=x)
    except _native.NativeUnsupported as e:
        _fallback_warning("wmma_dx", e)
        return _stock_dx(x, weight, go, st, pd, dl)


# ---------------------------------------------------------------------------
# nn.Module drop-ins (reference conv3d_wmma.py:1412-1443)
# ---------------------------------------------------------------------------
def swap_conv3d(module: nn.Module, transpose: bool = False) -> int:
    """Replace every nn.Conv3d (exact type) with Conv3dWmma, copying weights. Returns count.

    Device, dtype and padding_mode are preserved.  With transpose=True,
    nn.ConvTranspose3d modules are swapped for ConvTranspose3dWmma too (off by
    default, as in the reference, and not counted in the return value).
    """
    n = 0
    for name, child in list(module.named_children()):
        if type(child) is nn.Conv3d:
            new = Conv3dWmma(
                child.in_channels, child.out_channels, child.kernel_size,
                stride=child.stride, padding=child.padding,
                dilation=child.dilation, groups=child.groups,
                bias=child.bias is not None, padding_mode=child.padding_mode,
                device=child.weight.device, dtype=child.weight.dtype,
            )
            with torch.no_grad():
                new.weight.copy_(child.weight)
                if child.bias is not None:
                    new.bias.copy_(child.bias)
            new.train(child.training)
            setattr(module, name, new)
            n += 1
        elif transpose and type(child) is nn.ConvTranspose3d:
            new = ConvTranspose3dWmma(
                child.in_channels, child.out_channels, child.kernel_size,
                stride=child.stride, padding=child.padding, output_padding=child.output_padding,
                groups=child.groups, bias=child.bias is not None, dilation=child.dilation,
                padding_mode=child.padding_mode, device=child.weight.device, dtype=child.weight.dtype,
            )
            with torch.no_grad():
                new.weight.copy_(child.weight)
                if child.bias is not None:
                    new.bias.copy_(child.bias)
            new.train(child.training)
            setattr(module, name, new)
        else:
            n += swap_conv3d(child, transpose=transpose)
    return n


class Conv3dWmma(nn.Conv3d):
    """Drop-in nn.Conv3d: native gfx950 kernels where the plan says so, else nn.Conv3d."""

    def forward(self, x):
        if (self.groups != 1 or not x.is_cuda or self.padding_mode != "zeros"
                or isinstance(self.padding, str)):
            return super().forward(x)
        cin, cout = int(x.shape[1]), int(self.weight.shape[0])
        plan = conv3d_plan(cin, cout, self.kernel_size, self.stride, self.dilation, self.groups)
        if plan["fwd"] == "miopen" and plan["dw"] == "miopen" and plan["dx"] == "miopen":
            return super().forward(x)
        return conv3d_wmma(x, self.weight, self.bias, self.stride, self.padding, self.dilation, 1)

    def forward_cat(self, xa, xb):
        """self(torch.cat((xa, xb), 1)) without writing the concatenation: a
        k=3 stride-1 layer on contiguous NCDHW half-precision inputs (or under
        autocast) reads the two tensors directly and returns the gradients of
        xa and xb as two tensors.  Anything else concatenates and calls forward."""
        if not self._cat_native_ok(xa, xb):
            return self.forward(torch.cat((xa, xb), 1))
        xa, w, b = _autocast_args(xa, self.weight, self.bias)
        xb = xb.to(xa.dtype) if xb.dtype != xa.dtype else xb
        if xa.dtype not in _HALF:
            return self.forward(torch.cat((xa, xb), 1))
        _ensure_native(xa.device)
        return _Conv3dCatFn.apply(xa, xb, w, b, _t3(self.padding))

    def _cat_native_ok(self, xa, xb) -> bool:
        if (self.groups != 1 or self.padding_mode != "zeros" or isinstance(self.padding, str)
                or tuple(self.kernel_size) != (3, 3, 3) or _t3(self.stride) != (1, 1, 1)
                or _t3(self.dilation) != (1, 1, 1) or not _wmma_hw()):
            return False
        if not (_native_tensors_ok(xa, xb) and xa.dim() == 5 and xb.dim() == 5):
            return False
        if int(xa.shape[1]) + int(xb.shape[1]) != int(self.weight.shape[1]):
            return False
        dt = _autocast_dtype() or xa.dtype
        if dt not in _HALF or not (xa.dtype == xb.dtype and (xa.dtype == dt or _autocast_dtype() is not None)):
            return False
        if not _native.cat_tensors_ok(xa, xb):
            return False
        return _native.cat_plans_ok(xa, xb, self.weight.shape, _t3(self.padding), dt)


class _Conv3dCatFn(torch.autograd.Function):
    """k=3 Conv3d over cat(xa, xb) on the native kernels (xa, xb in the compute
    dtype; weight and bias in their parameter dtype, cast here for the kernels)."""

    @staticmethod
    def forward(ctx, xa, xb, weight, bias, padding):
        wc = weight if weight.dtype == xa.dtype else weight.to(xa.dtype)
        bc = bias if bias is None or bias.dtype == xa.dtype else bias.to(xa.dtype)
        with torch.cuda.device(xa.device):
            y = _native.conv3d_cat_fwd(xa, xb, wc, bc, padding)
        ctx.save_for_backward(xa, xb, weight)
        ctx.padding = padding
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        return y

    @staticmethod
    def backward(ctx, go):
        xa, xb, weight = ctx.saved_tensors
        go = go.to(xa.dtype).contiguous()
        need_a, need_b_in, need_w, need_bias = ctx.needs_input_grad[:4]
        dxa = dxb = dw = db = None
        with torch.cuda.device(xa.device):
            if need_a or need_b_in:
                wc = weight if weight.dtype == xa.dtype else weight.to(xa.dtype)
                dxa, dxb = _native.conv3d_cat_dx(go, wc, xa.shape, xb.shape, ctx.padding)
            if need_w or (need_bias and ctx.has_bias):
                dw, db = _native.conv3d_cat_dw(xa, xb, go, weight.shape, ctx.padding, torch.float32,
                                               want_db=need_bias and ctx.has_bias,
                                               db_dtype=_db_dtype(ctx.bias_dtype, xa.dtype))
                dw = dw.to(weight.dtype) if need_w else None
                if db is not None and db.dtype != ctx.bias_dtype:
                    db = db.to(ctx.bias_dtype)
        return dxa, dxb, dw, db, None


# ---------------------------------------------------------------------------
# ConvTranspose3d k=2 s=2 p=0 (reference conv3d_wmma.py:1446-1595)
# ---------------------------------------------------------------------------
def _convt_native_ok(x, weight) -> bool:
    if x.dim() != 5 or weight.dim() != 5 or tuple(weight.shape[2:]) != (2, 2, 2):
        return False
    if int(x.shape[1]) != int(weight.shape[0]):
        return False
    if not _native_tensors_ok(x, weight):
        return False
    compute = x.dtype if x.dtype in _HALF else torch.float16
    return _native.convt_plans_ok(x, weight.shape, compute)


def transpose_k2s2_fwd(x, weight, bias=None):
    """weight is PyTorch ConvTranspose3d layout (Cin, Cout, 2, 2, 2)."""
    _ensure_native(x.device)
    with torch.cuda.device(x.device):
        return _native.convt_fwd(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype))


def transpose_k2s2_dx(x_shape, weight, go, like=None):
    _ensure_native(go.device)
    with torch.cuda.device(go.device):
        return _native.convt_dx(go, weight.to(go.dtype), x_shape, like=go if like is None else like)


def transpose_k2s2_dw(x, weight_shape, go, dw_dtype=None):
    _ensure_native(x.device)
    with torch.cuda.device(x.device):
        dw, _ = _native.convt_dw(x, go, weight_shape, dw_dtype or go.dtype)
    return dw


def _stock_convt_grads(x, weight, go, need_x, need_w):
    """dX (x's layout) and dW (weight's dtype) of a k=2 s=2 ConvTranspose3d by PyTorch."""
    with torch.enable_grad():
        xr = x.detach().requires_grad_(need_x)
        wr = weight.detach().to(go.dtype).requires_grad_(need_w)
        y = F.conv_transpose3d(xr.to(go.dtype), wr, None, stride=2)
        ins = [t for t, n in ((xr, need_x), (wr, need_w)) if n]
        grads = list(torch.autograd.grad(y, ins, go))
    gx = _follow_layout(grads.pop(0), x) if need_x else None
    dw = grads.pop(0).to(weight.dtype) if need_w else None
    return gx, dw


class ConvTranspose3dWmmaFn(torch.autograd.Function):
    @staticmethod
    def forward(x, weight, bias):
        compute_dtype = x.dtype
        if compute_dtype not in _HALF:
            x = x.to(torch.float16)
            weight = weight.to(torch.float16)
            bias = None if bias is None else bias.to(torch.float16)
        try:
            y = transpose_k2s2_fwd(x, weight, bias)
        except _native.NativeUnsupported as e:
            _fallback_warning("ConvTranspose3d forward", e)
            y = F.conv_transpose3d(x, weight.to(x.dtype), None if bias is None else bias.to(x.dtype), stride=2)
        if compute_dtype not in _HALF:
            y = y.to(compute_dtype)
        return y

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, weight, bias = inputs
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_b = ctx.needs_input_grad[2] and ctx.has_bias
        half = x.dtype if x.dtype in _HALF else torch.float16
        go = grad_out if grad_out.dtype == half else grad_out.to(half)
        gx = dw = db = None
        _ensure_native(x.device)
        with torch.cuda.device(x.device):
            if need_x:
                w_c = weight if weight.dtype == half else weight.to(half)
                try:
                    gx = _native.convt_dx(go, w_c, x.shape, like=x)
                except _native.NativeUnsupported as e:
                    _fallback_warning("ConvTranspose3d dX", e)
                    gx, _ = _stock_convt_grads(x.to(half), w_c, go, True, False)
                if gx.dtype != x.dtype:
                    gx = gx.to(x.dtype)
            if need_w or need_b:
                x_c = x if x.dtype == half else x.to(half)
                dw_dtype = torch.float32 if weight.dtype == torch.float32 else half
                try:
                    dw, db = _native.convt_dw(x_c, go, weight.shape, dw_dtype, want_db=need_b,
                                              db_dtype=_db_dtype(ctx.bias_dtype, half))
                except _native.NativeUnsupported as e:
                    _fallback_warning("ConvTranspose3d dW", e)
                    _, dw = _stock_convt_grads(x_c, weight, go, False, True)
                    db = go.float().sum(dim=(0, 2, 3, 4)) if need_b else None
                dw = dw.to(weight.dtype) if need_w else None
                if need_b and db.dtype != ctx.bias_dtype:
                    db = db.to(ctx.bias_dtype)
        return gx, dw, db


class ConvTranspose3dWmma(nn.ConvTranspose3d):
    """k=2 s=2 pad=0 drop-in. Other configurations run nn.ConvTranspose3d."""

    def forward(self, x, output_size=None):
        if (output_size is not None or self.kernel_size != (2, 2, 2) or self.stride != (2, 2, 2)
                or self.padding != (0, 0, 0) or self.output_padding != (0, 0, 0) or self.groups != 1
                or self.dilation != (1, 1, 1) or self.padding_mode != "zeros" or not x.is_cuda
                or not _wmma_hw()):
            return super().forward(x, output_size)
        xa, weight, bias = _autocast_args(x, self.weight, self.bias)
        if not _convt_native_ok(xa, weight):
            return super().forward(x, output_size)
        return ConvTranspose3dWmmaFn.apply(xa, weight, bias)
