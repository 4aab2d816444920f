"""Native Conv3d with stride > 1 (the downsampling convolution).

The reference's policy admits stride 1 only (``_geom_ok``,
src/rdna4_conv3d/conv3d_wmma.py:89-95): a strided ``Conv3dWmma`` runs
``nn.Conv3d.forward`` and its autograd.  That contract is kept
(``conv3d_plan(..., stride=2)`` still answers ``miopen``).  This module is the
opt-in widening: ``StridedConv3dWmma`` is a drop-in for ``nn.Conv3d`` (same
parameters and state dict) whose forward, dX and dW run the library's
``r3c_conv3d_strided_*`` entry points on a gfx950 GPU for kernel 1 or 3,
stride 1 .. 8 per dimension, dilation 1, groups 1, zero padding, fp16 / bf16
(fp32 without autocast computes in fp16 and returns fp32, as the reference's
Conv3dWmmaFn does, conv3d_wmma.py:1244-1248).  Anything else runs
``nn.Conv3d.forward``.  ``swap_strided_conv3d`` swaps the strided
``nn.Conv3d`` children of a module tree (``swap_conv3d`` keeps its reference
semantics and leaves them alone).
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from rdna4_conv3d import _native
from rdna4_conv3d.conv3d_wmma import _HALF, _autocast_args, _db_dtype, _ensure_native, _t3, _wmma_hw


def _dense_or_cl(t: torch.Tensor) -> bool:
    return t.is_contiguous() or t.is_contiguous(memory_format=torch.channels_last_3d)


def strided_native_ok(x: torch.Tensor, weight: torch.Tensor, stride, padding, dilation=1, groups=1) -> bool:
    """The native strided path applies to this call (geometry, tensors, plans)."""
    if groups != 1 or isinstance(padding, str) or not _wmma_hw():
        return False
    if x.dim() != 5 or weight.dim() != 5 or not x.is_cuda or x.numel() == 0 or not weight.is_cuda:
        return False
    ks, st, pd = tuple(int(v) for v in weight.shape[2:]), _t3(stride), _t3(padding)
    if ks not in ((1, 1, 1), (3, 3, 3)) or _t3(dilation) != (1, 1, 1) or int(x.shape[1]) != int(weight.shape[1]):
        return False
    if any(s < 1 or s > 8 for s in st) or any(p < 0 or p > 64 for p in pd):
        return False
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        return False
    compute = x.dtype if x.dtype in _HALF else torch.float16
    return _native.strided_plans_ok(x, weight.shape, st, pd, compute)


class StridedConv3dFn(torch.autograd.Function):
    """Strided Conv3d on the native kernels; setup_context saves the tensors."""

    @staticmethod
    def forward(x, weight, bias, stride, padding):
        _ensure_native(x.device)
        compute = x.dtype
        if compute not in _HALF:
            x, weight = x.to(torch.float16), weight.to(torch.float16)
            bias = None if bias is None else bias.to(torch.float16)
        else:
            weight = weight.to(compute)
            bias = None if bias is None else bias.to(compute)
        with torch.cuda.device(x.device):
            y = _native.conv3d_strided_fwd(x, weight, bias, stride, padding)
        return y if compute in _HALF else y.to(compute)

    @staticmethod
    def setup_context(ctx, inputs, output):
        x, weight, bias, stride, padding = inputs
        ctx.save_for_backward(x, weight)
        ctx.has_bias = bias is not None
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.stride = stride
        ctx.padding = padding

    @staticmethod
    def backward(ctx, grad_out):
        x, weight = ctx.saved_tensors
        need_x, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        need_b = ctx.needs_input_grad[2] and ctx.has_bias
        half = x.dtype if x.dtype in _HALF else torch.float16
        go = grad_out if grad_out.dtype == half else grad_out.to(half)
        if not _dense_or_cl(go):
            go = go.contiguous()
        gx = dw = db = None
        with torch.cuda.device(x.device):
            if need_x:
                w_c = weight if weight.dtype == half else weight.to(half)
                gx = _native.conv3d_strided_dx(go, w_c, x.shape, ctx.stride, ctx.padding, like=x)
                if gx.dtype != x.dtype:
                    gx = gx.to(x.dtype)
            if need_w or need_b:
                x_c = x if x.dtype == half else x.to(half)
                dw_dtype = weight.dtype if weight.dtype == half else torch.float32
                dw, db = _native.conv3d_strided_dw(x_c, go, weight.shape, ctx.stride, ctx.padding, dw_dtype,
                                                   want_db=need_b, db_dtype=_db_dtype(ctx.bias_dtype, half))
                dw = dw.to(weight.dtype) if need_w else None
                if need_b and db.dtype != ctx.bias_dtype:
                    db = db.to(ctx.bias_dtype)
        return gx, dw, db, None, None


def conv3d_strided(x, weight, bias=None, stride=2, padding=0, dilation=1, groups=1):
    """Functional form: F.conv3d semantics; native where strided_native_ok."""
    xa, wa, ba = _autocast_args(x, weight, bias)
    if not strided_native_ok(xa, wa, stride, padding, dilation, groups):
        return F.conv3d(x, weight, bias, stride, padding, dilation, groups)
    return StridedConv3dFn.apply(xa, wa, ba, _t3(stride), _t3(padding))


class StridedConv3dWmma(nn.Conv3d):
    """nn.Conv3d whose strided forward / backward run the native kernels."""

    def forward(self, x):
        if self.padding_mode != "zeros" or isinstance(self.padding, str):
            return super().forward(x)
        xa, wa, ba = _autocast_args(x, self.weight, self.bias)
        if not strided_native_ok(xa, wa, self.stride, self.padding, self.dilation, self.groups):
            return super().forward(x)
        return StridedConv3dFn.apply(xa, wa, ba, _t3(self.stride), _t3(self.padding))


def swap_strided_conv3d(module: nn.Module) -> int:
    """Replace every exact-type nn.Conv3d child with stride != 1 by a
    StridedConv3dWmma holding the same parameters (device, dtype and
    padding_mode kept); returns the count.  Recursive."""
    count = 0
    for name, child in module.named_children():
        if type(child) is nn.Conv3d and _t3(child.stride) != (1, 1, 1):
            new = StridedConv3dWmma(child.in_channels, child.out_channels, child.kernel_size, stride=child.stride,
                                    padding=child.padding, dilation=child.dilation, groups=child.groups,
                                    bias=child.bias is not None, padding_mode=child.padding_mode,
                                    device=child.weight.device, dtype=child.weight.dtype)
            new.load_state_dict(child.state_dict())
            setattr(module, name, new)
            count += 1
        else:
            count += swap_strided_conv3d(child)
    return count
