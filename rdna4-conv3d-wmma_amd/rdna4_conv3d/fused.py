"""Native BatchNorm3d + ReLU and MaxPool3d(2) for the UNet3D the reference
accelerates (reference benches/unet_e2e.py:13-37, examples/drop_in_unet.py).

BatchNormReLU3d is an opt-in replacement for the pair
``nn.BatchNorm3d(C), nn.ReLU(inplace=True)``: the same parameters, buffers
and state dict as nn.BatchNorm3d, PyTorch's training semantics (batch
statistics with the biased variance, running statistics updated with the
unbiased variance and ``momentum``, or the cumulative average when momentum is
None) and evaluation semantics (running statistics), followed by ReLU.  On a
gfx950 GPU, for tensors whose (sample, channel) planes are contiguous (NCDHW)
with fp32 parameters and buffers, it runs the library's BatchNorm + ReLU
kernels (r3c_bn_relu_fwd / r3c_bn_relu_bwd: one statistics pass and one
normalise + ReLU pass forward, one sums pass and one dY pass backward, each a
single stream over the tensors, every reduction in a fixed order).  Anything
else runs nn.BatchNorm3d followed by F.relu.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from rdna4_conv3d import _native
from rdna4_conv3d.conv3d_wmma import _ensure_native, _wmma_hw


class _BnReluFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, running_mean, running_var, training, momentum, eps):
        z, mean, invstd = _native.bn_relu_fwd(x, weight, bias, running_mean, running_var, training, momentum, eps)
        ctx.save_for_backward(x, weight, bias, mean, invstd)
        ctx.training = training
        return z

    @staticmethod
    def backward(ctx, dz):
        x, weight, bias, mean, invstd = ctx.saved_tensors
        if not _native.bn_plane_ok(dz) or dz.dtype != x.dtype:
            dz = dz.to(x.dtype).contiguous()
        need_w = ctx.needs_input_grad[1] and weight is not None
        need_b = ctx.needs_input_grad[2] and bias is not None
        dx, dg, db = _native.bn_relu_bwd(dz, x, weight, bias, mean, invstd, ctx.training, need_w, need_b)
        return dx, dg, db, None, None, None, None, None


class BatchNormReLU3d(nn.BatchNorm3d):
    """nn.BatchNorm3d followed by ReLU, on the native kernels where they apply."""

    def _native_ok(self, x: torch.Tensor) -> bool:
        if not (x.is_cuda and x.dim() == 5 and int(x.shape[1]) == self.num_features and x.numel() > 0):
            return False
        if not _wmma_hw() or x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            return False
        for t in (self.weight, self.bias, self.running_mean, self.running_var):
            if t is not None and (t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous()):
                return False
        return _native.bn_plane_ok(x)

    def forward(self, x):
        if not self._native_ok(x):
            return F.relu(super().forward(x))
        _ensure_native(x.device)
        # Momentum and buffer bookkeeping as in torch.nn.modules.batchnorm._BatchNorm.forward.
        factor = 0.0 if self.momentum is None else self.momentum
        if self.training and self.track_running_stats and self.num_batches_tracked is not None:
            self.num_batches_tracked.add_(1)
            factor = 1.0 / float(self.num_batches_tracked) if self.momentum is None else self.momentum
        bn_training = self.training or (self.running_mean is None and self.running_var is None)
        track = not self.training or self.track_running_stats
        rm = self.running_mean if track else None
        rv = self.running_var if track else None
        with torch.cuda.device(x.device):
            return _BnReluFn.apply(x, self.weight, self.bias, rm, rv, bn_training, float(factor), float(self.eps))


class _MaxPool2Fn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x):
        y, idx = _native.maxpool2_fwd(x)
        ctx.save_for_backward(idx)
        ctx.x_shape = tuple(x.shape)
        ctx.mark_non_differentiable(idx)
        return y

    @staticmethod
    def backward(ctx, dy):
        (idx,) = ctx.saved_tensors
        dy = dy.contiguous()
        if dy.data_ptr() % 16:
            dy = dy.clone()
        return _native.maxpool2_bwd(dy, idx, ctx.x_shape)


class _MaxPool2SkipFn(torch.autograd.Function):
    """(MaxPool3d(2)(x), x): a tensor that feeds both the pooling and a skip
    connection.  The backward receives both gradients and writes their sum in
    the pooling backward's one pass (r3c_maxpool2_bwd_add) instead of autograd
    adding them in a pass of its own; the sum is the same (fp32 add, one
    rounding)."""

    @staticmethod
    def forward(ctx, x):
        y, idx = _native.maxpool2_fwd(x)
        ctx.save_for_backward(idx)
        ctx.x_shape = tuple(x.shape)
        return y, x.view_as(x)

    @staticmethod
    def backward(ctx, dy, dskip):
        (idx,) = ctx.saved_tensors
        if dy is None:
            return dskip
        dy = dy.contiguous()
        if dy.data_ptr() % 16:
            dy = dy.clone()
        add = None
        if dskip is not None and dskip.dtype == dy.dtype and dskip.shape == ctx.x_shape and _native.pool_ok(dskip):
            add = dskip
        dx = _native.maxpool2_bwd(dy, idx, ctx.x_shape, add=add)
        if dskip is not None and add is None:
            dx = dx + dskip
        return dx


def _pair3(v):
    return (v, v, v) if isinstance(v, int) else tuple(v)


class MaxPool3dWmma(nn.MaxPool3d):
    """nn.MaxPool3d; kernel 2, stride 2 (no padding, dilation, ceil_mode or
    return_indices) runs the library's MaxPool3d kernels on CUDA NCDHW tensors
    with even d, h and w a multiple of 8: PyTorch's maximum (first in window
    order, NaN propagating), a one-byte window index kept for the backward
    instead of a 64-bit one.  Anything else is nn.MaxPool3d."""

    def _native_ok(self, x) -> bool:
        stride = self.stride if self.stride is not None else self.kernel_size
        return (_pair3(self.kernel_size) == (2, 2, 2) and _pair3(stride) == (2, 2, 2)
                and _pair3(self.padding) == (0, 0, 0) and _pair3(self.dilation) == (1, 1, 1)
                and not self.ceil_mode and not self.return_indices and x.is_cuda and _wmma_hw()
                and x.numel() > 0 and _native.pool_ok(x))

    def forward(self, x):
        if not self._native_ok(x):
            return super().forward(x)
        _ensure_native(x.device)
        with torch.cuda.device(x.device):
            return _MaxPool2Fn.apply(x)

    def forward_with_skip(self, x):
        """(self(x), x) for a tensor that also feeds a skip connection (the
        UNet3D encoder output): natively, the gradient arriving through the skip
        is added in the pooling backward's pass.  Elsewhere (x, self(x))."""
        if not self._native_ok(x):
            return super().forward(x), x
        _ensure_native(x.device)
        with torch.cuda.device(x.device):
            return _MaxPool2SkipFn.apply(x)
