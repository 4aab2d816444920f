"""MaxPool3dWmma (native MaxPool3d(2)) against nn.MaxPool3d(2) on the CPU.

The module replaces nn.MaxPool3d(2) of the reference's UNet3D down path
(benches/unet_e2e.py:27-37).  Taking a maximum and routing a gradient involve
no arithmetic, so the bar is bit-exact: from the same (rounded) input and
output gradient, the native output and dX must equal the CPU nn.MaxPool3d's in
the same dtype, ties and NaNs included (the CPU kernel's rule: the first
maximum in window order wins, NaN propagates, an all -inf window routes its
gradient to its first element).  The library's launch hook must record the
pool kernels, so a stock fallback cannot pass.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from _util import gen

pytestmark = pytest.mark.gpu


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")


def _cpu_ref(x, go):
    xr = x.detach().cpu().clone().requires_grad_(True)
    y = nn.MaxPool3d(2)(xr)
    y.backward(go.cpu())
    return y.detach(), xr.grad


def _run(x, go, expect_native=True):
    from rdna4_conv3d import _native
    from rdna4_conv3d.fused import MaxPool3dWmma
    xg = x.cuda().requires_grad_(True)
    _native.timing_filter(-1, None)
    _native.timing_enable(True)
    _native.timing_collect()
    y = MaxPool3dWmma(2)(xg)
    y.backward(go.cuda())
    torch.cuda.synchronize()
    kinds = {k for _, k, _ in _native.timing_collect()}
    _native.timing_enable(False)
    if expect_native:
        assert "pool" in kinds, kinds
    return y.detach().cpu(), xg.grad.cpu()


def _assert_same(a, b):
    assert a.dtype == b.dtype and a.shape == b.shape
    assert torch.equal(a.isnan(), b.isnan())
    m = ~a.isnan()
    assert torch.equal(a[m], b[m]), float((a[m].double() - b[m].double()).abs().max())


CASES = [
    # (n, c, d, h, w)
    (1, 1, 2, 2, 8),
    (2, 24, 8, 16, 16),
    (3, 5, 6, 10, 24),
    (4, 24, 64, 128, 128),   # the UNet3D config-5 first pooling
]


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}c{}_{}x{}x{}".format(*c))
def test_maxpool_bitwise_equals_cpu(case, dtype):
    print(f"case MaxPool3dWmma {case} {dtype}", flush=True)
    x = gen(case, 0).to(dtype)
    go = gen(tuple(case[:2]) + tuple(v // 2 for v in case[2:]), 1).to(dtype)
    y_r, dx_r = _cpu_ref(x, go)
    y, dx = _run(x, go)
    _assert_same(y, y_r)
    _assert_same(dx, dx_r)


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_maxpool_ties_nans_and_infinities(dtype):
    """Small integers (many ties in a window), NaNs, +-inf and whole -inf windows."""
    print(f"case MaxPool3dWmma special values {dtype}", flush=True)
    g = torch.Generator().manual_seed(5)
    x = torch.randint(-2, 3, (2, 3, 4, 6, 16), generator=g).float()
    flat = x.view(-1)
    pick = torch.randperm(flat.numel(), generator=g)
    flat[pick[:20]] = float("nan")
    flat[pick[20:40]] = float("inf")
    flat[pick[40:60]] = float("-inf")
    x[0, 0, 0:2, 0:2, 0:2] = float("-inf")        # one window of -inf only
    x[1, 2, 2:4, 4:6, 14:16] = float("nan")       # one window of NaN only
    x = x.to(dtype)
    go = gen((2, 3, 2, 3, 8), 2).to(dtype)
    y_r, dx_r = _cpu_ref(x, go)
    y, dx = _run(x, go)
    _assert_same(y, y_r)
    _assert_same(dx, dx_r)


@requires_gfx950
def test_maxpool_strided_channel_slice():
    """A channel slice of a wider tensor (dense planes, channel stride of the
    parent) runs natively without a copy; the result equals the CPU's."""
    base = gen((2, 16, 4, 8, 16), 3).to(torch.bfloat16)
    x = base[:, 4:12]
    assert not x.is_contiguous()
    go = gen((2, 8, 2, 4, 8), 4).to(torch.bfloat16)
    from rdna4_conv3d import _native
    from rdna4_conv3d.fused import MaxPool3dWmma
    xg = base.cuda()[:, 4:12].detach().requires_grad_(True)
    assert _native.pool_ok(xg)
    _native.timing_enable(True)
    _native.timing_collect()
    y = MaxPool3dWmma(2)(xg)
    y.backward(go.cuda())
    torch.cuda.synchronize()
    kinds = {k for _, k, _ in _native.timing_collect()}
    _native.timing_enable(False)
    assert "pool" in kinds
    y_r, dx_r = _cpu_ref(x.contiguous(), go)
    _assert_same(y.detach().cpu(), y_r)
    _assert_same(xg.grad.cpu(), dx_r)


@requires_gfx950
def test_maxpool_unsupported_shapes_fall_back_to_stock():
    """w not a multiple of 8, or odd d / h, or channels_last_3d: nn.MaxPool3d runs."""
    from rdna4_conv3d.fused import MaxPool3dWmma
    for shape, cl in [((1, 2, 4, 4, 12), False), ((1, 2, 5, 4, 8), False), ((1, 8, 4, 4, 8), True)]:
        x = gen(shape, 6).cuda()
        if cl:
            x = x.contiguous(memory_format=torch.channels_last_3d)
        mod = MaxPool3dWmma(2)
        assert not mod._native_ok(x)
        torch.testing.assert_close(mod(x), nn.MaxPool3d(2)(x), atol=0, rtol=0)


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
def test_maxpool_forward_with_skip_adds_the_skip_gradient(dtype):
    """forward_with_skip returns (pool(x), x); the backward writes
    pool_bwd(dy) + dskip in the pooling's pass (r3c_maxpool2_bwd_add), bitwise
    what autograd's add of the two gradients gives (fp32 add, one rounding)."""
    from rdna4_conv3d import _native
    from rdna4_conv3d.fused import MaxPool3dWmma
    case = (2, 24, 8, 16, 16)
    print(f"case MaxPool3dWmma.forward_with_skip {case} {dtype}", flush=True)
    x = gen(case, 0).to(dtype)
    go = gen((2, 24, 4, 8, 8), 1).to(dtype)
    gs = gen(case, 2).to(dtype)
    y_r, dx_r = _cpu_ref(x, go)
    want = (dx_r.float() + gs.float()).to(dtype)
    xg = x.cuda().requires_grad_(True)
    _native.timing_enable(True)
    _native.timing_collect()
    y, skip = MaxPool3dWmma(2).forward_with_skip(xg)
    torch.autograd.backward([y, skip], [go.cuda(), gs.cuda()])
    torch.cuda.synchronize()
    kinds = [k for _, k, _ in _native.timing_collect()]
    _native.timing_enable(False)
    assert kinds.count("pool") == 2, kinds  # forward, and one backward pass for both gradients
    _assert_same(y.detach().cpu(), y_r)
    assert torch.equal(skip.detach().cpu(), x)
    _assert_same(xg.grad.cpu(), want)
    # only one of the two outputs used: the other gradient is absent
    for use_pool in (True, False):
        xo = x.cuda().requires_grad_(True)
        y2, s2 = MaxPool3dWmma(2).forward_with_skip(xo)
        (y2 if use_pool else s2).backward(go.cuda() if use_pool else gs.cuda())
        _assert_same(xo.grad.cpu(), dx_r if use_pool else gs)
