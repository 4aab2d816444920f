"""Parity at the full sizes bench.py times (3 and 4).

Every pass the bench measures -- fwd, dX and dW (+ the fused db) of the four
UNet3D trunk k=3 layers (bf16), of the two pointwise k=1 layers (fp16,
post-ReLU inputs with about half zeros) and of the two ConvTranspose3d k2s2
layers (bf16) -- is run at its full shape through the same library calls the
bench makes, and compared with PyTorch's fp32 convolution on the GPU computed
from the same rounded inputs (F.conv3d, torch.nn.grad.conv3d_input /
conv3d_weight, F.conv_transpose3d + autograd; the float64 CPU path would take
minutes here).  At these sizes this pins the plans the small-shape tests never
reach: the 256-split dW reduce and the staged NCDHW halo of the
24-channel layer, the halved split counts of the 96 / 192-channel dW, the
row kernel's split K at 192 channels, the register-direct k=1 and
ConvTranspose dW and ConvTranspose dX.  Tolerances (north star):
max|out - ref| / max|ref| <= 1e-2 for fwd and dX, <= 3e-2 for dW and db.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import bench
from _util import gen, kaiming_weight

pytestmark = pytest.mark.gpu

TOL_FWD = 1e-2
TOL_DX = 1e-2
TOL_DW = 3e-2


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")


def _rel(out, ref):
    """max|out - ref| / max|ref|, on the GPU."""
    out, ref = out.double(), ref.double()
    return float((out - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def _layout(t, layout):
    return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()


def _check(name, got, ref, tol):
    e = _rel(got, ref)
    print(f"  {name}: maxrel {e:.2e}", flush=True)
    assert e <= tol, f"{name}: {e:.3e} > {tol}"


@requires_gfx950
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("shape", bench.TRUNK, ids=lambda s: "k3_{1}to{2}_{3}x{4}x{5}".format(*s))
def test_trunk_k3_full_size(shape, layout):
    from rdna4_conv3d import _native as nat
    n, ci, co, d, h, w = shape
    print(f"case trunk k3 {shape} {layout} bf16", flush=True)
    dt = torch.bfloat16
    x = _layout(gen((n, ci, d, h, w), 0, dt).cuda(), layout)
    go = _layout(gen((n, co, d, h, w), 2, dt).cuda(), layout)
    wt = kaiming_weight((co, ci, 3, 3, 3), ci * 27, 1, dt).cuda()
    b = kaiming_weight((co,), ci * 27, 3, dt).cuda()
    y = nat.conv3d_fwd(x, wt, b, (1, 1, 1))
    dx = nat.conv3d_dx(go, wt, x.shape, (1, 1, 1), like=x)
    dw, db = nat.conv3d_dw(x, go, wt.shape, (1, 1, 1), torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    xf, gof, wf = x.float(), go.float(), wt.float()
    _check("y", y, F.conv3d(xf, wf, b.float(), 1, 1), TOL_FWD)
    del y
    _check("dx", dx, torch.nn.grad.conv3d_input(x.shape, wf, gof, 1, 1), TOL_DX)
    del dx
    _check("dw", dw, torch.nn.grad.conv3d_weight(xf, wt.shape, gof, 1, 1), TOL_DW)
    _check("db", db, gof.sum((0, 2, 3, 4)), TOL_DW)


@requires_gfx950
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("shape", bench.POINTWISE, ids=lambda s: "k1_{1}to{2}_{3}x{4}x{5}".format(*s))
def test_pointwise_k1_full_size(shape, layout):
    """fp16, x = relu(N(0,1)) (about half zeros)."""
    from rdna4_conv3d import _native as nat
    n, ci, co, d, h, w = shape
    print(f"case pointwise k1 {shape} {layout} fp16 relu inputs", flush=True)
    dt = torch.float16
    x = _layout(gen((n, ci, d, h, w), 0, dt, relu=True).cuda(), layout)
    frac0 = float((x == 0).float().mean())
    assert 0.45 < frac0 < 0.55
    go = _layout(gen((n, co, d, h, w), 2, dt).cuda(), layout)
    wt = kaiming_weight((co, ci, 1, 1, 1), ci, 1, dt).cuda()
    y = nat.conv3d_fwd(x, wt, None, (0, 0, 0))
    dx = nat.conv3d_dx(go, wt, x.shape, (0, 0, 0), like=x)
    dw, db = nat.conv3d_dw(x, go, wt.shape, (0, 0, 0), torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    xf, gof, wf = x.float(), go.float(), wt.float()
    _check("y", y, F.conv3d(xf, wf, None), TOL_FWD)
    del y
    _check("dx", dx, torch.nn.grad.conv3d_input(x.shape, wf, gof), TOL_DX)
    del dx
    _check("dw", dw, torch.nn.grad.conv3d_weight(xf, wt.shape, gof), TOL_DW)
    _check("db", db, gof.sum((0, 2, 3, 4)), TOL_DW)


@requires_gfx950
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("shape", bench.CONVT, ids=lambda s: "t2_{1}to{2}_{3}x{4}x{5}".format(*s))
def test_convt_full_size(shape, layout):
    """ConvTranspose3d k=2 s=2, bf16."""
    from rdna4_conv3d import _native as nat
    n, ci, co, d, h, w = shape
    print(f"case convt k2s2 {shape} {layout} bf16", flush=True)
    dt = torch.bfloat16
    x = _layout(gen((n, ci, d, h, w), 0, dt).cuda(), layout)
    go = _layout(gen((n, co, 2 * d, 2 * h, 2 * w), 2, dt).cuda(), layout)
    wt = kaiming_weight((ci, co, 2, 2, 2), co * 8, 1, dt).cuda()
    b = kaiming_weight((co,), co * 8, 3, dt).cuda()
    y = nat.convt_fwd(x, wt, b)
    dx = nat.convt_dx(go, wt, x.shape, like=x)
    dw, db = nat.convt_dw(x, go, wt.shape, torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    xf = x.float().requires_grad_(True)
    wf = wt.float().requires_grad_(True)
    yr = F.conv_transpose3d(xf, wf, b.float(), stride=2)
    dx_ref, dw_ref = torch.autograd.grad(yr, (xf, wf), go.float())
    _check("y", y, yr.detach(), TOL_FWD)
    _check("dx", dx, dx_ref, TOL_DX)
    _check("dw", dw, dw_ref, TOL_DW)
    _check("db", db, go.float().sum((0, 2, 3, 4)), TOL_DW)
