"""Conv3d with stride > 1 on the native kernels (r3c_conv3d_strided_*) against
float64 PyTorch on the CPU from the same rounded inputs.

The reference routes strided convolutions to F.conv3d (its _geom_ok admits
stride 1 only, src/rdna4_conv3d/conv3d_wmma.py:89-95); the native strided path
is the opt-in widening (rdna4_conv3d.strided).  Tolerances are the north
star's: max|out - ref| / max|ref| <= 1e-2 for forward and dX, <= 3e-2 for dW
and db.  The library's timing hook must record the strided kernels, so a stock
fallback cannot pass.

The cases reach every kernel path: the gathering kernel (ragged channels,
stride 3, k=1, more than two column blocks), the LDS row-segment forward on
NDHWC sources and on NCDHW sources read in place (8-32 channels), the
row-segment dX (dY up to 64 channels), the direct dW on NCDHW operands and on
NCDHW copies of NDHWC ones, and the dY-scatter dW for the rest; the full-size
cases add two position blocks per wave.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from _util import gen, kaiming_weight, max_rel, to_layout

pytestmark = pytest.mark.gpu

TOL_FWD = 1e-2
TOL_DX = 1e-2
TOL_DW = 3e-2


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")


def _ref(x, w, b, stride, pad, go):
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = w.detach().double().cpu().requires_grad_(True)
    bd = b.detach().double().cpu().requires_grad_(True)
    y = F.conv3d(xd, wd, bd, stride, pad)
    y.backward(go.detach().double().cpu())
    return y.detach(), xd.grad, wd.grad, bd.grad


CASES = [
    # (n, cin, cout, d, h, w, k, pad, stride)
    (2, 24, 48, 8, 16, 16, 3, (1, 1, 1), (2, 2, 2)),     # the UNet-style downsampling conv
    (1, 5, 7, 7, 9, 11, 3, (1, 1, 1), (2, 2, 2)),        # ragged channels, odd extents
    (1, 16, 40, 6, 7, 13, 3, (0, 1, 2), (1, 2, 3)),      # mixed strides and paddings
    (2, 20, 3, 5, 6, 9, 1, (0, 0, 1), (2, 1, 2)),        # k = 1
    (1, 8, 130, 4, 5, 12, 3, (1, 1, 1), (2, 2, 2)),      # two column tiles (5 blocks of 32)
    (1, 32, 16, 9, 10, 70, 3, (2, 2, 2), (3, 3, 3)),     # stride 3, w blocks of 32 per residue class
    # direct dW kernel in NCDHW (w stride 1 or 2, w pad 1, W % 8 == 0, OW % 16 == 0)
    (2, 24, 48, 8, 32, 32, 3, (1, 1, 1), (2, 2, 2)),     # the downsampling conv, one 16-wide w block
    (1, 40, 70, 5, 7, 64, 3, (0, 1, 1), (1, 2, 2)),      # ragged channel blocks, d stride 1 pad 0
    (1, 8, 16, 4, 6, 48, 3, (1, 1, 1), (2, 1, 1)),       # w stride 1: three w blocks per row
    (2, 16, 32, 16, 32, 64, 3, (1, 1, 1), (2, 2, 2)),    # many K blocks per split
    # dX through LDS dY row segments with two column blocks (Cin 33-64)
    (1, 40, 32, 6, 10, 32, 3, (1, 1, 1), (2, 2, 2)),
    (1, 48, 24, 5, 6, 16, 3, (1, 1, 1), (1, 1, 1)),      # stride 1 through the strided entry points
    (1, 32, 40, 6, 8, 64, 3, (1, 1, 1), (2, 2, 2)),      # forward row segments on 4 channel groups
]


def _direct_dw(case, layout):
    """Which path the strided dW takes: "direct" (the direct kernel on the
    NCDHW operands), "copies" (NDHWC operands copied to NCDHW, then the direct
    kernel) or "scatter" (dY scattered onto the stride-1 grid)."""
    n, cin, cout, d, h, w, k, pad, stride = case
    od, oh, ow = ((s + 2 * p - k) // st + 1 for s, p, st in zip((d, h, w), pad, stride))
    if not (k == 3 and stride[2] in (1, 2) and pad[2] == 1 and w % 8 == 0 and ow % 16 == 0):
        return "scatter"
    if layout == "ncdhw":
        return "direct"
    ok = cin % 8 == 0 and cout % 8 == 0 and (d * h * w) % 8 == 0 and (od * oh * ow) % 8 == 0
    return "copies" if ok else "scatter"


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}s{}".format(
    *c[:7], "".join(map(str, c[7])), "".join(map(str, c[8]))))
def test_strided_native_parity(case, layout, dtype):
    from rdna4_conv3d import _native
    n, cin, cout, d, h, w, k, pad, stride = case
    print(f"case strided {case} {layout} {dtype}", flush=True)
    x = gen((n, cin, d, h, w), 0, dtype)
    wt = kaiming_weight((cout, cin, k, k, k), cin * k ** 3, 1, dtype)
    b = gen((cout,), 4, dtype)
    y_shape = _native.strided_out_shape(x.shape, wt.shape, stride, pad)
    go = gen(y_shape, 2, dtype)
    y_ref, dx_ref, dw_ref, db_ref = _ref(x, wt, b, stride, pad, go)
    xg = to_layout(x.cuda(), layout)
    gog = to_layout(go.cuda(), layout)
    wg, bg = wt.cuda(), b.cuda()
    _native.timing_enable(True)
    _native.timing_collect()
    y = _native.conv3d_strided_fwd(xg, wg, bg, stride, pad)
    dx = _native.conv3d_strided_dx(gog, wg, xg.shape, stride, pad, like=xg)
    torch.cuda.synchronize()
    kinds = [kd for _, kd, _ in _native.timing_collect()]
    dw, db = _native.conv3d_strided_dw(xg, gog, wg.shape, stride, pad, torch.float32, want_db=True,
                                       db_dtype=torch.float32)
    torch.cuda.synchronize()
    dw_kinds = [kd for _, kd, _ in _native.timing_collect()]
    _native.timing_enable(False)
    assert kinds.count("row") >= 2, kinds
    path = _direct_dw(case, layout)
    if path == "direct":
        assert dw_kinds == ["wgrad", "reduce"], dw_kinds
    elif path == "copies":
        assert dw_kinds == ["layout", "layout", "wgrad", "reduce"], dw_kinds
    else:
        assert "layout" in dw_kinds and "reduce" in dw_kinds, dw_kinds
    assert tuple(y.shape) == tuple(y_ref.shape) and dx.shape == dx_ref.shape and dw.shape == dw_ref.shape
    e = [max_rel(y, y_ref), max_rel(dx, dx_ref), max_rel(dw, dw_ref), max_rel(db, db_ref)]
    print("  maxrel y {:.2e} dx {:.2e} dw {:.2e} db {:.2e}".format(*e), flush=True)
    assert e[0] <= TOL_FWD and e[1] <= TOL_DX and e[2] <= TOL_DW and e[3] <= TOL_DW


@requires_gfx950
def test_strided_module_matches_nn_conv3d_under_autocast():
    """StridedConv3dWmma in a bf16 autocast step: output dtype bf16 (autocast
    contract), gradients of the fp32 master parameters in fp32, every result
    within tolerance of nn.Conv3d in fp32 on the same rounded values."""
    from rdna4_conv3d import _native
    from rdna4_conv3d.strided import StridedConv3dWmma
    torch.manual_seed(1)
    ref = nn.Conv3d(24, 48, 3, stride=2, padding=1).cuda()
    mod = StridedConv3dWmma(24, 48, 3, stride=2, padding=1).cuda()
    mod.load_state_dict(ref.state_dict())
    x = gen((2, 24, 16, 32, 32), 0, torch.float32).cuda()
    go = gen((2, 48, 8, 16, 16), 2, torch.bfloat16).cuda()
    xm = x.clone().requires_grad_(True)
    _native.timing_enable(True)
    _native.timing_collect()
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = mod(xm)
    assert y.dtype == torch.bfloat16
    y.backward(go)
    torch.cuda.synchronize()
    kinds = [kd for _, kd, _ in _native.timing_collect()]
    _native.timing_enable(False)
    assert "row" in kinds and "reduce" in kinds, kinds
    assert mod.weight.grad.dtype == torch.float32 and mod.bias.grad.dtype == torch.float32
    xr = x.to(torch.bfloat16).float().requires_grad_(True)
    wr = ref.weight.detach().to(torch.bfloat16).float().requires_grad_(True)
    br = ref.bias.detach().to(torch.bfloat16).float().requires_grad_(True)
    yr = F.conv3d(xr, wr, br, 2, 1)
    yr.backward(go.float())
    assert max_rel(y.float(), yr) <= TOL_FWD
    assert max_rel(xm.grad, xr.grad) <= TOL_DX
    assert max_rel(mod.weight.grad, wr.grad) <= TOL_DW
    assert max_rel(mod.bias.grad, br.grad) <= TOL_DW


@requires_gfx950
def test_strided_module_falls_back_where_not_native():
    """Dilation 2, groups 2 or a 5x5x5 kernel run nn.Conv3d.forward unchanged."""
    from rdna4_conv3d.strided import StridedConv3dWmma, strided_native_ok
    x = gen((1, 8, 9, 9, 9), 0, torch.float16).cuda()
    for kw in ({"dilation": 2}, {"groups": 2}, {"kernel_size": 5}):
        args = {"kernel_size": 3, "stride": 2, "padding": 1}
        args.update(kw)
        ks = args.pop("kernel_size")
        mod = StridedConv3dWmma(8, 8, ks, **args).cuda().half()
        assert not strided_native_ok(x, mod.weight, mod.stride, mod.padding, mod.dilation, mod.groups)
        torch.testing.assert_close(mod(x), nn.Conv3d.forward(mod, x), atol=0, rtol=0)


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("shape", [(4, 24, 48, 64, 128, 128), (2, 16, 32, 32, 64, 128)],
                         ids=["bench", "half"])
def test_strided_native_large_vs_fp32(shape, layout, dtype):
    """Full-size strided passes (the bench's k=3 stride 2 shape, where the
    planner gives each wave two blocks of 32 positions, and a half-size one,
    where dX does) against PyTorch's fp32 convolution of the same rounded
    values on the GPU; tolerances as above."""
    from rdna4_conv3d import _native
    n, cin, cout, d, h, w = shape
    stride, pad = (2, 2, 2), (1, 1, 1)
    print(f"case strided large {shape} {layout} {dtype}", flush=True)
    x = to_layout(gen((n, cin, d, h, w), 0, dtype).cuda(), layout)
    wt = kaiming_weight((cout, cin, 3, 3, 3), cin * 27, 1, dtype).cuda()
    b = gen((cout,), 4, dtype).cuda()
    y_shape = _native.strided_out_shape(x.shape, wt.shape, stride, pad)
    go = to_layout(gen(y_shape, 2, dtype).cuda(), layout)
    y = _native.conv3d_strided_fwd(x, wt, b, stride, pad)
    dx = _native.conv3d_strided_dx(go, wt, x.shape, stride, pad, like=x)
    dw, db = _native.conv3d_strided_dw(x, go, wt.shape, stride, pad, torch.float32, want_db=True,
                                       db_dtype=torch.float32)
    xr = x.detach().float().requires_grad_(True)
    wr = wt.detach().float().requires_grad_(True)
    br = b.detach().float().requires_grad_(True)
    yr = F.conv3d(xr, wr, br, stride, pad)
    yr.backward(go.float())
    torch.cuda.synchronize()
    e = [max_rel(y, yr), max_rel(dx, xr.grad), max_rel(dw, wr.grad), max_rel(db, br.grad)]
    print("  maxrel y {:.2e} dx {:.2e} dw {:.2e} db {:.2e}".format(*e), flush=True)
    assert e[0] <= TOL_FWD and e[1] <= TOL_DX and e[2] <= TOL_DW and e[3] <= TOL_DW
