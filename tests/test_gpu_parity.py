"""GPU parity of the native HIP kernels against the fp32/fp64 reference path.

Inputs are generated on the CPU with fixed seeds, rounded to bf16/fp16, and the
reference is computed in float64 from the same rounded values (F.conv3d /
conv_transpose3d / autograd on the CPU, the reference package's own oracle), and
at the smallest shapes also by the C oracle.  Tolerances (north star):
max|out - ref| / max|ref| <= 1e-2 for fwd and dX, <= 3e-2 for dW.
"""
from __future__ import annotations

import pytest
import torch
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


def _native():
    from rdna4_conv3d import _native
    _native.load()
    return _native


def _ref_conv(x, w, b, pad, go):
    """float64 CPU reference: y, dx, dw, db from the same rounded inputs."""
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = w.detach().double().cpu().requires_grad_(True)
    bd = None if b is None else b.detach().double().cpu().requires_grad_(True)
    y = F.conv3d(xd, wd, bd, 1, pad)
    y.backward(go.detach().double().cpu())
    return y.detach(), xd.grad, wd.grad, (None if bd is None else bd.grad)


CONV_CASES = [
    # (n, cin, cout, d, h, w, k, pad)  -- the reference's test_conv3d.py:51-54 shapes first
    (2, 5, 7, 9, 11, 13, 3, 1),
    (2, 24, 1, 8, 16, 16, 1, 0),
    # k=1 with at most 4 output channels on NCDHW: the streaming skinny kernels
    # (the UNet3D head 24 -> 2; channel counts off the 8-channel blocks)
    (2, 24, 2, 8, 16, 16, 1, 0),
    (1, 40, 4, 4, 8, 24, 1, 0),
    (3, 20, 3, 5, 6, 8, 1, 0),
    (1, 24, 24, 8, 16, 16, 3, 1),
    (1, 1, 24, 8, 16, 16, 3, 1),
    (1, 8, 16, 6, 7, 9, 3, 0),
    (1, 8, 16, 6, 7, 9, 3, 2),
    (1, 16, 8, 5, 6, 7, 1, 1),
    (1, 48, 48, 8, 8, 16, 3, 1),
    (1, 40, 96, 4, 8, 16, 3, 1),
    (1, 96, 40, 4, 8, 20, 3, 1),
    (2, 48, 24, 4, 9, 33, 1, 0),
    (2, 40, 24, 5, 9, 24, 1, 0),     # k=1 unpadded, w % 8 == 0: both dW operands channel-major in NCDHW
    (1, 48, 56, 3, 6, 32, 1, 0),
    (1, 40, 72, 4, 8, 24, 1, 0),     # D*H*W % 256 == 0: flat position order in the k=1 passes
    (2, 24, 24, 16, 64, 64, 3, 1),   # more tiles than CUs: multi-job workgroups, no split K
    (2, 20, 24, 18, 70, 40, 3, 1),   # the same with ragged channels and box edges
    (2, 1, 24, 16, 64, 64, 3, 1),    # one source channel (the first UNet layer)
    # One source channel: the dedicated kernels (r3c_stem.hip).  Forward with
    # pad 0 (a partial 32-position tile) and pad 2 with two output-channel
    # blocks (dW on the general kernels: OW % 16 != 0); dW with two channel
    # blocks and a partial row block; more dW jobs than workgroups.
    (1, 1, 16, 6, 9, 24, 3, 0),
    (1, 1, 40, 5, 7, 16, 3, 2),
    (1, 1, 40, 6, 10, 32, 3, 1),
    (4, 1, 32, 40, 42, 128, 3, 1),
    # NCDHW rows of 128 / 64 positions with enough boxes: full-width tap boxes
    # (whole rows, 2 x 4 per box) with ragged d and h edges, and the
    # row-walking dW over columns of odd length
    (4, 8, 8, 13, 62, 128, 3, 1),
    (4, 8, 16, 15, 30, 64, 3, 1),
    # k=1 unpadded with D*H*W % 64 == 0 (NCDHW: register-direct dW when Cout > 32):
    # 2 x 1 tile groups over two column groups, a 3 x 1 tile group
    (2, 96, 40, 4, 4, 32, 1, 0),
    (2, 24, 96, 2, 8, 32, 1, 0),
]


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", CONV_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}".format(*c))
def test_conv3d_native_parity(case, layout, dtype):
    nat = _native()
    n, cin, cout, d, h, w, k, pad = case
    print(f"case conv {case} {layout} {dtype}", flush=True)
    x = gen((n, cin, d, h, w), 0, dtype)
    wt = kaiming_weight((cout, cin, k, k, k), cin * k ** 3, 1, dtype)
    b = gen((cout,), 4, dtype)
    od, oh, ow = d + 2 * pad - k + 1, h + 2 * pad - k + 1, w + 2 * pad - k + 1
    go = gen((n, cout, od, oh, ow), 2, dtype)
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(x, wt, b, pad, go)

    xg = to_layout(x.cuda(), layout)
    gog = to_layout(go.cuda(), layout)
    wg, bg = wt.cuda(), b.cuda()
    y = nat.conv3d_fwd(xg, wg, bg, (pad, pad, pad))
    dx = nat.conv3d_dx(gog, wg, xg.shape, (pad, pad, pad), like=xg)
    dw, db = nat.conv3d_dw(xg, gog, wg.shape, (pad, pad, pad), torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    assert y.shape == y_ref.shape and dx.shape == dx_ref.shape and dw.shape == dw_ref.shape
    if layout == "ndhwc" and not xg.is_contiguous():
        # outputs follow the input layout; a tensor that is both NCDHW- and
        # NDHWC-contiguous (C == 1) counts as NCDHW, as in torch
        assert y.is_contiguous(memory_format=torch.channels_last_3d)
        assert dx.is_contiguous(memory_format=torch.channels_last_3d)
    e_y, e_dx, e_dw, e_db = max_rel(y, y_ref), max_rel(dx, dx_ref), max_rel(dw, dw_ref), max_rel(db, db_ref)
    print(f"  maxrel y {e_y:.2e} dx {e_dx:.2e} dw {e_dw:.2e} db {e_db:.2e}", flush=True)
    assert e_y <= TOL_FWD
    assert e_dx <= TOL_DX
    assert e_dw <= TOL_DW
    assert e_db <= TOL_DW


CONVT_CASES = [
    # (n, cin, cout, d, h, w)
    (1, 16, 8, 3, 4, 5),
    (2, 24, 48, 2, 3, 17),
    (1, 48, 24, 4, 8, 16),
    (1, 192, 96, 2, 4, 16),
    (1, 5, 3, 2, 2, 3),
    (2, 40, 24, 3, 5, 40),   # w % 8 == 0 with a ragged second line and a ragged channel chunk (NCDHW: channel-major staging)
    # NCDHW register-direct dW (w % 16 == 0): 32-position K blocks (w % 32 == 0)
    # over four column tile groups; a 3 x 1 tile group (Cout * 8 <= 32)
    (1, 24, 40, 2, 3, 64),
    (1, 70, 4, 2, 2, 32),
]


def _ref_convt(x, w, b, go):
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = w.detach().double().cpu().requires_grad_(True)
    bd = None if b is None else b.detach().double().cpu().requires_grad_(True)
    y = F.conv_transpose3d(xd, wd, bd, stride=2)
    y.backward(go.detach().double().cpu())
    return y.detach(), xd.grad, wd.grad, (None if bd is None else bd.grad)


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", CONVT_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}".format(*c))
def test_convt_native_parity(case, layout, dtype):
    nat = _native()
    n, cin, cout, d, h, w = case
    print(f"case convt {case} {layout} {dtype}", flush=True)
    x = gen((n, cin, d, h, w), 0, dtype)
    wt = kaiming_weight((cin, cout, 2, 2, 2), cout * 8, 1, dtype)
    b = gen((cout,), 4, dtype)
    go = gen((n, cout, 2 * d, 2 * h, 2 * w), 2, dtype)
    y_ref, dx_ref, dw_ref, db_ref = _ref_convt(x, wt, b, go)
    xg = to_layout(x.cuda(), layout)
    gog = to_layout(go.cuda(), layout)
    wg, bg = wt.cuda(), b.cuda()
    y = nat.convt_fwd(xg, wg, bg)
    dx = nat.convt_dx(gog, wg, xg.shape, like=xg)
    dw, db = nat.convt_dw(xg, gog, wg.shape, torch.float32, want_db=True, db_dtype=torch.float32)
    torch.cuda.synchronize()
    e_y, e_dx, e_dw, e_db = max_rel(y, y_ref), max_rel(dx, dx_ref), max_rel(dw, dw_ref), max_rel(db, db_ref)
    print(f"  maxrel y {e_y:.2e} dx {e_dx:.2e} dw {e_dw:.2e} db {e_db:.2e}", flush=True)
    assert e_y <= TOL_FWD
    assert e_dx <= TOL_DX
    assert e_dw <= TOL_DW
    assert e_db <= TOL_DW


# Shapes that take the scheduling branches: split K in the row kernel (fewer
# output tiles than CUs), the NDHWC copy of a low-channel NCDHW operand, and a
# many-split weight-gradient reduce (the tree-shaped single launch).
DETERMINISM_CASES = [
    (1, 192, 192, 4, 8, 16, 3, 1),   # row kernel split K (fwd and dX)
    (2, 24, 24, 16, 32, 32, 3, 1),   # NCDHW copy path; dW with a many-split reduce
    (2, 24, 48, 8, 16, 32, 1, 0),    # k=1: register-direct dW (NCDHW) with a many-split reduce
    (4, 1, 24, 40, 42, 128, 3, 1),   # one source channel: dedicated kernels, 1024 dW partials
]


@requires_gfx950
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", DETERMINISM_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}".format(*c))
def test_native_bitwise_repeatable(case, layout):
    """Fixed split and fixed-order sums: two runs give identical bits, and the
    result matches the float64 reference (same tolerances as above)."""
    nat = _native()
    n, cin, cout, d, h, w, k, pad = case
    print(f"case determinism {case} {layout}", flush=True)
    dtype = torch.bfloat16
    x = gen((n, cin, d, h, w), 0, dtype)
    wt = kaiming_weight((cout, cin, k, k, k), cin * k ** 3, 1, dtype)
    b = gen((cout,), 4, dtype)
    go = gen((n, cout, d, h, w), 2, dtype)
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(x, wt, b, pad, go)
    xg = to_layout(x.cuda(), layout)
    gog = to_layout(go.cuda(), layout)
    wg, bg = wt.cuda(), b.cuda()
    runs = []
    for _ in range(2):
        y = nat.conv3d_fwd(xg, wg, bg, (pad, pad, pad))
        dx = nat.conv3d_dx(gog, wg, xg.shape, (pad, pad, pad), like=xg)
        dw, db = nat.conv3d_dw(xg, gog, wg.shape, (pad, pad, pad), torch.float32, want_db=True,
                               db_dtype=torch.float32)
        torch.cuda.synchronize()
        runs.append([t.detach().cpu() for t in (y, dx, dw, db)])
    for a_, b_ in zip(*runs):
        assert torch.equal(a_, b_)
    y, dx, dw, db = runs[0]
    assert max_rel(y, y_ref) <= TOL_FWD
    assert max_rel(dx, dx_ref) <= TOL_DX
    assert max_rel(dw, dw_ref) <= TOL_DW
    assert max_rel(db, db_ref) <= TOL_DW


# Shapes large enough to reach the k=3 kernel's biggest boxes (32 lines of 32
# per workgroup, resident or per-stage weights) and its 16-wide-line mode with
# split K; the reference is torch's own fp32 convolution on the GPU from the
# same rounded inputs (the float64 CPU path would take minutes here).
K3_LARGE_CASES = [
    # (n, cin, cout, d, h, w)
    (2, 24, 24, 16, 128, 64),    # one column block, 32-line boxes, all weights resident
    (1, 200, 16, 16, 128, 128),  # one column block, 32-line boxes, per-stage weights (25 chunks)
    (1, 48, 48, 16, 128, 64),    # two column blocks, 16-line boxes
    (1, 96, 96, 16, 64, 64),     # three column blocks, 8-line boxes
    (4, 192, 192, 8, 16, 16),    # 16-wide lines, two column tiles, split K
]


@requires_gfx950
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", K3_LARGE_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}".format(*c))
def test_conv3d_k3_large_fwd_dx(case, layout):
    nat = _native()
    n, cin, cout, d, h, w = case
    print(f"case k3 large {case} {layout}", flush=True)
    dtype = torch.bfloat16
    x = gen((n, cin, d, h, w), 0, dtype).cuda()
    wt = kaiming_weight((cout, cin, 3, 3, 3), cin * 27, 1, dtype).cuda()
    b = gen((cout,), 4, dtype).cuda()
    go = gen((n, cout, d, h, w), 2, dtype).cuda()
    y_ref = F.conv3d(x.float(), wt.float(), b.float(), 1, 1)
    dx_ref = torch.nn.grad.conv3d_input(x.shape, wt.float(), go.float(), 1, 1)
    xg, gog = to_layout(x, layout), to_layout(go, layout)
    y = nat.conv3d_fwd(xg, wt, b, (1, 1, 1))
    dx = nat.conv3d_dx(gog, wt, xg.shape, (1, 1, 1), like=xg)
    torch.cuda.synchronize()
    e_y, e_dx = max_rel(y, y_ref), max_rel(dx, dx_ref)
    print(f"  maxrel y {e_y:.2e} dx {e_dx:.2e}", flush=True)
    assert e_y <= TOL_FWD
    assert e_dx <= TOL_DX
