"""GPU parity through the public API (the reference's L1-L4 layers:
src/rdna4_conv3d/conv3d_wmma.py:1233-1409 and 1545-1595; its GPU tests
tests/test_conv3d.py:38-75).

Every case runs the package's entry point on cuda:0 -- Conv3dWmma,
conv3d_wmma (+ autograd), wmma_fwd / wmma_dw / wmma_dx, ConvTranspose3dWmma --
and compares it with a float64 CPU reference computed from the same values the
native kernels see (inputs rounded to the compute dtype first).  Tolerances
(north star): max|out - ref| / max|ref| <= 1e-2 for fwd and dX, <= 3e-2 for
dW and db.  The tests also assert the output layout and dtype contract
(output follows the input's memory format; under autocast the output is in
the autocast dtype and fp32 parameters get fp32 gradients) and that the native
library ran (its launch-timing hook records the kernels), so a silent fallback
cannot pass.  The stock-fallback cases (stride 2, groups, padding_mode,
dilation, output_size, a misaligned input) assert the result equals the stock
PyTorch module's.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from _util import gen, max_rel

pytestmark = pytest.mark.gpu

TOL_FWD = 1e-2
TOL_DX = 1e-2
TOL_DW = 3e-2


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")


class _NativeRan:
    """Context manager: records the library's kernel launches (timing hook)."""

    def __enter__(self):
        from rdna4_conv3d import _native
        self.nat = _native
        _native.load()
        _native.timing_filter(-1, None)
        _native.timing_enable(True)
        _native.timing_collect()
        return self

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self.kinds = {k for _, k, _ in self.nat.timing_collect()}
        self.nat.timing_enable(False)
        return False


def _ref_conv(x, w, b, pad, go, transpose=False):
    """float64 CPU reference (y, dx, dw, db) from the given (already rounded) values."""
    xd = x.detach().double().cpu().requires_grad_(True)
    wd = w.detach().double().cpu().requires_grad_(True)
    bd = None if b is None else b.detach().double().cpu().requires_grad_(True)
    y = F.conv_transpose3d(xd, wd, bd, stride=2) if transpose else F.conv3d(xd, wd, bd, 1, pad)
    y.backward(go.detach().double().cpu())
    return y.detach(), xd.grad, wd.grad, (None if bd is None else bd.grad)


def _layout(t, layout):
    return t.contiguous(memory_format=torch.channels_last_3d) if layout == "ndhwc" else t.contiguous()


def _assert_layout(t, layout):
    if layout == "ndhwc":
        assert t.is_contiguous(memory_format=torch.channels_last_3d)
    else:
        assert t.is_contiguous()


# ---------------------------------------------------------------------------
# Conv3dWmma module: dtype x layout x autocast
# ---------------------------------------------------------------------------
MODULE_CASES = [
    # (n, cin, cout, d, h, w, k, pad)
    (2, 8, 16, 6, 7, 9, 3, 1),
    (1, 24, 24, 8, 16, 16, 3, 1),
    (2, 16, 8, 5, 6, 32, 1, 0),
    (1, 8, 8, 4, 5, 6, 3, 0),
]


@requires_gfx950
@pytest.mark.parametrize("mode", ["fp32", "bf16", "fp16", "amp_bf16", "amp_fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", MODULE_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}".format(*c))
def test_conv3d_module(case, layout, mode):
    from rdna4_conv3d import Conv3dWmma
    n, cin, cout, d, h, w, k, pad = case
    print(f"case Conv3dWmma {case} {layout} {mode}", flush=True)
    param_dtype = {"fp32": torch.float32, "bf16": torch.bfloat16, "fp16": torch.float16}.get(mode, torch.float32)
    amp = {"amp_bf16": torch.bfloat16, "amp_fp16": torch.float16}.get(mode)
    # the dtype the kernels compute in: fp32 without autocast computes in fp16
    compute = amp or (param_dtype if param_dtype != torch.float32 else torch.float16)
    torch.manual_seed(1)
    conv = Conv3dWmma(cin, cout, k, padding=pad).cuda().to(param_dtype)
    x = gen((n, cin, d, h, w), 0, torch.float32)
    xg = _layout(x.to(param_dtype).cuda(), layout).requires_grad_(True)
    od, oh, ow = d + 2 * pad - k + 1, h + 2 * pad - k + 1, w + 2 * pad - k + 1
    go = gen((n, cout, od, oh, ow), 2, torch.float32).to(compute)
    with _NativeRan() as rec:
        with torch.autocast("cuda", dtype=amp or torch.bfloat16, enabled=amp is not None):
            y = conv(xg)
        y.backward(_layout(go.cuda(), layout).to(y.dtype))
    assert "row" in rec.kinds and "wgrad" in rec.kinds, rec.kinds
    # dtype / layout contract
    assert y.dtype == (amp or param_dtype)
    _assert_layout(y, layout)
    _assert_layout(xg.grad, layout)
    assert xg.grad.dtype == param_dtype
    assert conv.weight.grad.dtype == param_dtype and conv.bias.grad.dtype == param_dtype
    # reference from the values the kernels saw
    rx = xg.detach().to(compute)
    rw, rb = conv.weight.detach().to(compute), conv.bias.detach().to(compute)
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(rx, rw, rb, pad, go)
    e = (max_rel(y, y_ref), max_rel(xg.grad, dx_ref), max_rel(conv.weight.grad, dw_ref),
         max_rel(conv.bias.grad, db_ref))
    print(f"  maxrel y {e[0]:.2e} dx {e[1]:.2e} dw {e[2]:.2e} db {e[3]:.2e}", flush=True)
    assert e[0] <= TOL_FWD and e[1] <= TOL_DX and e[2] <= TOL_DW and e[3] <= TOL_DW


@requires_gfx950
def test_conv3d_module_fp32_params_get_fp32_grads_under_autocast():
    """AMP: fp32 master weights, bf16 compute; dW and db come back in fp32 and
    match the float64 gradient of the bf16-rounded problem."""
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(3)
    conv = Conv3dWmma(24, 48, 3, padding=1).cuda()
    x = gen((2, 24, 8, 16, 16), 0).cuda().requires_grad_(True)
    go = gen((2, 48, 8, 16, 16), 2).to(torch.bfloat16)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = conv(x)
    y.backward(go.cuda())
    assert y.dtype == torch.bfloat16
    assert conv.weight.grad.dtype == torch.float32 and conv.bias.grad.dtype == torch.float32
    assert x.grad.dtype == torch.float32
    _, dx_ref, dw_ref, db_ref = _ref_conv(x.detach().to(torch.bfloat16), conv.weight.detach().to(torch.bfloat16),
                                          conv.bias.detach().to(torch.bfloat16), 1, go)
    assert max_rel(x.grad, dx_ref) <= TOL_DX
    assert max_rel(conv.weight.grad, dw_ref) <= TOL_DW
    assert max_rel(conv.bias.grad, db_ref) <= TOL_DW


# ---------------------------------------------------------------------------
# conv3d_wmma functional + autograd (the reference's test_wmma_close_to_fp16_miopen
# shapes, tests/test_conv3d.py:47-75): against float64, and against MIOpen fp16
# with the reference's own tolerances.
# ---------------------------------------------------------------------------
REF_CASES = [
    (2, 5, 7, 9, 11, 13, 3, 1),
    (2, 24, 1, 8, 16, 16, 1, 0),
    (1, 24, 24, 8, 16, 16, 3, 1),
    (1, 1, 24, 8, 16, 16, 3, 1),
]


@requires_gfx950
@pytest.mark.parametrize("case", REF_CASES, ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}".format(*c))
def test_conv3d_wmma_functional_fp16(case):
    from rdna4_conv3d import conv3d_wmma
    n, cin, cout, d, h, w, k, pad = case
    print(f"case conv3d_wmma {case}", flush=True)
    x = gen((n, cin, d, h, w), 0, torch.float16).cuda().requires_grad_(True)
    wt = gen((cout, cin, k, k, k), 1, torch.float16).cuda().requires_grad_(True)
    b = gen((cout,), 4, torch.float16).cuda().requires_grad_(True)
    x2, w2, b2 = (t.detach().clone().requires_grad_(True) for t in (x, wt, b))
    with _NativeRan() as rec:
        y = conv3d_wmma(x, wt, b, 1, pad)
        go = gen(tuple(y.shape), 2, torch.float16).cuda()
        y.backward(go)
    assert "row" in rec.kinds and "wgrad" in rec.kinds, rec.kinds
    y2 = F.conv3d(x2, w2, b2, 1, pad)
    y2.backward(go)
    # the reference test's bounds against MIOpen fp16
    torch.testing.assert_close(y, y2, atol=2e-2, rtol=8e-2)
    torch.testing.assert_close(x.grad, x2.grad, atol=8e-2, rtol=8e-2)
    torch.testing.assert_close(wt.grad, w2.grad, atol=0.5, rtol=0.5)
    # and the north-star bounds against float64
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(x, wt, b, pad, go)
    assert max_rel(y, y_ref) <= TOL_FWD
    assert max_rel(x.grad, dx_ref) <= TOL_DX
    assert max_rel(wt.grad, dw_ref) <= TOL_DW
    assert max_rel(b.grad, db_ref) <= TOL_DW


# ---------------------------------------------------------------------------
# Isolated passes (conv3d_wmma.py:1368-1409, used by benches/isolated.py:57-58)
# ---------------------------------------------------------------------------
@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", [(2, 24, 24, 8, 16, 16, 3, 1), (1, 48, 24, 4, 8, 32, 1, 0),
                                  (1, 16, 8, 6, 7, 9, 3, 2)],
                         ids=lambda c: "n{}c{}-{}_{}x{}x{}_k{}p{}".format(*c))
def test_isolated_passes(case, layout, dtype):
    from rdna4_conv3d import wmma_dw, wmma_dx, wmma_fwd
    n, cin, cout, d, h, w, k, pad = case
    print(f"case wmma_* {case} {layout} {dtype}", flush=True)
    x = gen((n, cin, d, h, w), 0, dtype)
    wt = gen((cout, cin, k, k, k), 1, dtype) * 0.1
    wt = wt.to(dtype)
    b = gen((cout,), 4, dtype)
    od, oh, ow = d + 2 * pad - k + 1, h + 2 * pad - k + 1, w + 2 * pad - k + 1
    go = gen((n, cout, od, oh, ow), 2, dtype)
    y_ref, dx_ref, dw_ref, _ = _ref_conv(x, wt, b, pad, go)
    xg, gog, wg, bg = _layout(x.cuda(), layout), _layout(go.cuda(), layout), wt.cuda(), b.cuda()
    with _NativeRan() as rec:
        y = wmma_fwd(xg, wg, bg, 1, pad)
        dw = wmma_dw(xg, wg, gog, 1, pad)
        dx = wmma_dx(xg, wg, gog, 1, pad)
    assert {"row", "wgrad"} <= rec.kinds, rec.kinds
    _assert_layout(y, layout)
    _assert_layout(dx, layout)
    assert dw.shape == wt.shape and dw.dtype == dtype  # OIDHW in go.dtype, as the reference's wmma_dw
    assert y.dtype == dtype and dx.dtype == dtype
    assert max_rel(y, y_ref) <= TOL_FWD
    assert max_rel(dx, dx_ref) <= TOL_DX
    assert max_rel(dw, dw_ref) <= TOL_DW


@requires_gfx950
def test_isolated_passes_fall_back_on_unsupported_geometry():
    """Stride 2 is not a native geometry: wmma_* return the stock results instead of raising."""
    from rdna4_conv3d import wmma_dw, wmma_dx, wmma_fwd
    x = gen((1, 8, 8, 8, 8), 0, torch.float16).cuda()
    wt = (gen((8, 8, 3, 3, 3), 1, torch.float16) * 0.1).to(torch.float16).cuda()
    go = gen((1, 8, 4, 4, 4), 2, torch.float16).cuda()
    y = wmma_fwd(x, wt, None, 2, 1)
    torch.testing.assert_close(y, F.conv3d(x, wt, None, 2, 1), atol=1e-2, rtol=1e-2)
    dw = wmma_dw(x, wt, go, 2, 1)
    torch.testing.assert_close(dw, torch.nn.grad.conv3d_weight(x, wt.shape, go, 2, 1), atol=1e-2, rtol=1e-2)
    dx = wmma_dx(x, wt, go, 2, 1)
    torch.testing.assert_close(dx, torch.nn.grad.conv3d_input(x.shape, wt, go, 2, 1), atol=1e-2, rtol=1e-2)


# ---------------------------------------------------------------------------
# ConvTranspose3dWmma
# ---------------------------------------------------------------------------
@requires_gfx950
@pytest.mark.parametrize("mode", ["fp32", "bf16", "amp_bf16", "amp_fp16"])
@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("case", [(2, 48, 24, 4, 8, 16), (1, 16, 8, 3, 4, 5)],
                         ids=lambda c: "n{}c{}-{}_{}x{}x{}".format(*c))
def test_convt_module(case, layout, mode):
    from rdna4_conv3d import ConvTranspose3dWmma
    n, cin, cout, d, h, w = case
    print(f"case ConvTranspose3dWmma {case} {layout} {mode}", flush=True)
    param_dtype = {"fp32": torch.float32, "bf16": torch.bfloat16}.get(mode, torch.float32)
    amp = {"amp_bf16": torch.bfloat16, "amp_fp16": torch.float16}.get(mode)
    compute = amp or (param_dtype if param_dtype != torch.float32 else torch.float16)
    torch.manual_seed(2)
    up = ConvTranspose3dWmma(cin, cout, 2, stride=2).cuda().to(param_dtype)
    x = gen((n, cin, d, h, w), 0).to(param_dtype)
    xg = _layout(x.cuda(), layout).requires_grad_(True)
    go = gen((n, cout, 2 * d, 2 * h, 2 * w), 2).to(compute)
    with _NativeRan() as rec:
        with torch.autocast("cuda", dtype=amp or torch.bfloat16, enabled=amp is not None):
            y = up(xg)
        y.backward(_layout(go.cuda(), layout).to(y.dtype))
    assert "row" in rec.kinds, rec.kinds
    assert y.dtype == (amp or param_dtype)
    _assert_layout(y, layout)
    _assert_layout(xg.grad, layout)
    assert up.weight.grad.dtype == param_dtype and xg.grad.dtype == param_dtype
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(xg.detach().to(compute), up.weight.detach().to(compute),
                                              up.bias.detach().to(compute), 0, go, transpose=True)
    e = (max_rel(y, y_ref), max_rel(xg.grad, dx_ref), max_rel(up.weight.grad, dw_ref), max_rel(up.bias.grad, db_ref))
    print(f"  maxrel y {e[0]:.2e} dx {e[1]:.2e} dw {e[2]:.2e} db {e[3]:.2e}", flush=True)
    assert e[0] <= TOL_FWD and e[1] <= TOL_DX and e[2] <= TOL_DW and e[3] <= TOL_DW


@requires_gfx950
def test_convt_output_size_runs_stock():
    """forward(x, output_size) is honoured (the reference drops it): the stock module runs."""
    from rdna4_conv3d import ConvTranspose3dWmma
    torch.manual_seed(0)
    up = ConvTranspose3dWmma(8, 4, 2, stride=2).cuda()
    ref = nn.ConvTranspose3d(8, 4, 2, stride=2).cuda()
    ref.load_state_dict(up.state_dict())
    x = gen((1, 8, 3, 4, 5), 0).cuda()
    y = up(x, output_size=[7, 9, 11])
    assert y.shape == (1, 4, 7, 9, 11)
    torch.testing.assert_close(y, ref(x, output_size=[7, 9, 11]), atol=1e-5, rtol=1e-5)


@requires_gfx950
def test_convt_misaligned_input_is_handled():
    """An input whose storage starts 2 bytes past an aligned address (storage
    offset 1) no longer raises: every pass returns the float64 reference's
    results within the north-star bounds."""
    from rdna4_conv3d import ConvTranspose3dWmma
    torch.manual_seed(0)
    up = ConvTranspose3dWmma(16, 8, 2, stride=2).cuda().to(torch.bfloat16)
    base = gen((1 * 16 * 4 * 4 * 32 + 1,), 0, torch.bfloat16).cuda()
    x = base[1:].view(1, 16, 4, 4, 32)
    assert x.data_ptr() % 4 == 2
    x.requires_grad_(True)
    go = gen((1, 8, 8, 8, 64), 2, torch.bfloat16)
    y = up(x)
    y.backward(go.cuda())
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(x.detach(), up.weight.detach(), up.bias.detach(), 0, go,
                                              transpose=True)
    assert max_rel(y, y_ref) <= TOL_FWD
    assert max_rel(x.grad, dx_ref) <= TOL_DX
    assert max_rel(up.weight.grad, dw_ref) <= TOL_DW
    assert max_rel(up.bias.grad, db_ref) <= TOL_DW


@requires_gfx950
def test_conv3d_misaligned_input():
    """A Conv3d input at storage offset 1 runs natively (scalar staging) and matches float64."""
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(0)
    conv = Conv3dWmma(16, 24, 3, padding=1).cuda().to(torch.bfloat16)
    base = gen((16 * 4 * 8 * 16 + 1,), 0, torch.bfloat16).cuda()
    x = base[1:].view(1, 16, 4, 8, 16).requires_grad_(True)
    go = gen((1, 24, 4, 8, 16), 2, torch.bfloat16)
    with _NativeRan() as rec:
        y = conv(x)
        y.backward(go.cuda())
    assert "row" in rec.kinds
    y_ref, dx_ref, dw_ref, db_ref = _ref_conv(x.detach(), conv.weight.detach(), conv.bias.detach(), 1, go)
    assert max_rel(y, y_ref) <= TOL_FWD
    assert max_rel(x.grad, dx_ref) <= TOL_DX
    assert max_rel(conv.weight.grad, dw_ref) <= TOL_DW
    assert max_rel(conv.bias.grad, db_ref) <= TOL_DW


# ---------------------------------------------------------------------------
# Stock fallbacks on the GPU (reference tests/test_conv3d.py:38-44 and the
# geometries its policy declines)
# ---------------------------------------------------------------------------
FALLBACKS = [
    dict(kernel_size=3, stride=2, padding=1),                 # the reference's own fallback case
    dict(kernel_size=3, padding=1, groups=2),
    dict(kernel_size=3, padding=1, padding_mode="reflect"),
    dict(kernel_size=3, padding="same"),
    dict(kernel_size=3, padding=2, dilation=2),
    dict(kernel_size=5, padding=2),
]


@requires_gfx950
@pytest.mark.parametrize("kw", FALLBACKS, ids=lambda k: "-".join(f"{a}{b}" for a, b in k.items()))
def test_conv3d_module_stock_fallback(kw):
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(0)
    conv = Conv3dWmma(4, 6, **kw).cuda()
    ref = nn.Conv3d(4, 6, **kw).cuda()
    ref.load_state_dict(conv.state_dict())
    x = gen((1, 4, 8, 8, 8), 0).cuda()
    x1, x2 = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    y = conv(x1)
    y2 = ref(x2)
    torch.testing.assert_close(y, y2, atol=1e-5, rtol=1e-5)
    g = gen(tuple(y.shape), 2).cuda()
    y.backward(g)
    y2.backward(g)
    torch.testing.assert_close(x1.grad, x2.grad, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(conv.weight.grad, ref.weight.grad, atol=1e-4, rtol=1e-4)
