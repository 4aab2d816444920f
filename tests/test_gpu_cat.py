"""Conv3dWmma.forward_cat: a k=3 Conv3d over torch.cat((xa, xb), 1) without
writing the concatenation (the UNet3D decoder's skip connection, reference
benches/unet_e2e.py:38).

On the GPU each case compares, from the same rounded inputs, the output, the
gradients of xa and xb, dW and db with a float64 CPU evaluation of
F.conv3d(torch.cat(...)); tolerances are the north star's (1e-2 fwd / dX,
3e-2 dW).  The library's launch hook must record the native kernels, and the
native result must equal (bitwise) the native conv over the materialised
concatenation: the same kernels add the same products in the same order.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from _util import gen, kaiming_weight, max_rel

pytestmark = pytest.mark.gpu


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")

CASES = [
    # (n, ca, cb, cout, d, h, w)
    (2, 24, 24, 24, 6, 16, 128),   # the level-0 decoder block (48 -> 24 over rows of 128)
    (2, 48, 48, 48, 4, 10, 64),    # level 1 (96 -> 48, rows of 64)
    (1, 96, 96, 96, 4, 8, 32),     # level 2 (192 -> 96, rows of 32)
    (2, 16, 8, 20, 5, 7, 64),      # ragged: split at 16, 24 input channels, 20 outputs
]


def _ref(xa, xb, w, b, go):
    xa_ = xa.detach().double().cpu().requires_grad_(True)
    xb_ = xb.detach().double().cpu().requires_grad_(True)
    w_ = w.detach().double().cpu().requires_grad_(True)
    b_ = b.detach().double().cpu().requires_grad_(True)
    y = F.conv3d(torch.cat((xa_, xb_), 1), w_, b_, 1, 1)
    y.backward(go.double().cpu())
    return y.detach(), xa_.grad, xb_.grad, w_.grad, b_.grad


@requires_gfx950
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}a{}b{}o{}_{}x{}x{}".format(*c))
def test_forward_cat_matches_reference_and_materialised_cat(case, dtype):
    from rdna4_conv3d import Conv3dWmma
    from rdna4_conv3d import _native
    n, ca, cb, co, d, h, w = case
    print(f"case forward_cat {case} {dtype}", flush=True)
    xa = gen((n, ca, d, h, w), 0).to(dtype)
    xb = gen((n, cb, d, h, w), 1).to(dtype)
    go = gen((n, co, d, h, w), 2).to(dtype)
    wt = kaiming_weight((co, ca + cb, 3, 3, 3), (ca + cb) * 27, 3, dtype)
    bt = gen((co,), 4, dtype)
    ref = _ref(xa, xb, wt, bt, go)
    conv = Conv3dWmma(ca + cb, co, 3, padding=1).cuda().to(dtype)
    with torch.no_grad():
        conv.weight.copy_(wt)
        conv.bias.copy_(bt)
    outs = []
    for use_cat in (True, False):
        conv.zero_grad()
        a_ = xa.cuda().requires_grad_(True)
        b_ = xb.cuda().requires_grad_(True)
        _native.timing_filter(-1, None)
        _native.timing_enable(True)
        _native.timing_collect()
        y = conv.forward_cat(a_, b_) if use_cat else conv(torch.cat((a_, b_), 1))
        y.backward(go.cuda())
        torch.cuda.synchronize()
        kinds = {k for _, k, _ in _native.timing_collect()}
        _native.timing_enable(False)
        assert {"row", "wgrad"} <= kinds, kinds
        outs.append([t.detach().cpu() for t in (y, a_.grad, b_.grad, conv.weight.grad, conv.bias.grad)])
    y, ga, gb, gw, gbias = outs[0]
    e = {"y": max_rel(y, ref[0]), "dxa": max_rel(ga, ref[1]), "dxb": max_rel(gb, ref[2]),
         "dw": max_rel(gw, ref[3]), "db": max_rel(gbias, ref[4])}
    print("  " + " ".join(f"{k} {v:.2e}" for k, v in e.items()), flush=True)
    tol = {"y": 1e-2, "dxa": 1e-2, "dxb": 1e-2, "dw": 3e-2, "db": 3e-2}
    for k, v in e.items():
        assert v <= tol[k], f"{k}: {v:.3e} > {tol[k]}"
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


@requires_gfx950
def test_forward_cat_under_autocast_keeps_fp32_params():
    """fp32 module and inputs under bf16 autocast: bf16 output, fp32 grads of the parameters."""
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(0)
    conv = Conv3dWmma(48, 24, 3, padding=1).cuda()
    xa = gen((2, 24, 4, 8, 64), 0).cuda().requires_grad_(True)
    xb = gen((2, 24, 4, 8, 64), 1).cuda().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = conv.forward_cat(xa, xb)
    assert y.dtype == torch.bfloat16
    y.float().sum().backward()
    assert conv.weight.grad.dtype == torch.float32 and conv.bias.grad.dtype == torch.float32
    assert xa.grad.dtype == torch.float32 and xb.grad.shape == xb.shape


@requires_gfx950
def test_forward_cat_falls_back_where_no_plan():
    """Rows of 16 positions (no row-walking dW plan) and a split off the 8-channel
    blocks run torch.cat + forward; results equal the module on the concatenation."""
    from rdna4_conv3d import Conv3dWmma
    torch.manual_seed(0)
    for ca, cb, w in [(24, 24, 16), (12, 12, 64)]:
        conv = Conv3dWmma(ca + cb, 8, 3, padding=1).cuda().to(torch.bfloat16)
        xa = gen((1, ca, 4, 8, w), 0, torch.bfloat16).cuda()
        xb = gen((1, cb, 4, 8, w), 1, torch.bfloat16).cuda()
        assert not conv._cat_native_ok(xa, xb)
        torch.testing.assert_close(conv.forward_cat(xa, xb), conv(torch.cat((xa, xb), 1)), atol=0, rtol=0)
