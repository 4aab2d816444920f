"""BatchNormReLU3d (native BatchNorm + ReLU) against nn.BatchNorm3d + ReLU.

The module replaces the BatchNorm3d + ReLU pair of the reference's UNet3D
block (benches/unet_e2e.py:13-21).  On the GPU each case compares, from the
same input: the output, dX, dgamma, dbeta and the running statistics (and
num_batches_tracked) with a float64 CPU evaluation of nn.BatchNorm3d + ReLU
on the same (rounded) values.  Tolerances: max|out - ref| / max|ref| <= 1e-2
for the output and dX (half-precision outputs carry one rounding), 1e-3 for
the fp32 statistics, dgamma and dbeta.  The library's launch hook must record
the BatchNorm kernels, so a stock fallback cannot pass.
"""
from __future__ import annotations

import copy

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

from _util import gen, max_rel

pytestmark = pytest.mark.gpu


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


requires_gfx950 = pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")


def _ref(mod_state, x, go, training, momentum, affine):
    """float64 CPU nn.BatchNorm3d + ReLU from the same values; returns
    (z, dx, dgamma, dbeta, running_mean, running_var)."""
    bn = nn.BatchNorm3d(x.shape[1], momentum=momentum, affine=affine).double()
    bn.load_state_dict({k: v.double() if v.is_floating_point() else v for k, v in mod_state.items()})
    bn.train(training)
    xd = x.detach().double().cpu().requires_grad_(True)
    z = F.relu(bn(xd))
    z.backward(go.double().cpu())
    dg = bn.weight.grad if affine else None
    db = bn.bias.grad if affine else None
    return z.detach(), xd.grad, dg, db, bn.running_mean, bn.running_var


CASES = [
    # (n, c, d, h, w)
    (2, 24, 8, 16, 16),
    (1, 48, 4, 8, 32),
    (4, 8, 3, 5, 8),       # plane of 120 positions (not a chunk multiple)
    (2, 16, 40, 64, 64),   # several chunks per plane
]


@requires_gfx950
@pytest.mark.parametrize("momentum", [0.1, None], ids=["m0.1", "mNone"])
@pytest.mark.parametrize("mode", ["train", "eval", "train_noaffine"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "n{}c{}_{}x{}x{}".format(*c))
def test_bnrelu_matches_batchnorm_relu(case, dtype, mode, momentum):
    from rdna4_conv3d import _native
    from rdna4_conv3d.fused import BatchNormReLU3d
    n, c, d, h, w = case
    print(f"case BatchNormReLU3d {case} {dtype} {mode} momentum={momentum}", flush=True)
    affine = mode != "train_noaffine"
    training = mode != "eval"
    torch.manual_seed(0)
    mod = BatchNormReLU3d(c, momentum=momentum, affine=affine).cuda()
    with torch.no_grad():
        if affine:
            mod.weight.copy_(1.0 + 0.5 * gen((c,), 7))
            mod.bias.copy_(0.3 * gen((c,), 8))
        mod.running_mean.copy_(0.2 * gen((c,), 9))
        mod.running_var.copy_(1.0 + 0.5 * gen((c,), 10).abs())
        mod.num_batches_tracked.fill_(3)
    mod.train(training)
    state0 = copy.deepcopy({k: v.detach().cpu() for k, v in mod.state_dict().items()})
    x = (1.5 * gen((n, c, d, h, w), 0) + 0.25).to(dtype)
    go = gen((n, c, d, h, w), 2).to(dtype)
    xg = x.cuda().requires_grad_(True)
    _native.timing_filter(-1, None)
    _native.timing_enable(True)
    _native.timing_collect()
    z = mod(xg)
    z.backward(go.cuda())
    torch.cuda.synchronize()
    kinds = {k for _, k, _ in _native.timing_collect()}
    _native.timing_enable(False)
    assert "bn" in kinds, kinds
    assert z.dtype == dtype and xg.grad.dtype == dtype
    z_r, dx_r, dg_r, db_r, rm_r, rv_r = _ref(state0, x, go, training, momentum, affine)
    e = {"z": max_rel(z, z_r), "dx": max_rel(xg.grad, dx_r)}
    tol = {"z": 1e-2, "dx": 1e-2}
    if affine:
        e["dgamma"] = max_rel(mod.weight.grad, dg_r)
        e["dbeta"] = max_rel(mod.bias.grad, db_r)
        tol["dgamma"] = tol["dbeta"] = 1e-3 if dtype == torch.float32 else 1e-2
    e["running_mean"] = max_rel(mod.running_mean, rm_r)
    e["running_var"] = max_rel(mod.running_var, rv_r)
    tol["running_mean"] = tol["running_var"] = 1e-3
    print("  " + " ".join(f"{k} {v:.2e}" for k, v in e.items()), flush=True)
    for k, v in e.items():
        assert v <= tol[k], f"{k}: {v:.3e} > {tol[k]}"
    assert int(mod.num_batches_tracked) == (4 if training else 3)


@requires_gfx950
def test_bnrelu_bitwise_repeatable():
    """Fixed chunking and fixed-order sums: two runs give identical bits."""
    from rdna4_conv3d.fused import BatchNormReLU3d
    x = gen((2, 24, 16, 32, 64), 0, torch.bfloat16).cuda()
    go = gen((2, 24, 16, 32, 64), 2, torch.bfloat16).cuda()
    outs = []
    for _ in range(2):
        torch.manual_seed(0)
        mod = BatchNormReLU3d(24).cuda()
        xg = x.clone().requires_grad_(True)
        z = mod(xg)
        z.backward(go)
        torch.cuda.synchronize()
        outs.append([t.detach().cpu() for t in (z, xg.grad, mod.weight.grad, mod.bias.grad, mod.running_mean,
                                                 mod.running_var)])
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@requires_gfx950
def test_bnrelu_channels_last_falls_back_to_stock():
    """NDHWC inputs run nn.BatchNorm3d + ReLU (the native path takes NCDHW planes)."""
    from rdna4_conv3d.fused import BatchNormReLU3d
    torch.manual_seed(0)
    mod = BatchNormReLU3d(16).cuda()
    ref = nn.BatchNorm3d(16).cuda()
    ref.load_state_dict(mod.state_dict())
    x = gen((2, 16, 4, 8, 8), 0).cuda().contiguous(memory_format=torch.channels_last_3d)
    torch.testing.assert_close(mod(x), F.relu(ref(x)))
