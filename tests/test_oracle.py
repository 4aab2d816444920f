"""Pins the C oracle (oracle/conv3d_oracle.c) before anything is checked against it.

Checks, chosen so that a plausible mistake (dropped or shifted padding, a
missing kernel flip, a transposed tap, a wrong ConvTranspose tap order, a dropped
bias gradient) fails at least one of them:
  * the golden vectors (torch float64 F.conv3d / conv_transpose3d / autograd,
    tests/golden/conv3d_golden.npz);
  * torch float64 on random shapes, all paddings 0..2, k = 1 and 3;
  * closed forms: the impulse response of a correlation is the weight window,
    k=1 is a channel matmul, ConvTranspose k2s2 writes each output voxel from
    exactly one tap (no overlap);
  * adjoint identities <conv(x), dy> = <x, dX(dy)> and <conv(x; w), dy> = <w, dW(x, dy)>;
  * planted faults (oracle_set_fault) must each be caught by the checks above.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc

GOLDEN = Path(__file__).resolve().parent / "golden" / "conv3d_golden.npz"


def rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-300))


@pytest.fixture(autouse=True)
def _no_fault():
    orc.set_fault(orc.FAULT_NONE)
    yield
    orc.set_fault(orc.FAULT_NONE)


# ---------------------------------------------------------------- golden vectors
def _golden_checks():
    z = np.load(GOLDEN)
    names = sorted({k.split(".")[0] for k in z.files})
    errs = {}
    for nm in names:
        g = {k.split(".")[1]: z[k] for k in z.files if k.startswith(nm + ".")}
        if nm.startswith("conv_"):
            n, cin, cout, d, h, w, k, pad = (int(v) for v in g["meta"])
            y = orc.conv3d_fwd(g["x"], g["w"], g["b"], pad)
            dx = orc.conv3d_dx(g["dy"], g["w"], g["x"].shape, pad)
            dw, db = orc.conv3d_dw(g["x"], g["dy"], k, pad)
        else:
            y = orc.convt_fwd(g["x"], g["w"], g["b"])
            dx = orc.convt_dx(g["dy"], g["w"], g["x"].shape)
            dw, db = orc.convt_dw(g["x"], g["dy"])
        errs[nm] = max(rel(y, g["y"]), rel(dx, g["dx"]), rel(dw, g["dw"]), rel(db, g["db"]))
    return errs


def test_oracle_matches_golden_vectors():
    errs = _golden_checks()
    assert len(errs) == 7
    for nm, e in errs.items():
        assert e < 1e-6, (nm, e)


# ---------------------------------------------------------------- torch float64
def _torch_checks(seed=0):
    rng = np.random.default_rng(seed)
    worst = 0.0
    for k in (1, 3):
        for pad in (0, 1, 2):
            n, cin, cout = 2, int(rng.integers(1, 5)), int(rng.integers(1, 5))
            d, h, w = (int(v) for v in rng.integers(k, 6, size=3))
            x = rng.standard_normal((n, cin, d, h, w)).astype(np.float32)
            wt = rng.standard_normal((cout, cin, k, k, k)).astype(np.float32)
            b = rng.standard_normal(cout).astype(np.float32)
            xt = torch.from_numpy(x).double().requires_grad_(True)
            wtt = torch.from_numpy(wt).double().requires_grad_(True)
            bt = torch.from_numpy(b).double().requires_grad_(True)
            y = F.conv3d(xt, wtt, bt, 1, pad)
            dy = rng.standard_normal(tuple(y.shape)).astype(np.float32)
            y.backward(torch.from_numpy(dy).double())
            dw, db = orc.conv3d_dw(x, dy, k, pad)
            worst = max(worst, rel(orc.conv3d_fwd(x, wt, b, pad), y.detach()),
                        rel(orc.conv3d_dx(dy, wt, x.shape, pad), xt.grad), rel(dw, wtt.grad), rel(db, bt.grad))
    # ConvTranspose k2s2
    x = rng.standard_normal((2, 3, 2, 3, 4)).astype(np.float32)
    wt = rng.standard_normal((3, 5, 2, 2, 2)).astype(np.float32)
    b = rng.standard_normal(5).astype(np.float32)
    xt = torch.from_numpy(x).double().requires_grad_(True)
    wtt = torch.from_numpy(wt).double().requires_grad_(True)
    bt = torch.from_numpy(b).double().requires_grad_(True)
    y = F.conv_transpose3d(xt, wtt, bt, stride=2)
    dy = rng.standard_normal(tuple(y.shape)).astype(np.float32)
    y.backward(torch.from_numpy(dy).double())
    dw, db = orc.convt_dw(x, dy)
    worst = max(worst, rel(orc.convt_fwd(x, wt, b), y.detach()), rel(orc.convt_dx(dy, wt, x.shape), xt.grad),
                rel(dw, wtt.grad), rel(db, bt.grad))
    return worst


def test_oracle_matches_torch_float64():
    assert _torch_checks() < 1e-6


# ---------------------------------------------------------------- closed forms
def _impulse_check():
    """A correlation's response to a unit impulse at i0 is y[i0 - t + p] = w[t]."""
    worst = 0.0
    for pad in (0, 1, 2):
        x = np.zeros((1, 1, 7, 7, 7), np.float32)
        x[0, 0, 3, 3, 3] = 1.0
        wt = np.arange(2 * 27, dtype=np.float32).reshape(2, 1, 3, 3, 3) + 1.0
        y = orc.conv3d_fwd(x, wt, None, pad)
        for kd in range(3):
            for kh in range(3):
                for kw in range(3):
                    o = (3 - kd + pad, 3 - kh + pad, 3 - kw + pad)
                    worst = max(worst, abs(float(y[0, :, o[0], o[1], o[2]][0]) - float(wt[0, 0, kd, kh, kw])),
                                abs(float(y[0, :, o[0], o[1], o[2]][1]) - float(wt[1, 0, kd, kh, kw])))
        assert abs(float(y.sum()) - float(wt.sum())) < 1e-3
    return worst


def test_impulse_response_is_weight_window():
    assert _impulse_check() == 0.0


def test_k1_is_channel_matmul():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 6, 3, 4, 5)).astype(np.float32)
    wt = rng.standard_normal((4, 6, 1, 1, 1)).astype(np.float32)
    ref = np.einsum("ncdhw,oc->nodhw", x.astype(np.float64), wt[:, :, 0, 0, 0].astype(np.float64))
    assert rel(orc.conv3d_fwd(x, wt, None, 0), ref) < 1e-6


def _convt_no_overlap_check():
    """Each ConvTranspose k2s2 output voxel (2i + t) is x[i] . w[:, :, t] (one tap)."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1, 3, 2, 2, 3)).astype(np.float64)
    wt = rng.standard_normal((3, 2, 2, 2, 2)).astype(np.float64)
    ref = np.zeros((1, 2, 4, 4, 6))
    for kd in range(2):
        for kh in range(2):
            for kw in range(2):
                ref[:, :, kd::2, kh::2, kw::2] = np.einsum("ncdhw,co->nodhw", x, wt[:, :, kd, kh, kw])
    return rel(orc.convt_fwd(x, wt, None), ref)


def test_convt_single_tap_per_output_voxel():
    assert _convt_no_overlap_check() < 1e-6


def _adjoint_checks():
    rng = np.random.default_rng(5)
    worst = 0.0
    for k, pad in ((3, 0), (3, 1), (3, 2), (1, 0), (1, 1)):
        x = rng.standard_normal((2, 3, 4, 5, 6)).astype(np.float32)
        wt = rng.standard_normal((4, 3, k, k, k)).astype(np.float32)
        y = orc.conv3d_fwd(x, wt, None, pad)
        dy = rng.standard_normal(y.shape).astype(np.float32)
        dx = orc.conv3d_dx(dy, wt, x.shape, pad)
        dw, db = orc.conv3d_dw(x, dy, k, pad)
        lhs = float(np.sum(y.astype(np.float64) * dy))
        worst = max(worst, abs(lhs - float(np.sum(x.astype(np.float64) * dx))) / abs(lhs),
                    abs(lhs - float(np.sum(wt.astype(np.float64) * dw))) / abs(lhs))
        worst = max(worst, rel(db, dy.astype(np.float64).sum(axis=(0, 2, 3, 4))))
    x = rng.standard_normal((2, 3, 2, 3, 4)).astype(np.float32)
    wt = rng.standard_normal((3, 4, 2, 2, 2)).astype(np.float32)
    y = orc.convt_fwd(x, wt, None)
    dy = rng.standard_normal(y.shape).astype(np.float32)
    dx = orc.convt_dx(dy, wt, x.shape)
    dw, db = orc.convt_dw(x, dy)
    lhs = float(np.sum(y.astype(np.float64) * dy))
    worst = max(worst, abs(lhs - float(np.sum(x.astype(np.float64) * dx))) / abs(lhs),
                abs(lhs - float(np.sum(wt.astype(np.float64) * dw))) / abs(lhs),
                rel(db, dy.astype(np.float64).sum(axis=(0, 2, 3, 4))))
    return worst


def test_adjoint_identities():
    assert _adjoint_checks() < 1e-5


# ---------------------------------------------------------------- planted faults
@pytest.mark.parametrize("fault", [orc.FAULT_FWD_PAD_OFF_BY_ONE, orc.FAULT_DX_NO_FLIP, orc.FAULT_DW_SWAP_HW,
                                   orc.FAULT_CONVT_TAP_ORDER, orc.FAULT_DB_DROPPED])
def test_planted_fault_is_caught(fault):
    orc.set_fault(fault)
    golden_bad = max(_golden_checks().values()) > 1e-3
    torch_bad = _torch_checks() > 1e-3
    closed_bad = (_impulse_check() > 1e-3 or _convt_no_overlap_check() > 1e-3 or _adjoint_checks() > 1e-3)
    assert golden_bad and torch_bad, f"fault {fault} slipped past the golden/torch pins"
    assert closed_bad, f"fault {fault} slipped past the closed-form/adjoint pins"


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(6)
    v = np.concatenate([(rng.standard_normal(4096) * 10.0 ** rng.integers(-8, 8, 4096)).astype(np.float32),
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.0078125, 3.3895314e38, 1e-40], np.float32)])
    ours = orc.round_bf16(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours, ref)
