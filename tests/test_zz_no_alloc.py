"""The allocation-free dW entry point r3c_conv3d_dw_static (workspace in the
library's static device array) against r3c_conv3d_dw with a caller workspace:
called through the C ABI, two calls in a row on one GPU -- the second with a
smaller input, so it runs on scratch the first call left behind -- each
bitwise equal to the allocating entry point (same plan, same fixed-order sums)
and within the north-star dW bound of the float64 reference.  The size check
(a pass needing more than the 64 MiB array) is host-side and runs without a
GPU."""
from __future__ import annotations

import ctypes

import pytest
import torch
import torch.nn.functional as F

from _util import gen, kaiming_weight, max_rel

TOL_DW = 3e-2


def _gpu_ok():
    if not torch.cuda.is_available():
        return False
    return (torch.cuda.get_device_properties(0).gcnArchName or "").startswith("gfx950")


def _desc(nat, x, go, k, pad):
    return nat.make_desc(x.shape, go.shape, k, (pad,) * 3, x.dtype, x.stride(), go.stride())


def test_static_dw_rejects_passes_beyond_the_scratch_on_host():
    from rdna4_conv3d import _native as nat
    lib = nat.load()
    # 96 -> 96 channels over many positions: the plan wants more than 64 MiB of partials
    x = torch.empty(4, 192, 32, 64, 64, dtype=torch.bfloat16, device="meta")
    go = torch.empty(4, 192, 32, 64, 64, dtype=torch.bfloat16, device="meta")
    d = _desc(nat, x, go, 3, 1)
    need = lib.r3c_conv3d_dw_workspace(ctypes.byref(d))
    assert need > (64 << 20)
    rc = lib.r3c_conv3d_dw_static(ctypes.byref(d), None, None, None, nat.R3C_F32, None, nat.R3C_F32, None)
    assert rc == nat.R3C_UNSUPPORTED
    msg = lib.r3c_last_error().decode()
    assert str(need) in msg and str(64 << 20) in msg


CASES = [
    # (n, cin, cout, d, h, w, k, pad, layout): first call, then a smaller second call
    ((2, 24, 24, 8, 32, 32, 3, 1, "ncdhw"), (1, 16, 8, 4, 8, 16, 3, 1, "ncdhw")),
    ((1, 48, 40, 6, 16, 24, 3, 1, "ndhwc"), (1, 8, 24, 4, 6, 8, 3, 0, "ndhwc")),
    ((2, 40, 72, 4, 8, 24, 1, 0, "ncdhw"), (1, 24, 96, 2, 8, 32, 1, 0, "ncdhw")),
]


@pytest.mark.gpu
@pytest.mark.skipif(not _gpu_ok(), reason="needs a gfx950 GPU")
@pytest.mark.parametrize("pair", CASES, ids=lambda p: "{}then{}".format(p[0][:6], p[1][:6]))
def test_static_dw_matches_allocating_entry_point(pair):
    from rdna4_conv3d import _native as nat
    lib = nat.load()
    dev = torch.device("cuda", 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    for (n, cin, cout, d, h, w, k, pad, layout) in pair:
        print(f"case static dW {(n, cin, cout, d, h, w, k, pad, layout)}", flush=True)
        dt = torch.bfloat16
        fmt = torch.channels_last_3d if layout == "ndhwc" else torch.contiguous_format
        x = gen((n, cin, d, h, w), 0, dt).to(dev).contiguous(memory_format=fmt)
        od, oh, ow = d + 2 * pad - k + 1, h + 2 * pad - k + 1, w + 2 * pad - k + 1
        go = gen((n, cout, od, oh, ow), 2, dt).to(dev).contiguous(memory_format=fmt)
        desc = _desc(nat, x, go, k, pad)
        need = lib.r3c_conv3d_dw_workspace(ctypes.byref(desc))
        assert 0 <= need <= (64 << 20)
        ws = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
        dw_a = torch.empty(cout, cin, k, k, k, dtype=torch.float32, device=dev)
        db_a = torch.empty(cout, dtype=torch.float32, device=dev)
        dw_s = torch.full_like(dw_a, float("nan"))
        db_s = torch.full_like(db_a, float("nan"))
        P = lambda t: ctypes.c_void_p(t.data_ptr())
        rc = lib.r3c_conv3d_dw(ctypes.byref(desc), P(x), P(go), P(dw_a), nat.R3C_F32, P(db_a), nat.R3C_F32, P(ws),
                               ws.numel(), stream)
        assert rc == 0, lib.r3c_last_error()
        rc = lib.r3c_conv3d_dw_static(ctypes.byref(desc), P(x), P(go), P(dw_s), nat.R3C_F32, P(db_s), nat.R3C_F32,
                                      stream)
        assert rc == 0, lib.r3c_last_error()
        torch.cuda.synchronize()
        assert torch.equal(dw_s, dw_a) and torch.equal(db_s, db_a)
        xd = x.double().cpu()
        god = go.double().cpu()
        dw_ref = torch.nn.grad.conv3d_weight(xd, dw_a.shape, god, 1, pad)
        assert max_rel(dw_s, dw_ref) <= TOL_DW
        assert max_rel(db_s, god.sum((0, 2, 3, 4))) <= TOL_DW
