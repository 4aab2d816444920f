"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, agrees with the header on the ABI version and the descriptor
layout, and validates descriptors on the host (no compute calls here)."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from rdna4_conv3d import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "rdna4_conv3d.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(r3c_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _native.load()
    names = _declared()
    assert len(names) >= 18
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.library_path())], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\bT (r3c_\w+)", out))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert getattr(lib, n) is not None


def test_abi_version_matches_header():
    m = re.search(r"#define R3C_ABI_VERSION (\d+)", HEADER.read_text())
    assert _native.load().r3c_abi_version() == int(m.group(1)) == _native.ABI_VERSION


def test_descriptor_layout_matches_c(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "rdna4_conv3d.h"\n'
        "int main(void){printf(\"%zu %zu %zu %zu\\n\", sizeof(r3c_conv_desc), offsetof(r3c_conv_desc, kernel),"
        " offsetof(r3c_conv_desc, x_strides), offsetof(r3c_conv_desc, y_strides)); return 0;}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()
    D = _native.ConvDesc
    assert [int(v) for v in got] == [ctypes.sizeof(D), D.kernel.offset, D.x_strides.offset, D.y_strides.offset]


@pytest.mark.parametrize("name,fields", [
    ("r3c_bn_desc", ("s", "y_strides", "g_strides", "o_strides", "training", "eps", "momentum")),
    ("r3c_pool_desc", ("w", "x_strides", "y_strides")),
])
def test_bn_and_pool_descriptor_layouts_match_c(tmp_path, name, fields):
    src = tmp_path / "layout.c"
    offs = "".join(f", offsetof({name}, {f})" for f in fields)
    fmt = " ".join(["%zu"] * (len(fields) + 1))
    src.write_text(
        '#include <stdio.h>\n#include <stddef.h>\n#include "rdna4_conv3d.h"\n'
        f'int main(void){{printf("{fmt}\\n", sizeof({name}){offs}); return 0;}}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    D = _native.BnDesc if name == "r3c_bn_desc" else _native.PoolDesc
    assert got == [ctypes.sizeof(D)] + [getattr(D, f).offset for f in fields]


def _desc(k=3, pad=1, n=2, cin=8, cout=16, sp=(6, 7, 9), transpose=False, dtype=_native.R3C_BF16):
    import torch
    d, h, w = sp
    if transpose:
        od, oh, ow = 2 * d, 2 * h, 2 * w
    else:
        od, oh, ow = d + 2 * pad - k + 1, h + 2 * pad - k + 1, w + 2 * pad - k + 1
    x = torch.empty(n, cin, d, h, w)
    y = torch.empty(n, cout, od, oh, ow)
    desc = _native.make_desc(x.shape, y.shape, k, (pad,) * 3, torch.bfloat16, x.stride(), y.stride())
    desc.dtype = dtype
    return desc


def test_workspace_queries_validate_on_host():
    lib = _native.load()
    ok = _desc()
    assert lib.r3c_conv3d_fwd_workspace(ctypes.byref(ok)) > 0
    assert lib.r3c_conv3d_dx_workspace(ctypes.byref(ok)) > 0
    assert lib.r3c_conv3d_dw_workspace(ctypes.byref(ok)) > 0
    t = _desc(k=2, pad=0, transpose=True)
    for name in ("fwd", "dx", "dw"):
        assert getattr(lib, f"r3c_convt_k2s2_{name}_workspace")(ctypes.byref(t)) > 0
    assert lib.r3c_conv3d_fwd_workspace(ctypes.byref(_desc(k=5, pad=2))) == -1   # kernel 5
    bad = _desc()
    bad.od += 1                                                                  # inconsistent dims
    assert lib.r3c_conv3d_fwd_workspace(ctypes.byref(bad)) == -1
    assert lib.r3c_conv3d_fwd_workspace(ctypes.byref(_desc(dtype=_native.R3C_F32))) == -1
    assert lib.r3c_convt_k2s2_fwd_workspace(ctypes.byref(ok)) == -1             # k3 desc on ConvT


def test_invalid_calls_fail_before_touching_a_device():
    lib = _native.load()
    rc = lib.r3c_conv3d_fwd(None, None, None, None, None, None, 0, None)
    assert rc == _native.R3C_INVALID
    assert b"NULL" in lib.r3c_last_error()
    bad = _desc(k=5, pad=2)
    assert lib.r3c_conv3d_dw(ctypes.byref(bad), None, None, None, 2, None, 2, None, 0, None) == _native.R3C_UNSUPPORTED
    assert b"kernel 5" in lib.r3c_last_error()


@pytest.mark.parametrize("k,pad", [(3, 1), (3, 0), (1, 0), (1, 2)])
def test_dw_workspace_scales_with_problem(k, pad):
    lib = _native.load()
    small = lib.r3c_conv3d_dw_workspace(ctypes.byref(_desc(k=k, pad=pad, sp=(4, 4, 16))))
    big = lib.r3c_conv3d_dw_workspace(ctypes.byref(_desc(k=k, pad=pad, sp=(32, 64, 64))))
    assert 0 < small <= big <= (96 << 20) + (1 << 20)


def _desc_strided(shape_x, shape_y, k, pad, channels_last=False, transpose=False):
    """Descriptor with dense NCDHW (or NDHWC) strides computed from the shapes
    (no tensor is allocated, so samples past 1 GiB cost nothing here)."""
    def st(s):
        n, c, d, h, w = s
        return (c * d * h * w, 1, h * w * c, w * c, c) if channels_last else (c * d * h * w, d * h * w, h * w, w, 1)
    import torch
    return _native.make_desc(shape_x, shape_y, k, (pad,) * 3, torch.bfloat16, st(shape_x), st(shape_y))


@pytest.mark.parametrize("channels_last", [False, True], ids=["ncdhw", "ndhwc"])
def test_workspace_query_rejects_samples_of_1gib(channels_last):
    """A sample of 1 GiB or more needs offsets past the kernels' 32-bit buffer
    ranges: every workspace query returns -1 for it (the caller falls back
    before running anything), while the same layer at half the depth is
    accepted."""
    lib = _native.load()
    big_x = (1, 64, 128, 256, 256)   # 2^30 bytes of bf16 per sample
    ok_x = (1, 64, 64, 256, 256)
    for xs, expect_ok in ((big_x, False), (ok_x, True)):
        for k, pad in ((3, 1), (1, 0)):
            d = _desc_strided(xs, (xs[0], 64) + xs[2:], k, pad, channels_last)
            for name in ("fwd", "dx", "dw"):
                v = getattr(lib, f"r3c_conv3d_{name}_workspace")(ctypes.byref(d))
                assert (v >= 0) == expect_ok, (xs, k, name, v)
        t = _desc_strided(xs, (xs[0], 8) + tuple(2 * v for v in xs[2:]), 2, 0, channels_last, transpose=True)
        for name in ("fwd", "dx", "dw"):
            v = getattr(lib, f"r3c_convt_k2s2_{name}_workspace")(ctypes.byref(t))
            assert (v >= 0) == expect_ok, (xs, name, v)


def test_plan_check_declines_1gib_sample_on_host():
    """The Python predicate the autograd Functions use before a native forward
    (conv_plans_ok) says no for the 1 GiB sample and yes at half its depth;
    meta tensors carry the shapes and strides, nothing is allocated."""
    import torch
    big = torch.empty(1, 64, 128, 256, 256, dtype=torch.bfloat16, device="meta")
    ok = torch.empty(1, 64, 64, 256, 256, dtype=torch.bfloat16, device="meta")
    w = (64, 64, 3, 3, 3)
    assert not _native.conv_plans_ok(big, w, (1, 1, 1), torch.bfloat16)
    assert _native.conv_plans_ok(ok, w, (1, 1, 1), torch.bfloat16)
    assert not _native.convt_plans_ok(big, (64, 8, 2, 2, 2), torch.bfloat16)
    assert _native.convt_plans_ok(ok, (64, 8, 2, 2, 2), torch.bfloat16)


def test_bn_workspace_query_validates_on_host():
    """BatchNorm + ReLU descriptors: the workspace query accepts planes the
    16-byte kernels take and returns -1 otherwise (the module then runs stock)."""
    lib = _native.load()

    def bn_desc(n, c, s, dtype, stride_c=None):
        d = _native.BnDesc()
        d.dtype, d.n, d.c, d.s = dtype, n, c, s
        sc = s if stride_c is None else stride_c
        d.y_strides[0] = d.g_strides[0] = d.o_strides[0] = c * sc
        d.y_strides[1] = d.g_strides[1] = d.o_strides[1] = sc
        d.training, d.eps, d.momentum = 1, 1e-5, 0.1
        return d

    ok = bn_desc(4, 24, 64 * 128 * 128, _native.R3C_BF16)
    ws = lib.r3c_bn_relu_workspace(ctypes.byref(ok))
    nchunk = -(-64 * 128 * 128 // 8192)
    assert ws >= 4 * nchunk * 24 * 2 * 4 + 24 * 16
    assert lib.r3c_bn_relu_workspace(ctypes.byref(bn_desc(2, 8, 12, _native.R3C_F32))) > 0      # 12 % 4 == 0
    assert lib.r3c_bn_relu_workspace(ctypes.byref(bn_desc(2, 8, 12, _native.R3C_BF16))) == -1    # 12 % 8 != 0
    assert lib.r3c_bn_relu_workspace(ctypes.byref(bn_desc(2, 8, 16, _native.R3C_BF16, 20))) == -1  # odd stride
    assert lib.r3c_bn_relu_workspace(ctypes.byref(bn_desc(1, 70000, 16, _native.R3C_BF16))) == -1
    assert lib.r3c_bn_relu_workspace(ctypes.byref(bn_desc(0, 8, 16, _native.R3C_BF16))) == -1
    rc = lib.r3c_bn_relu_fwd(ctypes.byref(ok), None, None, None, None, None, None, None, None, None, 0, None)
    assert rc == _native.R3C_INVALID


def test_pool_descriptors_validate_on_host():
    """MaxPool3d(2) entry points reject shapes and strides the 16-byte kernels
    do not take with R3C_UNSUPPORTED, and NULL pointers with R3C_INVALID, all
    before any device call."""
    lib = _native.load()

    def call(shape, dtype=_native.R3C_BF16, xs=None, ys=None):
        n, c, d, h, w = shape
        desc = _native.PoolDesc()
        desc.dtype, desc.n, desc.c, desc.d, desc.h, desc.w = dtype, n, c, d, h, w
        pin = d * h * w
        pout = pin // 8
        desc.x_strides[0], desc.x_strides[1] = xs if xs else (c * pin, pin)
        desc.y_strides[0], desc.y_strides[1] = ys if ys else (c * pout, pout)
        return (lib.r3c_maxpool2_fwd(ctypes.byref(desc), None, None, None, None),
                lib.r3c_maxpool2_bwd(ctypes.byref(desc), None, None, None, None))

    U, I = _native.R3C_UNSUPPORTED, _native.R3C_INVALID
    assert call((4, 24, 64, 128, 128)) == (I, I)          # valid descriptor, NULL pointers
    assert call((2, 8, 4, 4, 8), _native.R3C_F32) == (I, I)
    assert call((2, 8, 5, 4, 8)) == (U, U)                # odd d
    assert call((2, 8, 4, 3, 8)) == (U, U)                # odd h
    assert call((2, 8, 4, 4, 12)) == (U, U)               # w % 8
    assert call((2, 8, 4, 4, 8), xs=(8 * 128 + 4, 128)) == (U, U)  # x sample stride not a multiple of 8
    assert call((2, 8, 2, 2, 8)) == (I, I)                # y channel stride 4
    assert call((2, 8, 4, 4, 8), ys=(8 * 16 + 2, 16)) == (U, U)    # y sample stride not a multiple of 4
    assert call((2, 8, 4, 4, 8), dtype=7) == (U, U)
    assert lib.r3c_maxpool2_fwd(None, None, None, None, None) == I


def test_cat_workspace_query_decides_on_host():
    """Conv3d over a channel concatenation: the workspace query accepts k=3
    NCDHW layers whose three passes have plans (rows of 32-128 positions, a
    split on the 8-channel blocks) and returns -1 otherwise; bad descriptors
    are refused before any device call."""
    import torch
    lib = _native.load()

    def q(n, ca, cb, co, d, h, w, pass_=2, channels_last=False):
        x_shape, y_shape = (n, ca, d, h, w), (n, co, d, h, w)  # k=3, padding 1
        desc = _native._cat_desc(x_shape, cb, y_shape, 3, (1, 1, 1), torch.bfloat16,
                                 _native._dense_strides(y_shape, False))
        if channels_last:
            xs = _native._dense_strides((n, ca + cb, d, h, w), True)
            for i in range(5):
                desc.x_strides[i] = xs[i]
        return lib.r3c_conv3d_cat_workspace(ctypes.byref(desc), ca, cb * d * h * w, pass_)

    for p in (0, 1, 2):
        assert q(2, 24, 24, 24, 8, 16, 128, pass_=p) >= 0
        assert q(2, 48, 48, 48, 8, 16, 64, pass_=p) >= 0
    assert q(2, 12, 12, 24, 8, 16, 64) == -1          # split off the 8-channel blocks
    assert q(2, 24, 24, 24, 8, 16, 16) == -1          # rows of 16: no row-walking dW plan
    assert q(2, 24, 24, 24, 8, 16, 64, channels_last=True, pass_=0) == -1
    assert q(2, 24, 24, 24, 8, 16, 64, pass_=3) == -1
    desc = _native._cat_desc((2, 24, 8, 16, 64), 24, (2, 24, 8, 16, 64), 3, (1, 1, 1), torch.bfloat16,
                             _native._dense_strides((2, 24, 8, 16, 64), False))
    rc = lib.r3c_conv3d_cat_fwd(ctypes.byref(desc), 24, None, None, 24 * 8 * 16 * 64, None, None, None, None, 0, None)
    assert rc == _native.R3C_INVALID
    rc = lib.r3c_conv3d_cat_fwd(ctypes.byref(desc), 20, None, None, 24 * 8 * 16 * 64, None, None, None, None, 0, None)
    assert rc == _native.R3C_UNSUPPORTED


def test_strided_workspace_query_validates_on_host():
    """r3c_conv3d_strided_workspace: output dims (in + 2 pad - k) / stride + 1,
    strides 1 .. 8, a NULL stride and an unknown pass give -1; each pass of a
    valid descriptor has a plan (dW: the dY scatter plus the stride-1 dW)."""
    import torch
    lib = _native.load()
    x_shape = (2, 24, 9, 16, 17)
    y_shape = _native.strided_out_shape(x_shape, (48, 24, 3, 3, 3), (2, 2, 3), (1, 1, 0))
    assert y_shape == (2, 48, 5, 8, 5)
    x, y = torch.empty(x_shape), torch.empty(y_shape)
    d = _native.make_desc(x_shape, y_shape, 3, (1, 1, 0), torch.bfloat16, x.stride(), y.stride())
    st = _native._stride3((2, 2, 3))
    sizes = [lib.r3c_conv3d_strided_workspace(ctypes.byref(d), st, p) for p in (0, 1, 2)]
    assert all(s > 0 for s in sizes), sizes
    # dW holds the dense dY scatter onto the stride-1 grid (2 x 48 x 7 x 14 x 15 bf16) and more
    assert sizes[2] >= 2 * 48 * 7 * 14 * 15 * 2
    assert lib.r3c_conv3d_strided_workspace(ctypes.byref(d), st, 3) == -1
    assert lib.r3c_conv3d_strided_workspace(ctypes.byref(d), None, 0) == -1
    for bad in ((2, 2, 2), (0, 2, 3), (9, 2, 3)):   # dims no longer match, or stride out of range
        assert lib.r3c_conv3d_strided_workspace(ctypes.byref(d), _native._stride3(bad), 0) == -1
    # stride 1 through the strided entry points is a plain Conv3d descriptor
    y1 = torch.empty((2, 48, 9, 16, 15))
    d1 = _native.make_desc(x_shape, y1.shape, 3, (1, 1, 0), torch.bfloat16, x.stride(), y1.stride())
    assert lib.r3c_conv3d_strided_workspace(ctypes.byref(d1), _native._stride3((1, 1, 1)), 1) > 0


def test_strided_dw_workspace_covers_direct_paths():
    """The strided dW workspace holds every plan that may run: for a case the
    direct kernel takes (k=3, w stride 2, w pad 1, W % 8 == 0, OW % 16 == 0) the
    query covers the 256-split fp32 partials (at most 256 x Cout x 27 x Cin x 4
    bytes); in NDHWC it also covers the NCDHW copies of x and dY the direct
    kernel reads there."""
    import torch
    lib = _native.load()
    x_shape = (2, 24, 16, 64, 64)
    y_shape = _native.strided_out_shape(x_shape, (48, 24, 3, 3, 3), (2, 2, 2), (1, 1, 1))
    assert y_shape == (2, 48, 8, 32, 32)
    st = _native._stride3((2, 2, 2))
    x = torch.empty(x_shape)
    y = torch.empty(y_shape)
    d = _native.make_desc(x_shape, y_shape, 3, (1, 1, 1), torch.bfloat16, x.stride(), y.stride())
    ws = lib.r3c_conv3d_strided_workspace(ctypes.byref(d), st, 2)
    assert ws >= 48 * 27 * 24 * 4  # at least one split's partials
    xc = x.contiguous(memory_format=torch.channels_last_3d)
    yc = y.contiguous(memory_format=torch.channels_last_3d)
    dc = _native.make_desc(x_shape, y_shape, 3, (1, 1, 1), torch.bfloat16, xc.stride(), yc.stride())
    wsc = lib.r3c_conv3d_strided_workspace(ctypes.byref(dc), st, 2)
    copies = (x.numel() + y.numel()) * 2
    assert wsc >= copies + 48 * 27 * 24 * 4, (wsc, copies)
