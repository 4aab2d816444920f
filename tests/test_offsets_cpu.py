"""Out-of-range gating of the kernels' buffer loads, replayed on the CPU at the
extreme shapes the host planner admits.

The kernels read through buffer resources whose range (num_records) is one
sample (or one tensor's channel planes) and switch a load off by giving it an
offset at or past that range: either the constant kOob (0x7fffff00) plus the
channel offset, or the computed offset with bit 31 set.  That only works while
no 32-bit offset wraps back below the range.  The host guarantees it with
these bounds (csrc/r3c_capi.hip):

  * every sample (buffer range) below 1 GiB;
  * NCDHW k=3 staging (tap kernel mode 3, weight-gradient fl 3):
    2 * (C + 8) * channel_stride < 2^30;
  * padding at most 64 (halo offsets stay within a few rows of the volume).

For each formula this test enumerates the corners of the largest admitted
shapes -- first/last box, halo rows and columns outside the volume, the last
channel chunk past C -- and asserts: a load that should read is inside
[0, range), and every other load's unsigned 32-bit offset is at or past the
range.  Shrinking a bound in the host planner keeps this green; loosening one
past what the formulas tolerate makes it fail.
"""
from __future__ import annotations

import itertools

import pytest

KOOB = 0x7FFFFF00
GIB = 1 << 30


def u32(v: int) -> int:
    return v & 0xFFFFFFFF


def gate(off: int, on: bool) -> int:
    """(uint32)off | (!on << 31), as the kernels compute it (off is an int32)."""
    assert -(1 << 31) <= off < (1 << 31), "offset left int32 before gating"
    return u32(off) | (0 if on else 1 << 31)


def ncdhw_shapes():
    """NCDHW shapes at the planner's limits for the k=3 w-contiguous staging:
    2 (C + 8) * D*H*W just under 2^30 (so every sample is below 1 GiB too), W a
    multiple of 8, with ragged D and H and the largest padding the k=3 passes use."""
    out = []
    for c, w in [(8, 256), (24, 128), (64, 64), (200, 32), (1000, 8)]:
        plane_max = (GIB - 1) // (2 * (c + 8))
        hw = 37 * w                      # ragged h
        d = plane_max // hw              # as deep as the bound allows
        out.append((c, d, 37, w))
    return out


@pytest.mark.parametrize("shape", ncdhw_shapes(), ids=lambda s: "c{}_{}x{}x{}".format(*s))
@pytest.mark.parametrize("pad", [0, 1, 2])
def test_tap_mode3_staging_never_wraps_into_range(shape, pad):
    """Tap kernel mode 3: slot offset soff = 2 (gd ss2 + gh ss3 + gw) inside the
    volume, else kOob; the load of channel c0 + e adds 2 (c0 + e) ss1.  Range
    2 C ss1 (channel planes outermost)."""
    c, d, h, w = shape
    ss3, ss2, ss1 = w, h * w, d * h * w
    assert 2 * (c + 8) * ss1 < GIB
    rng = 2 * c * ss1
    lw = 32 if w >= 32 else 16
    chunks = (c + 7) // 8
    # Tile rows of the first and last box, segments covering [r0w - 8, r0w + lw + 8).
    for gd, gh in itertools.product([-pad, 0, d - 1, d - 1 + pad], [-pad, 0, h - 1, h - 1 + pad]):
        for gw in [-8, 0, w - 8, w, w + 8]:
            inside = 0 <= gd < d and 0 <= gh < h and 0 <= gw < w
            soff = 2 * (gd * ss2 + gh * ss3 + gw) if inside else KOOB
            for c0 in [0, 8 * (chunks - 1)]:
                for e in (0, 7):
                    off = soff + 2 * (c0 + e) * ss1
                    assert off < (1 << 32), "offset wrapped past 2^32"
                    if inside and c0 + e < c:
                        assert 0 <= off < rng
                    else:
                        assert u32(off) >= rng


@pytest.mark.parametrize("shape", ncdhw_shapes(), ids=lambda s: "c{}_{}x{}x{}".format(*s))
def test_wgrad_fl3_g_staging_never_wraps_into_range(shape):
    """General weight-gradient kernel, fl 3: G segment loads at
    gate(off + 2 e gs1, ok) with off = 2 (gd gs2 + gh gs3 + w - 8 + 8 j + (gc0 + cg 8) gs1);
    channels past Gc rely on the range alone."""
    c, d, h, w = shape
    gs3, gs2, gs1 = w, h * w, d * h * w
    rng = 2 * c * gs1
    gcw = 32 if c >= 32 else (c + 7) // 8 * 8
    for gd, gh, gw in itertools.product([-1, 0, d - 1, d], [-1, 0, h - 1, h], [-8, 0, w - 8, w, w + 8]):
        ok = 0 <= gd < d and 0 <= gh < h and 0 <= gw < w
        for gc0 in [0, ((c - 1) // gcw) * gcw]:
            for cg in range(gcw // 8):
                for e in (0, 7):
                    ch = gc0 + 8 * cg + e
                    off = 2 * (gd * gs2 + gh * gs3 + gw + (gc0 + 8 * cg) * gs1) + 2 * e * gs1
                    g = gate(off, ok)
                    if ok and ch < c:
                        assert 0 <= g < rng
                    else:
                        assert g >= rng


@pytest.mark.parametrize("c,w", [(24, 128), (48, 64), (96, 32), (1, 128)])
def test_row_walking_dw_loads_never_wrap_into_range(c, w):
    """Row-walking k=3 weight gradient: x row loads at gate(2 (xd gs2 + xr gs3) +
    2 (ch gs1 + 8 seg), ok), where a channel past C (switched off) contributes
    channel 0, with the x plane and row up to two past the volume on either
    side (the dY row loads have the same form).  Samples just under 1 GiB."""
    h = 61
    d = (GIB - 1) // (2 * c * h * w)
    gs3, gs2, gs1 = w, h * w, d * h * w
    rng = 2 * c * gs1
    assert rng < GIB
    for xd, xr in itertools.product([-2, -1, 0, d - 1, d, d + 1], [-2, -1, 0, h - 1, h, h + 7]):
        ok_pos = 0 <= xd < d and 0 <= xr < h
        for ch in [0, c - 1, c, c + 7]:
            for seg in [0, w // 8 - 1]:
                # A channel past C is switched off and keeps channel 0 in its offset.
                off = 2 * (xd * gs2 + xr * gs3) + 2 * ((ch if ch < c else 0) * gs1 + 8 * seg)
                g = gate(off, ok_pos and ch < c)
                if ok_pos and ch < c:
                    assert 0 <= g < rng and g + 16 <= rng
                else:
                    assert g >= rng


def test_library_rejects_samples_of_1gib_or_more():
    """The bound the replays above rest on, checked in the library itself."""
    import ctypes
    import torch
    from rdna4_conv3d import _native
    lib = _native.load()
    for (c, d, h, w), ok in [((64, 128, 256, 248), True), ((64, 128, 256, 256), False)]:
        x_shape = (1, c, d, h, w)
        y_shape = (1, 8, d, h, w)
        desc = _native.make_desc(x_shape, y_shape, 3, (1, 1, 1), torch.bfloat16,
                                 _native._dense_strides(x_shape, False), _native._dense_strides(y_shape, False))
        got = lib.r3c_conv3d_fwd_workspace(ctypes.byref(desc)) >= 0
        assert got == ok, (c, d, h, w)
