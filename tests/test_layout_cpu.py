"""Index math of the layout copies (csrc/r3c_aux.hip: to_channels_last_kernel,
NCDHW -> NDHWC, and to_channels_first_kernel, its inverse), replayed on the
CPU with numpy on 16-bit patterns.

Per workgroup the replay follows the kernel: the (sample, channel block,
position tile) of the block index, the load items (channel, 8-position group)
or (position, 8-channel group), their LDS addresses in the [channel][position]
tile of pitch 520 halves, and the store items.  It asserts every global and
LDS access inside its buffer, every 16-byte access 16-byte aligned, every LDS
element read after it was written in the same workgroup, every output element
written exactly once, and the result equal to numpy's transpose.  The host
admits C % 8 == 0 and D H W % 8 == 0 (csrc/r3c_capi.hip, ndhwc_copyable).
"""
from __future__ import annotations

import numpy as np
import pytest

TILE_P = 512
PITCH = TILE_P + 8


def _blocks(N, C, S):
    ncb = (C + 31) >> 5
    ntiles = (S + TILE_P - 1) // TILE_P
    for bid in range(ntiles * ncb * N):
        pt, b = bid % ntiles, bid // ntiles
        cb, n = b % ncb, b // ncb
        c0 = cb * 32
        cw = min(32, C - c0)
        p0 = pt * TILE_P
        np_ = min(TILE_P, S - p0)
        assert cw % 8 == 0 and np_ % 8 == 0
        yield n, c0, cw, p0, np_


def _vec(buf, off, size):
    """A 16-byte access of 8 halves at element offset off."""
    assert off % 8 == 0 and 0 <= off and off + 8 <= size
    return slice(off, off + 8)


def replay_to_channels_last(src, N, C, S):
    dst = np.zeros(N * S * C, dtype=np.uint16)
    hits = np.zeros(dst.size, dtype=np.int64)
    for n, c0, cw, p0, np_ in _blocks(N, C, S):
        tile = np.zeros(32 * PITCH, dtype=np.uint16)
        valid = np.zeros(tile.size, dtype=bool)
        base = (n * C + c0) * S + p0
        ngrp = np_ >> 3
        for it in range(cw * ngrp):
            c, j = divmod(it, ngrp)
            tile[_vec(tile, c * PITCH + j * 8, tile.size)] = src[_vec(src, base + c * S + j * 8, src.size)]
            valid[c * PITCH + j * 8:c * PITCH + j * 8 + 8] = True
        cgw = cw >> 3
        dbase = (n * S + p0) * C + c0
        for u in range(np_ * cgw):
            p, cg = divmod(u, cgw)
            idx = cg * 8 * PITCH + p + PITCH * np.arange(8)
            assert idx.max() < tile.size and valid[idx].all()
            sl = _vec(dst, dbase + p * C + cg * 8, dst.size)
            dst[sl] = tile[idx]
            hits[sl] += 1
    assert (hits == 1).all()
    return dst


def replay_to_channels_first(src, N, C, S):
    dst = np.zeros(N * C * S, dtype=np.uint16)
    hits = np.zeros(dst.size, dtype=np.int64)
    for n, c0, cw, p0, np_ in _blocks(N, C, S):
        tile = np.zeros(32 * PITCH, dtype=np.uint16)
        valid = np.zeros(tile.size, dtype=bool)
        base = (n * S + p0) * C + c0
        cgw = cw >> 3
        for u in range(np_ * cgw):
            p, cg = divmod(u, cgw)
            v = src[_vec(src, base + p * C + cg * 8, src.size)]
            idx = cg * 8 * PITCH + p + PITCH * np.arange(8)
            assert idx.max() < tile.size
            tile[idx] = v
            valid[idx] = True
        dbase = (n * C + c0) * S + p0
        ngrp = np_ >> 3
        for it in range(cw * ngrp):
            c, j = divmod(it, ngrp)
            t = _vec(tile, c * PITCH + j * 8, tile.size)
            assert valid[t].all()
            sl = _vec(dst, dbase + c * S + j * 8, dst.size)
            dst[sl] = tile[t]
            hits[sl] += 1
    assert (hits == 1).all()
    return dst


SHAPES = [(1, 8, 8), (2, 24, 512), (2, 32, 520), (1, 40, 1000), (2, 72, 1536), (1, 8, 4096)]


@pytest.mark.parametrize("N,C,S", SHAPES)
def test_to_channels_last_is_the_transpose(N, C, S):
    rng = np.random.default_rng(N * 1000 + C + S)
    x = rng.integers(0, 1 << 16, size=(N, C, S), dtype=np.uint16)
    y = replay_to_channels_last(x.reshape(-1), N, C, S)
    np.testing.assert_array_equal(y.reshape(N, S, C), x.transpose(0, 2, 1))


@pytest.mark.parametrize("N,C,S", SHAPES)
def test_to_channels_first_is_the_transpose(N, C, S):
    rng = np.random.default_rng(N * 1000 + C + S + 1)
    x = rng.integers(0, 1 << 16, size=(N, S, C), dtype=np.uint16)
    y = replay_to_channels_first(x.reshape(-1), N, C, S)
    np.testing.assert_array_equal(y.reshape(N, C, S), x.transpose(0, 2, 1))
    np.testing.assert_array_equal(replay_to_channels_last(y, N, C, S), x.reshape(-1))
