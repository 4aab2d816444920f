"""Index math of the k=1 kernels with at most 4 output channels
(csrc/r3c_skinny.hip: skinny_fwd_kernel, skinny_dx_kernel, skinny_dw_kernel)
replayed on the CPU in float64 and checked against PyTorch's convolution and
its gradients.

Per thread the replay follows the kernel: position group g -> (sample,
first position of its 8), 16-byte vectors at sample / channel strides that
may exceed the dense ones (the host admits channel strides >= the plane and
multiples of 8, csrc/r3c_capi.hip skinny_ok), the LDS weight copy w[o][c],
and for dW the split ranges of position groups, the two groups per thread and
iteration, the channel block of 8 per workgroup row and the partial slots
[s][o][c] (+ db [s][o] from block 0).  Every access is asserted inside its
buffer and 16-byte aligned, every dW position group is taken exactly once
per (split, channel block), and every partial slot is written exactly once.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

MAX_C = 64  # input channels whose weights the LDS copy holds


def _layout(rng, N, C, P, pad_c, pad_n):
    """A [N][C][P] tensor stored with channel stride P + pad_c and sample
    stride C (P + pad_c) + pad_n (pads multiples of 8)."""
    cs = P + pad_c
    ns = C * cs + pad_n
    buf = np.full(N * ns, np.nan)
    vals = rng.standard_normal((N, C, P))
    for n, c in itertools.product(range(N), range(C)):
        buf[n * ns + c * cs:n * ns + c * cs + P] = vals[n, c]
    return buf, vals, ns, cs


def _vec(size, off):
    assert off % 8 == 0 and 0 <= off and off + 8 <= size
    return slice(off, off + 8)


def _groups(N, P):
    return N * (P // 8)


def _group_at(P, g):
    gp = P >> 3
    n = g // gp
    return n, (g - n * gp) * 8


def replay_fwd(xb, xs, w, b, yb, ys, N, C, O, P):
    assert C <= MAX_C and O <= 4
    ws = np.full(4 * MAX_C, np.nan)
    for i in range(O * C):
        ws[i] = w.reshape(-1)[i]
    for g in range(_groups(N, P)):
        n, p = _group_at(P, g)
        acc = np.tile(np.asarray(b if b is not None else np.zeros(O), dtype=float)[:, None], (1, 8))
        for c in range(C):
            v = xb[_vec(xb.size, n * xs[0] + p + c * xs[1])]
            assert not np.isnan(v).any()
            for o in range(O):
                acc[o] += ws[o * C + c] * v
        for o in range(O):
            yb[_vec(yb.size, n * ys[0] + p + o * ys[1])] = acc[o]


def replay_dx(yb, ys, w, xb, xs, N, C, O, P):
    ws = w.reshape(-1)
    for g in range(_groups(N, P)):
        n, p = _group_at(P, g)
        gv = [yb[_vec(yb.size, n * ys[0] + p + o * ys[1])] for o in range(O)]
        for c in range(C):
            v = np.zeros(8)
            for o in range(O):
                v += ws[o * C + c] * gv[o]
            xb[_vec(xb.size, n * xs[0] + p + c * xs[1])] = v


def skinny_nsplit(N, P):
    """plan_skinny_dw: one split per 512 position groups, at most 4096."""
    return max(1, min(4096, -(-_groups(N, P) // 512)))


def replay_dw(xb, xs, yb, ys, N, C, O, P):
    ngroups = _groups(N, P)
    nsplit = skinny_nsplit(N, P)
    part = np.full((nsplit, O, C), np.nan)
    dbpart = np.full((nsplit, O), np.nan)
    hits = np.zeros(part.shape, dtype=np.int64)
    for s, by in itertools.product(range(nsplit), range(-(-C // 8))):
        g0, g1 = s * ngroups // nsplit, (s + 1) * ngroups // nsplit
        cb = 8 * by
        nc = min(8, C - cb)
        taken = np.zeros(ngroups, dtype=np.int64)
        red = np.zeros((256, O * 8 + O))  # per thread: [o * 8 + k] and db [O * 8 + o]
        for tid in range(256):
            g = g0 + tid
            while g < g1:
                for u in range(2):
                    gu = g + 256 * u
                    if gu >= g1:
                        continue
                    taken[gu] += 1
                    n, p = _group_at(P, gu)
                    gv = [yb[_vec(yb.size, n * ys[0] + p + o * ys[1])] for o in range(O)]
                    for o in range(O):
                        red[tid, O * 8 + o] += gv[o].sum()
                    for k in range(nc):
                        v = xb[_vec(xb.size, n * xs[0] + p + (cb + k) * xs[1])]
                        for o in range(O):
                            red[tid, o * 8 + k] += gv[o] @ v
                g += 512
        assert (taken[g0:g1] == 1).all() and taken.sum() == g1 - g0
        tot = red.sum(axis=0)
        for v in range(O * 8 + O):
            if v < O * 8:
                o, k = divmod(v, 8)
                if k < nc:
                    part[s, o, cb + k] = tot[v]
                    hits[s, o, cb + k] += 1
            elif cb == 0:
                dbpart[s, v - O * 8] = tot[v]
    assert (hits == 1).all() and not np.isnan(dbpart).any()
    return part.sum(axis=0), dbpart.sum(axis=0)


CASES = [  # N, C, O, (D, H, W), channel pad, sample pad
    (1, 1, 1, (2, 2, 2), 0, 0),
    (2, 24, 2, (4, 6, 8), 8, 16),
    (1, 40, 3, (8, 16, 33), 0, 8),
    (2, 64, 4, (3, 5, 8), 16, 0),
]


@pytest.mark.parametrize("N,C,O,dhw,pad_c,pad_n", CASES)
def test_skinny_passes_match_torch(N, C, O, dhw, pad_c, pad_n):
    rng = np.random.default_rng(N * 100 + C + O)
    P = int(np.prod(dhw))
    assert P % 8 == 0
    xb, x, xns, xcs = _layout(rng, N, C, P, pad_c, pad_n)
    yb0, dy, yns, ycs = _layout(rng, N, O, P, pad_c, pad_n)
    w = rng.standard_normal((O, C))
    b = rng.standard_normal(O)
    xt = torch.from_numpy(x.reshape(N, C, *dhw))
    dyt = torch.from_numpy(dy.reshape(N, O, *dhw))
    wt = torch.from_numpy(w.reshape(O, C, 1, 1, 1))

    yb = np.full_like(yb0, np.nan)
    replay_fwd(xb, (xns, xcs), w, b, yb, (yns, ycs), N, C, O, P)
    y = np.stack([[yb[n * yns + o * ycs:n * yns + o * ycs + P] for o in range(O)] for n in range(N)])
    ref = F.conv3d(xt, wt, torch.from_numpy(b)).numpy().reshape(N, O, P)
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-10)

    dxb = np.full_like(xb, np.nan)
    replay_dx(yb0, (yns, ycs), w, dxb, (xns, xcs), N, C, O, P)
    dx = np.stack([[dxb[n * xns + c * xcs:n * xns + c * xcs + P] for c in range(C)] for n in range(N)])
    ref_dx = torch.nn.grad.conv3d_input(xt.shape, wt, dyt).numpy().reshape(N, C, P)
    np.testing.assert_allclose(dx, ref_dx, rtol=1e-12, atol=1e-10)

    dw, db = replay_dw(xb, (xns, xcs), yb0, (yns, ycs), N, C, O, P)
    ref_dw = torch.nn.grad.conv3d_weight(xt, wt.shape, dyt).numpy().reshape(O, C)
    np.testing.assert_allclose(dw, ref_dw, rtol=1e-12, atol=1e-10)
    np.testing.assert_allclose(db, dy.sum(axis=(0, 2)), rtol=1e-12, atol=1e-10)


@pytest.mark.parametrize("N,P", [(1, 8), (2, 4096), (1, 8 * 512 * 3 + 8), (4, 64 * 128 * 128)])
def test_skinny_dw_splits_cover_every_group_once(N, P):
    """The split ranges of plan_skinny_dw tile [0, ngroups) without gaps or
    overlap, each split holds at most 512 groups (two per thread of 256), and
    the 4096 cap holds at the bench's full head size."""
    ng = _groups(N, P)
    ns = skinny_nsplit(N, P)
    assert 1 <= ns <= 4096
    bounds = [s * ng // ns for s in range(ns + 1)]
    assert bounds[0] == 0 and bounds[-1] == ng and all(a <= b for a, b in zip(bounds, bounds[1:]))
    if ns < 4096:
        assert max(b - a for a, b in zip(bounds, bounds[1:])) <= 512
