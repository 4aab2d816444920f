"""Index math of MaxPool3d(2) (csrc/r3c_pool.hip: maxpool2_fwd_kernel,
maxpool2_bwd_kernel) replayed on the CPU in float64 and checked against
PyTorch's CPU max_pool3d and its backward.

Per thread the replay follows the kernel: thread t -> (n, c, od, oh, ow0)
with 4 outputs along w, the four (kd, kh) input rows of 8 elements at sample
/ channel strides (dense planes; the host admits strides that are multiples
of the vector width, csrc/r3c_capi.hip pool_setup), the running maximum in
(kd, kh, kw) order where a greater value or a NaN replaces it, the one-byte
index kd * 4 + kh * 2 + kw packed 4 to a dword, and in the backward the
gradient routed by that index plus the optional second gradient.  Every access
is asserted inside its buffer and aligned to its vector, and every output and
every input-gradient element is written exactly once.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def _vec(size, off, n):
    assert off % n == 0 and 0 <= off and off + n <= size
    return slice(off, off + n)


def _store(vals, cs, ns):
    N, C = vals.shape[:2]
    plane = vals[0, 0].size
    buf = np.full(N * ns, np.nan)
    for n, c in itertools.product(range(N), range(C)):
        buf[n * ns + c * cs:n * ns + c * cs + plane] = vals[n, c].reshape(-1)
    return buf


def _threads(N, C, od, oh, ow):
    ow4 = ow >> 2
    for t in range(N * C * od * oh * ow4):
        ow0 = (t % ow4) * 4
        r = t // ow4
        yield r // oh // od // C, (r // oh // od) % C, (r // oh) % od, r % oh, ow0


def replay_fwd(xb, xs, ys, N, C, D, H, W, ysize):
    od, oh, ow = D // 2, H // 2, W // 2
    yb = np.full(ysize, np.nan)
    idx = np.full(N * C * od * oh * ow, -1, dtype=np.int64)
    yhits = np.zeros(ysize, dtype=np.int64)
    for n, c, d, h, w0 in _threads(N, C, od, oh, ow):
        base = n * xs[0] + c * xs[1] + 2 * d * H * W + 2 * h * W + 2 * w0
        m, k = [-np.inf] * 4, [0] * 4
        for r in range(4):
            v = xb[_vec(xb.size, base + (r >> 1) * H * W + (r & 1) * W, 8)]
            for j, kw in itertools.product(range(4), range(2)):
                val = v[2 * j + kw]
                if val > m[j] or np.isnan(val):
                    m[j], k[j] = val, r * 2 + kw
        yo = n * ys[0] + c * ys[1] + (d * oh + h) * ow + w0
        yb[_vec(ysize, yo, 4)] = m
        yhits[yo:yo + 4] += 1
        io = (((n * C + c) * od + d) * oh + h) * ow + w0
        assert io % 4 == 0 and io + 4 <= idx.size
        idx[io:io + 4] = k
    return yb, idx, yhits


def replay_bwd(dyb, ys, idx, xs, N, C, D, H, W, xsize, add=None, as_=None):
    od, oh, ow = D // 2, H // 2, W // 2
    dxb = np.full(xsize, np.nan)
    hits = np.zeros(xsize, dtype=np.int64)
    for n, c, d, h, w0 in _threads(N, C, od, oh, ow):
        g = dyb[_vec(dyb.size, n * ys[0] + c * ys[1] + (d * oh + h) * ow + w0, 4)]
        io = (((n * C + c) * od + d) * oh + h) * ow + w0
        kk = idx[io:io + 4]
        base = n * xs[0] + c * xs[1] + 2 * d * H * W + 2 * h * W + 2 * w0
        for r in range(4):
            v = np.array([g[j] if kk[j] == r * 2 + kw else 0.0 for j in range(4) for kw in range(2)])
            o = base + (r >> 1) * H * W + (r & 1) * W
            if add is not None:
                ao = n * as_[0] + c * as_[1] + (o - (n * xs[0] + c * xs[1]))
                v = v + add[_vec(add.size, ao, 8)]
            dxb[_vec(xsize, o, 8)] = v
            hits[o:o + 8] += 1
    return dxb, hits


CASES = [  # N, C, (D, H, W), x channel pad, x sample pad, y channel pad
    (1, 1, (2, 2, 8), 0, 0, 0),
    (2, 3, (4, 6, 16), 8, 16, 4),
    (1, 5, (6, 2, 24), 0, 8, 8),
]


@pytest.mark.parametrize("N,C,dhw,xpc,xpn,ypc", CASES)
@pytest.mark.parametrize("with_add", [False, True])
def test_maxpool2_replay_matches_torch(N, C, dhw, xpc, xpn, ypc, with_add):
    D, H, W = dhw
    rng = np.random.default_rng(N * 31 + C + D + with_add)
    # small integers: ties inside windows; plus NaN and -inf windows
    x = rng.integers(-3, 4, size=(N, C, D, H, W)).astype(np.float64)
    x[0, 0, 0, 0, 0] = np.nan
    x[0, 0, 0:2, 0:2, 2:4] = -np.inf
    xcs, ycs = D * H * W + xpc, (D // 2) * (H // 2) * (W // 2) + ypc
    xns, yns = C * xcs + xpn, C * ycs
    xb = _store(x, xcs, xns)
    ysize = N * yns
    yb, idx, yhits = replay_fwd(xb, (xns, xcs), (yns, ycs), N, C, D, H, W, ysize)
    od, oh, ow = D // 2, H // 2, W // 2
    y = np.stack([[yb[n * yns + c * ycs:n * yns + c * ycs + od * oh * ow] for c in range(C)] for n in range(N)])
    ref, ref_i = F.max_pool3d(torch.from_numpy(x), 2, return_indices=True)
    np.testing.assert_array_equal(y.reshape(ref.shape), ref.numpy())
    for n, c in itertools.product(range(N), range(C)):
        assert (yhits[n * yns + c * ycs:n * yns + c * ycs + od * oh * ow] == 1).all()
    # one-byte index -> PyTorch's flat index in the (d, h, w) plane
    k = idx.reshape(N, C, od, oh, ow)
    dd, hh, ww = np.meshgrid(np.arange(od), np.arange(oh), np.arange(ow), indexing="ij")
    flat = ((2 * dd + (k >> 2)) * H + 2 * hh + ((k >> 1) & 1)) * W + 2 * ww + (k & 1)
    np.testing.assert_array_equal(flat, ref_i.numpy())

    dy = rng.standard_normal((N, C, od, oh, ow))
    dyb = _store(dy, ycs, yns)
    add = as_ = None
    addv = np.zeros_like(x)
    if with_add:
        addv = rng.standard_normal(x.shape)
        acs, ans = D * H * W + 8, C * (D * H * W + 8) + 8
        add, as_ = _store(addv, acs, ans), (ans, acs)
    dxb, hits = replay_bwd(dyb, (yns, ycs), idx, (xns, xcs), N, C, D, H, W, xb.size, add, as_)
    dx = np.stack([[dxb[n * xns + c * xcs:n * xns + c * xcs + D * H * W] for c in range(C)] for n in range(N)])
    # max_pool3d's backward adds dy at its indices (checked equal to the replay's above)
    ref_dx = torch.zeros(x.shape, dtype=torch.float64).reshape(N, C, -1)
    ref_dx.scatter_add_(2, ref_i.reshape(N, C, -1), torch.from_numpy(dy).reshape(N, C, -1))
    np.testing.assert_array_equal(dx.reshape(x.shape), ref_dx.reshape(x.shape).numpy() + addv)
    for n, c in itertools.product(range(N), range(C)):
        assert (hits[n * xns + c * xcs:n * xns + c * xcs + D * H * W] == 1).all()
