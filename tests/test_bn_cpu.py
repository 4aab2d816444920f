"""BatchNorm3d + ReLU (csrc/r3c_bn.hip) replayed on the CPU in float64 and
checked against PyTorch's batch_norm + relu, its autograd backward and its
running-statistics update.

The replay follows the kernels' structure: chunks of 8192 positions of one
(sample, channel) plane; per chunk, each of 256 threads holds the (count,
mean, M2) of its vectors (VEC elements at t VEC, t VEC + 256 VEC, ...), a
butterfly of Chan et al.'s pairwise combination inside each 64-lane wave, then
the four waves in order; per channel the chunks' partials [n * nchunk + chunk]
combined the same way, the chunk counts recomputed from the chunk index (a
short last chunk); scale / shift, saved mean / invstd and the running-stat
update with the unbiased variance; the backward's chunk sums (sum g,
sum g xhat) under the forward's ReLU mask and the coefficients of
dy = scale g + b y + c.  A dropped term in the combination or in b / c, a wrong
chunk count or a biased running variance fails it.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

CHUNK = 8192
THREADS = 256


def _combine(a, b):
    """Chan et al.: (n, mean, M2) of the union of two disjoint sets."""
    an, am, a2 = a
    bn, bm, b2 = b
    n = an + bn
    safe = np.where(n > 0, n, 1.0)
    d = bm - am
    fb = bn / safe
    out = (n, am + d * fb, a2 + b2 + d * d * an * fb)
    keep_a, keep_b = bn == 0, (an == 0) & (bn != 0)
    return tuple(np.where(keep_a, x, np.where(keep_b, y, z)) for x, y, z in zip(a, b, out))


def _block_combine(m):
    """m: per-thread (n, mean, M2) arrays of 256; butterfly per wave, waves in order."""
    m = tuple(np.asarray(x, dtype=float).copy() for x in m)
    lanes = np.arange(THREADS)
    off = 32
    while off:
        partner = tuple(x[lanes ^ off] for x in m)
        m = _combine(m, partner)
        off >>= 1
    r = tuple(x[0] for x in m)
    for w in range(1, THREADS // 64):
        r = _combine(r, tuple(x[64 * w] for x in m))
    return r


def _thread_of(length, vec):
    return (np.arange(length) // vec) % THREADS


def replay_stats(y, vec):
    """bn_stats_kernel + bn_stats_final_kernel on y [N][C][S]: (mean, biased
    var, count) per channel, through the chunk partials."""
    N, C, S = y.shape
    nchunk = -(-S // CHUNK)
    part = np.zeros((N * nchunk, C, 2))
    for n in range(N):
        for c in range(C):
            for ch in range(nchunk):
                v = y[n, c, ch * CHUNK:min(S, (ch + 1) * CHUNK)]
                t = _thread_of(v.size, vec)
                cnt = np.bincount(t, minlength=THREADS).astype(float)
                s = np.bincount(t, weights=v, minlength=THREADS)
                sq = np.bincount(t, weights=v * v, minlength=THREADS)
                mean = np.where(cnt > 0, s / np.where(cnt > 0, cnt, 1), 0.0)
                m2 = np.where(cnt > 0, np.maximum(sq - s * mean, 0.0), 0.0)
                _, pm, p2 = _block_combine((cnt, mean, m2))
                part[n * nchunk + ch, c] = (pm, p2)
    out = []
    for c in range(C):
        nparts = N * nchunk
        m = (np.zeros(THREADS), np.zeros(THREADS), np.zeros(THREADS))
        m = [list(x) for x in m]
        for tid in range(THREADS):
            acc = (0.0, 0.0, 0.0)
            for i in range(tid, nparts, THREADS):
                ch = i % nchunk
                cnt = float(min(CHUNK, S - ch * CHUNK))
                acc = tuple(float(x) for x in _combine(acc, (cnt, part[i, c, 0], part[i, c, 1])))
            for k in range(3):
                m[k][tid] = acc[k]
        n_, mean, m2 = _block_combine(tuple(np.array(x) for x in m))
        out.append((mean, m2 / n_, n_, m2))
    return out


def replay_bwd_sums(y, dz, scale, shift, mean, invstd, vec):
    """bn_relu_bwd_sums_kernel + bn_relu_bwd_final_kernel: (sum g, sum g xhat) per channel."""
    N, C, S = y.shape
    nchunk = -(-S // CHUNK)
    part = np.zeros((N * nchunk, C, 2))
    for n in range(N):
        for c in range(C):
            for ch in range(nchunk):
                sl = slice(ch * CHUNK, min(S, (ch + 1) * CHUNK))
                yv, dv = y[n, c, sl], dz[n, c, sl]
                g = np.where(yv * scale[c] + shift[c] > 0, dv, 0.0)
                t = _thread_of(yv.size, vec)
                a = np.bincount(t, weights=g, minlength=THREADS)
                b = np.bincount(t, weights=g * (yv - mean[c]) * invstd[c], minlength=THREADS)
                part[n * nchunk + ch, c] = (a.sum(), b.sum())
    return part.sum(axis=0)


@pytest.mark.parametrize("vec", [8, 4])
@pytest.mark.parametrize("N,C,S", [(2, 3, 2 * CHUNK + 40), (1, 2, 1000), (3, 1, CHUNK)])
def test_bn_relu_replay_matches_torch(vec, N, C, S):
    rng = np.random.default_rng(N * 7 + C + S + vec)
    y = rng.standard_normal((N, C, S)) * 2.0 + rng.standard_normal((1, C, 1)) * 3.0
    dz = rng.standard_normal((N, C, S))
    gamma, beta = rng.standard_normal(C), rng.standard_normal(C)
    rm0, rv0 = rng.standard_normal(C), rng.random(C) + 0.5
    eps, momentum = 1e-5, 0.1

    st = replay_stats(y, vec)
    mean = np.array([s[0] for s in st])
    var = np.array([s[1] for s in st])
    cnt = np.array([s[2] for s in st])
    m2 = np.array([s[3] for s in st])
    assert (cnt == N * S).all()
    invstd = 1.0 / np.sqrt(var + eps)
    scale = gamma * invstd
    shift = beta - mean * scale
    unbiased = np.where(cnt > 1, m2 / np.maximum(cnt - 1, 1), var)
    rm = (1 - momentum) * rm0 + momentum * mean
    rv = (1 - momentum) * rv0 + momentum * unbiased
    z = np.maximum(y * scale[None, :, None] + shift[None, :, None], 0.0)

    yt = torch.from_numpy(y).requires_grad_(True)
    gt = torch.from_numpy(gamma).requires_grad_(True)
    bt = torch.from_numpy(beta).requires_grad_(True)
    rmt, rvt = torch.from_numpy(rm0.copy()), torch.from_numpy(rv0.copy())
    zt = F.relu(F.batch_norm(yt, rmt, rvt, gt, bt, training=True, momentum=momentum, eps=eps))
    zt.backward(torch.from_numpy(dz))
    np.testing.assert_allclose(z, zt.detach().numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(rm, rmt.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(rv, rvt.numpy(), rtol=1e-10, atol=1e-12)

    sums = replay_bwd_sums(y, dz, scale, shift, mean, invstd, vec)
    dbeta, dgamma = sums[:, 0], sums[:, 1]
    M = float(N * S)
    b = -scale * invstd * dgamma / M
    c0 = -scale * dbeta / M - b * mean
    g = np.where(y * scale[None, :, None] + shift[None, :, None] > 0, dz, 0.0)
    dy = scale[None, :, None] * g + b[None, :, None] * y + c0[None, :, None]
    np.testing.assert_allclose(dbeta, bt.grad.numpy(), rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(dgamma, gt.grad.numpy(), rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(dy, yt.grad.numpy(), rtol=1e-8, atol=1e-10)


def test_bn_relu_eval_coefficients_match_torch():
    """bn_eval_coef_kernel + the backward with running statistics (b = c = 0)."""
    rng = np.random.default_rng(5)
    N, C, S = 2, 3, 500
    y = rng.standard_normal((N, C, S))
    dz = rng.standard_normal((N, C, S))
    gamma, beta = rng.standard_normal(C), rng.standard_normal(C)
    rm, rv = rng.standard_normal(C), rng.random(C) + 0.5
    eps = 1e-5
    invstd = 1.0 / np.sqrt(rv + eps)
    scale, shift = gamma * invstd, beta - rm * gamma * invstd
    z = np.maximum(y * scale[None, :, None] + shift[None, :, None], 0.0)
    sums = replay_bwd_sums(y, dz, scale, shift, rm, invstd, 8)
    g = np.where(y * scale[None, :, None] + shift[None, :, None] > 0, dz, 0.0)
    dy = scale[None, :, None] * g

    yt = torch.from_numpy(y).requires_grad_(True)
    gt = torch.from_numpy(gamma).requires_grad_(True)
    bt = torch.from_numpy(beta).requires_grad_(True)
    zt = F.relu(F.batch_norm(yt, torch.from_numpy(rm), torch.from_numpy(rv), gt, bt, training=False, eps=eps))
    zt.backward(torch.from_numpy(dz))
    np.testing.assert_allclose(z, zt.detach().numpy(), rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(dy, yt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(sums[:, 0], bt.grad.numpy(), rtol=1e-9, atol=1e-9)
    np.testing.assert_allclose(sums[:, 1], gt.grad.numpy(), rtol=1e-9, atol=1e-9)
