"""Index math of the register-direct ConvTranspose3d(k2, s2) dX
(csrc/r3c_t2dx.h: t2dx_pack_kernel, t2dx_kernel) replayed on the CPU in
float64 and checked against PyTorch's autograd of conv_transpose3d.

The replay follows the kernel: the A fragments packed as [row block][k-step]
[lane] with k = 8 co + tap; per workgroup (row group, column-wave set) and
wave, the column blocks cb_first + i * 8 ncw; the stage schedule (column
block, chunk of KC k-steps) with the next stage's loads issued one stage
ahead into the other register set, the column block handed from the issuing
position (Pi) to the computing one (Pc) after its last chunk; the B fragment
of lane (g, i) at k-step s as four dword loads of dY channel 2 s + g at rows
(kd, kh) under position i's 2 x 2 x 2 block; and the epilogue's stores of
channel 8 q + 4 g + r at position i.  Every live dY load is asserted inside
the sample's range, every dX element (channel < Cin) is written exactly once.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

NUM_CUS = 256


def _mfma32_lanes(c):
    """v_mfma_f32_32x32x16 accumulators: lane (li, g) register v holds C[8 (v // 4) + 4 g + v % 4][li]."""
    out = np.zeros((2, 32, 16))
    for g, v in itertools.product(range(2), range(16)):
        out[g, :, v] = c[8 * (v // 4) + 4 * g + v % 4]
    return out


def plan(N, Cin, Cout, D, H, W):
    """plan_t2dx's grid: (nks, RB, nrg, ncb, ncw)."""
    S = D * H * W
    assert S % 32 == 0
    nks = -(-8 * Cout // 16)
    assert nks <= 64
    nrb = -(-Cin // 32)
    rb = 2 if (nrb >= 2 and 2 * nks <= 64) else 1
    nrg = -(-nrb // rb)
    RB = -(-nrb // nrg)
    ncb = S * N // 32
    ncw = max(1, min(-(-ncb // 8), -(-2 * NUM_CUS // nrg)))
    return nks, RB, nrg, ncb, ncw


def replay_pack(w, nks, nrg, RB):
    """t2dx_pack_kernel: fragment v = (rb nks + ks) 64 + lane -> 8 weights
    A[32 rb + i][16 ks + 8 g + e] = w[ci][k >> 3][k & 7]."""
    Cin, Cout = w.shape[:2]
    wf = w.reshape(Cin, Cout, 8)
    out = np.zeros((nrg * RB * nks * 64, 8))
    for v in range(out.shape[0]):
        lane, rest = v & 63, v >> 6
        ks, rb = rest % nks, rest // nks
        ci = rb * 32 + (lane & 31)
        for e in range(8):
            k = ks * 16 + 8 * (lane >> 5) + e
            if ci < Cin and k < 8 * Cout:
                out[v, e] = wf[ci, k >> 3, k & 7]
    return out


def replay_t2dx(dyb, ys, w, N, Cin, Cout, D, H, W, KC, xs, ncw_force=None):
    """ncw_force: a column-wave count other than the planner's (the kernel
    takes any >= 1; 1 gives each wave several column blocks)."""
    nks, RB, nrg, ncb, ncw = plan(N, Cin, Cout, D, H, W)
    if ncw_force is not None:
        ncw = ncw_force
    S, HW = D * H * W, H * W
    pk = replay_pack(w, nks, nrg, RB)
    extent = (Cout - 1) * ys[1] + (2 * D - 1) * ys[2] + (2 * H - 1) * ys[3] + 2 * W
    dx = np.full(N * xs[0], np.nan)
    hits = np.zeros(dx.size, dtype=np.int64)
    nkc = -(-nks // KC)
    cstride = ncw * 8

    def pos_of(cb):
        p0 = cb * 32
        n = p0 // S
        s = p0 - n * S + np.arange(32)
        d, rem = s // HW, s % HW
        h, ww = rem // W, rem % W
        return n, s, 2 * d * ys[2] + 2 * h * ys[3] + 2 * ww

    def issue(P, kc, live):
        """breg[j][lane][2 q + kw]"""
        n, _, ybase = P
        breg = np.zeros((KC, 64, 8))
        if not live:
            return breg
        for j, g in itertools.product(range(KC), range(2)):
            co = 2 * (kc * KC + j) + g
            if co >= Cout:
                continue
            for q in range(4):
                off = co * ys[1] + ybase + (q >> 1) * ys[2] + (q & 1) * ys[3]
                assert (off % 2 == 0).all() and off.min() >= 0 and (off + 2).max() <= extent
                for kw in range(2):
                    breg[j, 32 * g:32 * g + 32, 2 * q + kw] = dyb[n * ys[0] + off + kw]
        return breg

    for blk in range(nrg * ncw):
        rg, wc = blk % nrg, blk // nrg
        afr = pk[rg * RB * nks * 64:(rg + 1) * RB * nks * 64]
        for wv in range(8):
            cb_first = wc * 8 + wv
            nmy = -(-(ncb - cb_first) // cstride) if cb_first < ncb else 0
            nstage = nmy * nkc
            cb_i, kc_i = cb_first, 0
            Pi = pos_of(cb_i if cb_i < ncb else 0)
            Pc = Pi
            breg = [issue(Pi, 0, nstage > 0), None]

            def adv():
                nonlocal cb_i, kc_i, Pi
                kc_i += 1
                if kc_i == nkc:
                    kc_i = 0
                    cb_i += cstride
                    Pi = pos_of(cb_i if cb_i < ncb else 0)

            adv()
            acc = np.zeros((RB, 32, 32))  # [rb][ci][position]
            for t in range(nstage):
                st = t % 2
                breg[1 - st] = issue(Pi, kc_i, t + 1 < nstage)
                kc = t % nkc
                for j in range(KC):
                    ks = kc * KC + j
                    if ks < nks:
                        bmat = np.concatenate([breg[st][j, :32].T, breg[st][j, 32:].T], axis=0)  # [16 k][position]
                        for rb in range(RB):
                            a = afr[(rb * nks + ks) * 64:(rb * nks + ks) * 64 + 64]
                            amat = np.concatenate([a[:32], a[32:]], axis=1)  # [ci][16 k]
                            acc[rb] += amat @ bmat
                if kc == nkc - 1:
                    n, s, _ = Pc
                    for rb in range(RB):
                        lanes = _mfma32_lanes(acc[rb])
                        for q, r, g in itertools.product(range(4), range(4), range(2)):
                            ci = (rg * RB + rb) * 32 + 8 * q + 4 * g + r
                            if ci < Cin:
                                off = n * xs[0] + ci * xs[1] + s
                                dx[off] = lanes[g, :, 4 * q + r]
                                hits[off] += 1
                        acc[rb] = 0.0
                    Pc = Pi
                adv()
    return dx, hits


@pytest.mark.parametrize("ncw_force", [None, 1])
@pytest.mark.parametrize("KC", [1, 4])
@pytest.mark.parametrize("N,Cin,Cout,dhw,ypad", [
    (1, 8, 3, (2, 4, 4), 0),      # odd Cout: the last k-step's upper half gated
    (2, 40, 24, (2, 2, 8), 2),    # two row blocks in one group, padded dY channel stride
    (1, 72, 16, (4, 4, 8), 0),    # three row blocks: RB 2, two row groups
    (2, 8, 5, (4, 8, 8), 0),      # 16 column blocks: with ncw 1, waves take two each
])
def test_t2dx_replay_matches_conv_transpose3d_input_grad(KC, N, Cin, Cout, dhw, ypad, ncw_force):
    D, H, W = dhw
    S = D * H * W
    rng = np.random.default_rng(Cin + Cout + KC + N)
    w = rng.standard_normal((Cin, Cout, 2, 2, 2))
    dy = rng.standard_normal((N, Cout, 2 * D, 2 * H, 2 * W))
    ys1 = 8 * S + ypad
    ys = (Cout * ys1, ys1, 4 * H * W, 2 * W, 1)
    dyb = np.zeros(N * ys[0])
    for n, c in itertools.product(range(N), range(Cout)):
        dyb[n * ys[0] + c * ys1:n * ys[0] + c * ys1 + 8 * S] = dy[n, c].reshape(-1)
    xs = (Cin * (S + 32), S + 32)  # dense planes, padded channel stride
    dxb, hits = replay_t2dx(dyb, ys, w, N, Cin, Cout, D, H, W, KC, xs, ncw_force)
    dx = np.stack([[dxb[n * xs[0] + c * xs[1]:n * xs[0] + c * xs[1] + S] for c in range(Cin)] for n in range(N)])
    for n, c in itertools.product(range(N), range(Cin)):
        assert (hits[n * xs[0] + c * xs[1]:n * xs[0] + c * xs[1] + S] == 1).all()
    x = torch.zeros((N, Cin, D, H, W), dtype=torch.float64, requires_grad=True)
    F.conv_transpose3d(x, torch.from_numpy(w), stride=2).backward(torch.from_numpy(dy))
    np.testing.assert_allclose(dx.reshape(N, Cin, D, H, W), x.grad.numpy(), rtol=1e-12, atol=1e-10)
