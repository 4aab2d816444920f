"""Index math of the strided kernels that stage source rows through LDS
(csrc/r3c_strided.hip: strided_fwd_rs_kernel with an NDHWC source or an
NCDHW one read in place, strided_dx_rs_kernel), of the direct weight
gradient (strided_dw_kernel) and of the dY scatter of the other dW path
(dilate_kernel), replayed on the CPU with numpy and checked
against PyTorch's float64 convolution and its gradients, with every LDS slot
and every source element the replay touches asserted inside its buffer.

Per wave tile the replay follows the kernel step by step: the per-lane chunk
table (position, 8-channel group) of a row segment, the zero-filled K-padding
slots, the LDS slot of each chunk (pitch 2 NC + 1 slots per position), the
segment position each (block, lane, tap) fragment read uses, and the taps of
one residue class of w for dX (tap_range); the weight operand is the
replayed strided_pack_kernel output, read at the kernels' own fragment
addresses (the forward through the workgroup-shared stage copy s_w, dX from
global memory); with Cout % 8 == 0 the forward's results leave through the
dtile epilogue (accumulator lanes -> the wave's LDS block at pitch
32 NB + 8 -> 16-byte rows of the NDHWC destination), each element read
after it was written.  A plausible slip -- a wrong
segment origin, tap order, residue class or pitch -- changes the result or
trips a bounds assertion.  For dW the replay also follows the x window's
dword picks (v_alignbit / v_perm at 16-bit granularity), the K-block walk of
each split with its carries and zero pipeline padding, the XCD renumbering of
workgroups (a permutation of every (split, tile) pair), the accumulator lane
layout of v_mfma_f32_32x32x16 and the partial write-back, every partial slot
written exactly once.
"""
from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F


def tap_range(dx: bool, q: int, p: int, s: int, k: int = 3):
    """(k0, step, n, c0, dc) as the kernels' tap_range."""
    if not dx:
        return 0, 1, k, q * s - p, 1
    k0 = (q + p) % s
    n = (k - 1 - k0) // s + 1 if k0 < k else 0
    return k0, s, n, (q + p - k0) // s, -1


def run_segment_tile(lds, wslots, src, n, row, s0, seg, segmax, nc, cs, sw_len):
    """One row segment into the wave's LDS block, as issue() + commit(): chunk
    q of the segment is (position q // CG, group q % CG); positions outside
    the row or rows outside the volume load zeros."""
    cg_n = cs // 8
    pps = 2 * nc + 1
    for q in range(seg * cg_n):
        pos, cg = divmod(q, cg_n)
        slot = pos * pps + cg
        assert 0 <= slot < wslots and pos < segmax
        w = s0 + pos
        if row is not None and 0 <= w < sw_len:
            lds[slot] = src[n, row[0], row[1], w, 8 * cg:8 * cg + 8]
        else:
            lds[slot] = 0.0


def run_segment_tile_cf(lds, wslots, src, n, row, iw0, segp, nc, cs, sw_len):
    """The same segment from an NCDHW source read in place (CF): lane item
    (8 aligned positions from a0 = iw0 rounded down to a multiple of 8,
    8-channel group) loads 8 channels x 8 positions and stores position
    a0 + 8 ps + p at segment position a0 + 8 ps + p - iw0 when inside."""
    cg_n = cs // 8
    pps = 2 * nc + 1
    a0 = iw0 - (iw0 % 8)
    ns8 = (iw0 - a0 + segp + 7) // 8
    for it in range(ns8 * cg_n):
        ps, cg = divmod(it, cg_n)
        w8 = a0 + 8 * ps
        loaded = row is not None and 0 <= w8 < sw_len
        if loaded:
            assert w8 + 7 < sw_len
            block = src[n, 8 * cg:8 * cg + 8, row[0], row[1], w8:w8 + 8]  # [channel][position]
        for p in range(8):
            pos = w8 + p - iw0
            if 0 <= pos < segp:
                slot = pos * pps + cg
                assert slot < wslots
                lds[slot] = block[:, p] if loaded else 0.0


def replay_pack(wt, dx):
    """strided_pack_kernel: fragment v = ((c16 taps + t) nbt + nb) 64 + lane
    holds, for lane (li, g), K channels 16 c16 + 8 g + e (e = 0..7) of column
    32 nb + li at tap t, zero past either channel count.  Forward: K = Cin,
    column = Cout; dX: K = Cout, column = Cin (no tap flip).  One column tile
    (the row-segment kernels take at most two 32-column blocks): nbt = the
    32-column blocks."""
    cout, cin, taps = wt.shape[0], wt.shape[1], wt[0, 0].size
    kc, ncol = (cout, cin) if dx else (cin, cout)
    nc16, nbt = -(-kc // 16), -(-ncol // 32)
    wflat = wt.reshape(-1)
    v = np.arange(nc16 * taps * nbt * 64)
    lane, rest = v & 63, v >> 6
    nb, rest = rest % nbt, rest // nbt
    t, c16 = rest % taps, rest // taps
    col, g = nb * 32 + (lane & 31), lane >> 5
    out = np.zeros((v.size, 8))
    for e in range(8):
        kch = c16 * 16 + 8 * g + e
        ok = (col < ncol) & (kch < kc)
        co, ci = (kch, col) if dx else (col, kch)
        idx = (co * cin + ci) * taps + t
        assert (idx[ok] < wflat.size).all()
        out[ok, e] = wflat[idx[ok]]
    return out, nbt


def _weight_matrix(lanes):
    """The K x 32 operand of one 32x32x16 MFMA whose A fragment is the 64
    lanes' weight vectors: lane (li, g) element e is row 8 g + e, column li."""
    return np.concatenate([lanes[:32].T, lanes[32:].T], axis=0)


def _mfma32_lanes(c):
    """Accumulator registers of v_mfma_f32_32x32x16 for a 32 x 32 result C:
    lane (li, g) register v holds C[8 (v // 4) + 4 g + v % 4][li]."""
    out = np.zeros((2, 32, 16) + c.shape[2:])
    for g, v in itertools.product(range(2), range(16)):
        out[g, :, v] = c[8 * (v // 4) + 4 * g + v % 4]
    return out


def replay_fwd(x, wt, stride, pad, mb, sw, channels_first=False):
    """strided_fwd_rs_kernel on float64 x, NDHWC [n, D, H, W, Cs] (CF 0) or
    NCDHW [n, Cs, D, H, W] read in place (CF = Cs / 8); weight OIDHW."""
    if channels_first:
        n_, cs, D, H, W = x.shape
    else:
        n_, D, H, W, cs = x.shape
    co = wt.shape[0]
    nc = (cs + 15) // 16
    sd, sh, _ = stride
    pd, ph, pw = pad
    OD, OH, OW = ((v + 2 * p - 3) // s + 1 for v, p, s in zip((D, H, W), pad, stride))
    segp = (32 * mb - 1) * sw + 3
    pps = 2 * nc + 1
    p_epi = 32 * ((co + 31) // 32) + 8
    wslots = max(segp * pps, 4 * p_epi)
    nwb = -(-OW // (32 * mb))
    pk, nbt = replay_pack(wt, dx=False)
    nbw = nbt
    wfr = 3 * nc * nbw * 64  # weight fragments of one (kd, kh) stage, shared by the workgroup
    y = np.zeros((n_, OD, OH, OW, co))
    for n, od, oh, wb in itertools.product(range(n_), range(OD), range(OH), range(nwb)):
        ow0 = wb * mb * 32
        iw0 = ow0 * sw - pw
        lds = np.zeros((wslots, 8))
        for pos in range(segp):  # K-padding groups stay zero
            for cg in range(cs // 8, 2 * nc):
                lds[pos * pps + cg] = 0.0
        acc = np.zeros((mb, 32, 32 * nbw))
        for st in range(9):
            kd, kh = divmod(st, 3)
            s_w = np.zeros((wfr, 8))  # wissue(st) -> s_w, fragment f = ((kw NC + c) NB + nb) 64 + lane
            for f in range(wfr):
                ln, rest = f & 63, f >> 6
                nb, c, kw = rest % nbw, (rest // nbw) % nc, rest // (nbw * nc)
                src = ((c * 27 + st * 3 + kw) * nbt + nb) * 64 + ln
                assert src < len(pk)
                s_w[f] = pk[src]
            idd, ih = od * sd - pd + kd, oh * sh - ph + kh
            row = (idd, ih) if (0 <= idd < D and 0 <= ih < H) else None
            if channels_first:
                run_segment_tile_cf(lds, wslots, x, n, row, iw0, segp, nc, cs, W)
            else:
                run_segment_tile(lds, wslots, x, n, row, iw0, segp, segp, nc, cs, W)
            for kw, c in itertools.product(range(3), range(nc)):
                t = st * 3 + kw
                for m in range(mb):
                    li = np.arange(32)
                    frag = np.concatenate([lds[((m * 32 + li) * sw + kw) * pps + 2 * c + g] for g in (0, 1)], axis=1)
                    slots = ((m * 32 + li) * sw + kw) * pps + 2 * c + 1
                    assert slots.max() < wslots
                    for nb in range(nbw):
                        f0 = ((kw * nc + c) * nbw + nb) * 64
                        acc[m, :, 32 * nb:32 * nb + 32] += frag @ _weight_matrix(s_w[f0:f0 + 64])
        if co % 8 == 0:  # dtile epilogue (dense NDHWC destination, Cout % 8 == 0)
            pitch = 32 * nbw + 8
            for m in range(mb):
                w0 = ow0 + 32 * m
                if w0 >= OW:
                    break
                tb = np.full(wslots * 8, np.nan)  # the wave's LDS block as halves
                for nb in range(nbw):
                    lanes = _mfma32_lanes(acc[m, :, 32 * nb:32 * nb + 32].T)  # rows = channels, columns = positions
                    for g, q in itertools.product(range(2), range(4)):
                        c0 = nb * 32 + 8 * q + 4 * g
                        for li in range(32):
                            assert (li * pitch + c0) % 4 == 0 and li * pitch + c0 + 4 <= tb.size
                            tb[li * pitch + c0:li * pitch + c0 + 4] = lanes[g, li, 4 * q:4 * q + 4]
                npos, cpp = min(32, OW - w0), co // 8
                for k in range(npos * cpp):
                    pos, c8 = divmod(k, cpp)
                    src = pos * pitch + 8 * c8
                    assert src % 8 == 0 and src + 8 <= tb.size and not np.isnan(tb[src:src + 8]).any()
                    y[n, od, oh, w0 + pos, 8 * c8:8 * c8 + 8] = tb[src:src + 8]
        else:
            for m in range(mb):
                for li in range(32):
                    ow = ow0 + 32 * m + li
                    if ow < OW:
                        y[n, od, oh, ow] = acc[m, li, :co]
    return y


def replay_dx(dy, wt, x_shape, stride, pad, mb, sw):
    """strided_dx_rs_kernel on NDHWC float64 dY [n, OD, OH, OW, Cs = Cout]; weight OIDHW."""
    n_, OD, OH, OW, cs = dy.shape
    _, ci, D, H, W = x_shape
    nc = (cs + 15) // 16
    sd, sh, _ = stride
    pd, ph, pw = pad
    segmax = 32 * mb + 2
    pps = 2 * nc + 1
    p_epi = 32 * ((ci + 31) // 32) + 8
    wslots = max(segmax * pps, 4 * p_epi)
    nwb = -(-(-(-W // sw)) // (32 * mb))
    pk, nbt = replay_pack(wt, dx=True)
    dx = np.zeros((n_, D, H, W, ci))
    for n, rd, rh, res, wb in itertools.product(range(n_), range(D), range(H), range(sw), range(nwb)):
        td = tap_range(True, rd, pd, sd)
        th = tap_range(True, rh, ph, sh)
        tw = tap_range(True, res, pw, sw)
        j0 = wb * mb * 32
        seg = 32 * mb + (tw[2] - 1 if tw[2] > 0 else 0)
        s0 = j0 + tw[3] - (tw[2] - 1 if tw[2] > 0 else 0)
        assert seg <= segmax
        lds = np.zeros((wslots, 8))
        acc = np.zeros((mb, 32, 32 * nbt))
        for md, mh in itertools.product(range(td[2]), range(th[2])):
            cd, ch = td[3] + md * td[4], th[3] + mh * th[4]
            kd, kh = td[0] + md * td[1], th[0] + mh * th[1]
            row = (cd, ch) if (0 <= cd < OD and 0 <= ch < OH) else None
            run_segment_tile(lds, wslots, dy, n, row, s0, seg, segmax, nc, cs, OW)
            for mw in range(tw[2]):
                kw = tw[0] + mw * tw[1]
                t = (kd * 3 + kh) * 3 + kw
                pb = tw[2] - 1 - mw
                for c, m in itertools.product(range(nc), range(mb)):
                    li = np.arange(32)
                    pos = m * 32 + li + pb
                    assert pos.max() < seg
                    frag = np.concatenate([lds[pos * pps + 2 * c + g] for g in (0, 1)], axis=1)
                    for nb in range(nbt):  # wpk[((c taps + t) nbt + nb) 64 + lane], column tile 0
                        f0 = ((c * 27 + t) * nbt + nb) * 64
                        assert f0 + 64 <= len(pk)
                        acc[m, :, 32 * nb:32 * nb + 32] += frag @ _weight_matrix(pk[f0:f0 + 64])
        for m in range(mb):
            for li in range(32):
                w = res + sw * (j0 + 32 * m + li)
                if w < W:
                    dx[n, rd, rh, w] = acc[m, li, :ci]
    return dx


@pytest.mark.parametrize("layout", ["ndhwc", "ncdhw"])
@pytest.mark.parametrize("mb", [1, 2])
@pytest.mark.parametrize("sw", [1, 2])
@pytest.mark.parametrize("cs", [8, 24, 32])
@pytest.mark.parametrize("co", [5, 40])
def test_fwd_row_segments_match_conv3d(mb, sw, cs, layout, co):
    rng = np.random.default_rng(7 * mb + sw + cs + co)
    stride, pad = (2, 1, sw), (1, 0, 1)
    x = rng.standard_normal((1, cs, 4, 4, 72))  # W % 8 == 0 (in-place NCDHW reads whole 8-position runs)
    wt = rng.standard_normal((co, cs, 3, 3, 3))
    ref = F.conv3d(torch.from_numpy(x), torch.from_numpy(wt), None, stride, pad).numpy()
    if layout == "ncdhw":
        y = replay_fwd(x, wt, stride, pad, mb, sw, channels_first=True)
    else:
        y = replay_fwd(x.transpose(0, 2, 3, 4, 1).copy(), wt, stride, pad, mb, sw)
    np.testing.assert_allclose(y.transpose(0, 4, 1, 2, 3), ref, rtol=1e-12, atol=1e-10)


@pytest.mark.parametrize("mb", [1, 2])
@pytest.mark.parametrize("sw", [1, 2])
@pytest.mark.parametrize("cs", [8, 40, 64])
@pytest.mark.parametrize("ci", [6, 40])
def test_dx_row_segments_match_conv3d_input_grad(mb, sw, cs, ci):
    rng = np.random.default_rng(11 * mb + sw + cs + ci)
    stride, pad = (2, 1, sw), (1, 1, 1)
    x_shape = (1, ci, 5, 3, 67)
    wt = rng.standard_normal((cs, ci, 3, 3, 3))
    y_shape = (1, cs) + tuple((v + 2 * p - 3) // s + 1 for v, p, s in zip(x_shape[2:], pad, stride))
    dy = rng.standard_normal(y_shape)
    ref = torch.nn.grad.conv3d_input(x_shape, torch.from_numpy(wt), torch.from_numpy(dy), stride, pad).numpy()
    dx = replay_dx(dy.transpose(0, 2, 3, 4, 1).copy(), wt, x_shape, stride, pad, mb, sw)
    np.testing.assert_allclose(dx.transpose(0, 4, 1, 2, 3), ref, rtol=1e-12, atol=1e-10)


def _alignbit(hi, lo, shift):
    """v_alignbit_b32 on dwords of two 16-bit elements: ({hi, lo} >> shift)[31:0]."""
    assert shift in (0, 16)
    return (lo[0], lo[1]) if shift == 0 else (lo[1], hi[0])


def _perm(hi, lo, sel):
    """v_perm_b32 byte selection on dwords of two 16-bit elements: selector
    bytes 0-3 pick lo's bytes, 4-7 hi's; each result element must take an
    aligned byte pair."""
    halves = (lo[0], lo[1], hi[0], hi[1])
    out = []
    for r in range(2):
        b0, b1 = (sel >> (16 * r)) & 0xFF, (sel >> (16 * r + 8)) & 0xFF
        assert b0 % 2 == 0 and b1 == b0 + 1 and b0 < 8
        out.append(halves[b0 // 2])
    return tuple(out)


def replay_dw(x, dy, stride, pad, nsplit):
    """strided_dw_kernel plus the fixed-order reduce, on float64 NCDHW x and
    dY (contiguous; pad w must be 1, W % 8 == 0, OW % 16 == 0).  Per wave
    (kd, kh) and lane (li, g): the dY fragment (one 16-byte load per lane),
    the x window (edge dword, SW aligned 16-byte loads, edge dword; zero
    outside the row or volume), the alignbit (SW 1) / perm (SW 2) picks per kw,
    the K-block walk with its carries and zero pipeline padding, the
    accumulator -> (co, ci) write-back and the db of wave 0.  Returns
    (dW OIDHW, db)."""
    N, Cin, D, H, W = x.shape
    _, Cout, OD, OH, OW = dy.shape
    sd, sh, sw = stride
    pd, ph, pw = pad
    assert pw == 1 and W % 8 == 0 and OW % 16 == 0
    nw = 6 if sw == 1 else 10
    ncb = 2 if Cout > 32 else 1
    ncg, ngb = -(-Cout // (32 * ncb)), -(-Cin // 32)
    kpr = OW // 16
    nkb = N * OD * OH * kpr
    pf = 3 if ncb == 1 else 2
    ntile = ncg * ngb
    total = nsplit * ntile
    part = np.full((nsplit, Cout, 27, Cin), np.nan)
    dbpart = np.full((nsplit, Cout), np.nan)
    hits = np.zeros(part.shape, dtype=np.int64)
    seen = set()
    for blk in range(total):
        bid = (blk & 7) * (total >> 3) + (blk >> 3) if total % 8 == 0 else blk
        seen.add(bid)
        tile, split = bid % ntile, bid // ntile
        cb, gb = divmod(tile, ngb)
        k0, k1 = split * nkb // nsplit, (split + 1) * nkb // nsplit
        li = np.arange(32)
        ci = gb * 32 + li
        ci_ok = ci < Cin
        co = [(cb * ncb + c) * 32 + li for c in range(ncb)]
        for wv in range(9):
            kd, kh = divmod(wv, 3)
            acc = np.zeros((ncb, 3, 32, 32))  # [nc][kw][row co][col ci]
            dbs = np.zeros((ncb, 2, 32))       # [nc][g][li]
            r = k0
            kn = [r % kpr, (r // kpr) % OH, (r // kpr // OH) % OD, r // kpr // OH // OD]  # owb, oh, od, n

            def advance(kp):
                kp[0] += 1
                if kp[0] < kpr:
                    return
                kp[0] = 0
                kp[1] += 1
                if kp[1] < OH:
                    return
                kp[1] = 0
                kp[2] += 1
                if kp[2] < OD:
                    return
                kp[2] = 0
                kp[3] += 1

            def load(kp, live):
                owb, oh, od, n = kp
                ow0 = owb * 16
                af = np.zeros((ncb, 2, 32, 8))
                win = np.zeros((2, 32, 2 * nw))  # [g][li][window element]
                if not live:
                    return af, win
                assert n < N
                for c in range(ncb):
                    for g in range(2):
                        ok = co[c] < Cout
                        assert ow0 + 8 * g + 8 <= OW
                        af[c, g, ok] = dy[n, co[c][ok], od, oh, ow0 + 8 * g:ow0 + 8 * g + 8]
                idd, ih = od * sd - pd + kd, oh * sh - ph + kh
                if not (0 <= idd < D and 0 <= ih < H):
                    return af, win
                for g in range(2):
                    b = sw * (ow0 + 8 * g)
                    rows = x[n, ci[ci_ok], idd, ih]
                    if b >= 2:
                        win[g, ci_ok, 0:2] = rows[:, b - 2:b]
                    for c in range(sw):
                        if b + 8 * c < W:
                            assert b + 8 * c + 8 <= W
                            win[g, ci_ok, 2 + 8 * c:10 + 8 * c] = rows[:, b + 8 * c:b + 8 * c + 8]
                    if b + 8 * sw < W:
                        assert b + 8 * sw + 2 <= W
                        win[g, ci_ok, 2 * nw - 2:2 * nw] = rows[:, b + 8 * sw:b + 8 * sw + 2]
                return af, win

            def compute(frag):
                af, win = frag
                if wv == 0:
                    dbs[:] += af.sum(axis=3)
                for kw in range(3):
                    o = kw + 1
                    w0, odd = o >> 1, (o & 1) != 0
                    bq = np.zeros((2, 32, 8))
                    for g, l in itertools.product(range(2), range(32)):
                        dw = [tuple(win[g, l, 2 * k:2 * k + 2]) for k in range(nw)]
                        for q in range(4):
                            if sw == 1:
                                lo = dw[q + w0]
                                hi = dw[q + w0 + 1] if q + w0 + 1 < nw else (0.0, 0.0)
                                pair = _alignbit(hi, lo, 16 if odd else 0)
                            else:
                                lo, hi = dw[2 * q + w0], dw[2 * q + w0 + 1]
                                pair = _perm(hi, lo, 0x07060302 if odd else 0x05040100)
                            bq[g, l, 2 * q:2 * q + 2] = pair
                    # MFMA 32x32x16: A[li][8 g + e] = af lane (li, g); B[8 g + e][li] = bq lane (li, g)
                    bmat = np.concatenate([bq[0].T, bq[1].T], axis=0)  # [16][32]
                    for c in range(ncb):
                        amat = np.concatenate([af[c, 0], af[c, 1]], axis=1)  # [32][16]
                        acc[c, kw] += amat @ bmat

            nk = k1 - k0
            loaded = 0
            slots = [None] * pf

            def fetch(u):
                nonlocal loaded
                slots[u] = load(list(kn), loaded < nk)
                loaded += 1
                if loaded < nk:
                    advance(kn)

            for u in range(pf):
                fetch(u)
            for _ in range(0, nk, pf):
                for u in range(pf):
                    compute(slots[u])
                    fetch(u)
            # write-back of each lane's registers at the kernel's (co, ci)
            for c, kw in itertools.product(range(ncb), range(3)):
                lanes = _mfma32_lanes(acc[c, kw])
                t = wv * 3 + kw
                for g, v in itertools.product(range(2), range(16)):
                    cc = (cb * ncb + c) * 32 + 8 * (v >> 2) + 4 * g + (v & 3)
                    if cc < Cout:
                        part[split, cc, t, ci[ci_ok]] = lanes[g, ci_ok, v]
                        hits[split, cc, t, ci[ci_ok]] += 1
            if wv == 0 and gb == 0:
                for c in range(ncb):
                    ok = co[c] < Cout
                    dbpart[split, co[c][ok]] = (dbs[c, 0] + dbs[c, 1])[ok]
    assert seen == set(range(total))
    assert (hits == 1).all() and not np.isnan(dbpart).any()
    dw = part.sum(axis=0).reshape(Cout, 3, 3, 3, Cin).transpose(0, 4, 1, 2, 3)
    return dw, dbpart.sum(axis=0)


@pytest.mark.parametrize("sw", [1, 2])
@pytest.mark.parametrize("cin,cout", [(8, 16), (40, 72)])
@pytest.mark.parametrize("nsplit", [1, 5])
def test_direct_dw_matches_conv3d_weight_grad(sw, cin, cout, nsplit):
    rng = np.random.default_rng(3 * sw + cin + cout + nsplit)
    stride, pad = (2, 1, sw), (1, 0, 1)
    x_shape = (2, cin, 5, 3, 32)
    wt_shape = (cout, cin, 3, 3, 3)
    y_shape = (2, cout) + tuple((v + 2 * p - 3) // s + 1 for v, p, s in zip(x_shape[2:], pad, stride))
    assert y_shape[4] % 16 == 0
    x = rng.standard_normal(x_shape)
    dy = rng.standard_normal(y_shape)
    ref = torch.nn.grad.conv3d_weight(torch.from_numpy(x), wt_shape, torch.from_numpy(dy), stride, pad).numpy()
    dw, db = replay_dw(x, dy, stride, pad, nsplit)
    np.testing.assert_allclose(dw, ref, rtol=1e-12, atol=1e-10)
    np.testing.assert_allclose(db, dy.sum(axis=(0, 2, 3, 4)), rtol=1e-12, atol=1e-10)


def replay_dilate(dy_flat, ys, N, C, D1, H1, W1, W1p, sd, sh, sw):
    """dilate_kernel: thread gi writes elements w0 .. w0 + 7 (one 16-byte
    store) of row (n, c, d1, h1) of the stride-1 grid, pitch W1p; element w1 is
    dY at (d1 / sd, h1 / sh, w1 / sw) when all three divide, else zero."""
    rows = N * C * D1 * H1
    gpr = W1p >> 3
    gi = np.arange(rows * gpr)
    row, w0 = gi // gpr, (gi % gpr) * 8
    h1 = row % H1
    d1 = (row // H1) % D1
    nc = row // H1 // D1
    c, n = nc % C, nc // C
    assert (w0 + 8 <= W1p).all() and W1p % 8 == 0
    dst = np.full(rows * W1p, np.nan)
    for e in range(8):
        w1 = w0 + e
        take = (w1 < W1) & (w1 % sw == 0) & (d1 % sd == 0) & (h1 % sh == 0)
        off = n * ys[0] + c * ys[1] + (d1 // sd) * ys[2] + (h1 // sh) * ys[3] + (w1 // sw) * ys[4]
        assert (off[take] >= 0).all() and (off[take] < dy_flat.size).all()
        val = np.zeros(gi.size)
        val[take] = dy_flat[off[take]]
        dst[row * W1p + w1] = val
    assert not np.isnan(dst).any()
    return dst.reshape(N, C, D1, H1, W1p)


@pytest.mark.parametrize("layout", ["ncdhw", "ndhwc"])
@pytest.mark.parametrize("k,stride,pad", [(3, (2, 2, 2), (1, 1, 1)), (3, (2, 1, 3), (0, 1, 2)), (1, (2, 2, 2), (0, 0, 0)),
                                          (3, (3, 2, 4), (2, 0, 1))])
def test_dilated_dy_gives_the_strided_weight_grad(layout, k, stride, pad):
    """The scatter dW path: dW of the strided convolution equals dW of the
    stride-1 convolution (same input, padding, kernel) over dY scattered by
    dilate_kernel into the stride-1 output grid (rows padded to 8)."""
    rng = np.random.default_rng(sum(stride) * 10 + k + sum(pad))
    N, ci, co = 2, 5, 16
    x_shape = (N, ci, 7, 6, 13)
    y_shape = (N, co) + tuple((v + 2 * p - k) // s + 1 for v, p, s in zip(x_shape[2:], pad, stride))
    x = rng.standard_normal(x_shape)
    dy = rng.standard_normal(y_shape)
    if layout == "ndhwc":
        store = dy.transpose(0, 2, 3, 4, 1).copy()
        _, OD, OH, OW, _ = store.shape
        ys = (OD * OH * OW * co, 1, OH * OW * co, OW * co, co)
    else:
        store = dy
        ys = tuple(s // 8 for s in dy.strides)
    D1, H1, W1 = (v + 2 * p - k + 1 for v, p in zip(x_shape[2:], pad))
    W1p = (W1 + 7) // 8 * 8
    dy1 = replay_dilate(store.reshape(-1), ys, N, co, D1, H1, W1, W1p, *stride)[..., :W1]
    wt_shape = (co, ci, k, k, k)
    ref = torch.nn.grad.conv3d_weight(torch.from_numpy(x), wt_shape, torch.from_numpy(dy), stride, pad).numpy()
    got = torch.nn.grad.conv3d_weight(torch.from_numpy(x), wt_shape, torch.from_numpy(np.ascontiguousarray(dy1)), 1,
                                      pad).numpy()
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-10)
    np.testing.assert_allclose(dy1.sum(axis=(0, 2, 3, 4)), dy.sum(axis=(0, 2, 3, 4)), rtol=1e-12, atol=1e-10)
