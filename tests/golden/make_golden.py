"""Writes tests/golden/conv3d_golden.npz: small input/output vectors for the oracle tests.

The reference ships no golden files; its correctness oracle is live torch
(F.conv3d / torch.nn.grad, tests/test_conv3d.py:38-75 of the reference).  These
vectors are that oracle evaluated in float64 on the CPU, stored so the C oracle
(and anything else) is pinned against fixed numbers.  Inputs are seeded and
rounded to bf16 so they are exactly representable in every dtype under test.

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

OUT = Path(__file__).resolve().parent / "conv3d_golden.npz"


def rnd(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16).double()


def conv_case(name, n, cin, cout, d, h, w, k, pad, out):
    x = rnd((n, cin, d, h, w), 10).requires_grad_(True)
    wt = rnd((cout, cin, k, k, k), 11).requires_grad_(True)
    b = rnd((cout,), 12).requires_grad_(True)
    y = F.conv3d(x, wt, b, 1, pad)
    dy = rnd(tuple(y.shape), 13)
    y.backward(dy)
    for key, v in (("x", x), ("w", wt), ("b", b), ("dy", dy), ("y", y), ("dx", x.grad), ("dw", wt.grad),
                   ("db", b.grad)):
        out[f"{name}.{key}"] = v.detach().numpy().astype(np.float64)
    out[f"{name}.meta"] = np.array([n, cin, cout, d, h, w, k, pad], np.int64)


def convt_case(name, n, cin, cout, d, h, w, out):
    x = rnd((n, cin, d, h, w), 20).requires_grad_(True)
    wt = rnd((cin, cout, 2, 2, 2), 21).requires_grad_(True)
    b = rnd((cout,), 22).requires_grad_(True)
    y = F.conv_transpose3d(x, wt, b, stride=2)
    dy = rnd(tuple(y.shape), 23)
    y.backward(dy)
    for key, v in (("x", x), ("w", wt), ("b", b), ("dy", dy), ("y", y), ("dx", x.grad), ("dw", wt.grad),
                   ("db", b.grad)):
        out[f"{name}.{key}"] = v.detach().numpy().astype(np.float64)
    out[f"{name}.meta"] = np.array([n, cin, cout, d, h, w], np.int64)


def main():
    out = {}
    conv_case("conv_k3p0", 1, 3, 4, 4, 5, 6, 3, 0, out)
    conv_case("conv_k3p1", 2, 3, 4, 4, 5, 6, 3, 1, out)
    conv_case("conv_k3p2", 1, 2, 3, 3, 4, 5, 3, 2, out)
    conv_case("conv_k1p0", 2, 5, 3, 3, 4, 5, 1, 0, out)
    conv_case("conv_k1p1", 1, 4, 2, 2, 3, 4, 1, 1, out)
    convt_case("convt_a", 1, 4, 3, 2, 3, 4, out)
    convt_case("convt_b", 2, 3, 5, 1, 2, 3, out)
    np.savez_compressed(OUT, **out)
    print(OUT, sum(v.nbytes for v in out.values()), "bytes")


if __name__ == "__main__":
    main()
