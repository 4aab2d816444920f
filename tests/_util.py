"""Shared helpers for the tests (seeded inputs, error metrics)."""
from __future__ import annotations

import torch


def gen(shape, seed, dtype=torch.float32, relu=False):
    """Seeded N(0,1) on the CPU (identical on every machine), optionally |x| with ~50% zeros."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(*shape, generator=g, dtype=torch.float32)
    if relu:
        t = torch.relu(t)
    return t.to(dtype)


def kaiming_weight(shape, fan_in, seed, dtype=torch.float32):
    """PyTorch's default Conv init bound: U(-1/sqrt(fan_in), 1/sqrt(fan_in))."""
    g = torch.Generator().manual_seed(seed)
    bound = 1.0 / (fan_in ** 0.5)
    return ((torch.rand(*shape, generator=g) * 2 - 1) * bound).to(dtype)


def max_rel(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max|out - ref| / max|ref| (the north-star tolerance metric)."""
    out = out.detach().double().cpu()
    ref = ref.detach().double().cpu()
    den = ref.abs().max().item()
    num = (out - ref).abs().max().item()
    if den == 0.0:
        return num
    return num / den


def to_layout(t: torch.Tensor, layout: str) -> torch.Tensor:
    if layout == "ndhwc":
        return t.contiguous(memory_format=torch.channels_last_3d)
    return t.contiguous()
