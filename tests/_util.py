"""Shared helpers for the parity tests: seeded inputs and tolerances.

Tolerances (max abs error against the fp32 oracle on identical inputs):
attention output 2e-3 for float16 and 1.5e-2 for bfloat16, LSE 1e-3.
"""

import math

import torch

OUT_TOL = {torch.float16: 2e-3, torch.bfloat16: 1.5e-2}
LSE_TOL = 1e-3


def randn(gen, shape, dtype):
    """N(0,1) from a seeded CPU generator, rounded to dtype (CPU tensor)."""
    return torch.randn(*shape, generator=gen).to(dtype)


def outlier_k(k, gen, n_channels=4, factor=8.0):
    """Scale n K channels by `factor` in every head (logit outliers)."""
    ch = torch.randperm(k.shape[-1], generator=gen)[:n_channels]
    k = k.float().clone()
    k[..., ch] *= factor
    return k


def max_err(a, b):
    a = a.float().cpu()
    b = b.float().cpu()
    both_inf = torch.isinf(a) & torch.isinf(b) & (torch.sign(a) == torch.sign(b))
    d = (a - b).abs()
    d[both_inf] = 0
    return d.max().item() if d.numel() else 0.0


def scale_for(d):
    return 1.0 / math.sqrt(d)
