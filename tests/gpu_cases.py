"""Synthetic inputs shaped like the benchmark configurations (shared by GPU tests and bench).

X = Z B^T + 0.05 E with Z ~ N(0,1)^(N x 8), B ~ N(0,1)^(d x 8), E ~ N(0,1); then 0.1% of the
entries scaled x20 (outliers); optionally a per-channel log-normal(sigma=1) scale.  U is the QR
factor of a seeded Gaussian.  Seeds: X 1234, G 1235, U 1236, outlier mask 1237.
"""
from __future__ import annotations

import torch


def make_activation(rows: int, d: int, *, latent: int = 8, lognormal: bool = False, seed: int = 1234,
                    outlier_seed: int = 1237) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(rows, latent, generator=g)
    b = torch.randn(d, latent, generator=g)
    x = z @ b.t() + 0.05 * torch.randn(rows, d, generator=g)
    go = torch.Generator().manual_seed(outlier_seed)
    mask = torch.rand(rows, d, generator=go) < 0.001
    x = torch.where(mask, x * 20.0, x)
    if lognormal:
        x = x * torch.exp(torch.randn(d, generator=g))
    return x


def make_basis(d: int, rank: int, seed: int = 1236) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    q, _ = torch.linalg.qr(torch.randn(d, rank, generator=g))
    return q.contiguous()


def make_grad(rows: int, d_out: int, seed: int = 1235) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, d_out, generator=g)
