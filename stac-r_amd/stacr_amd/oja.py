"""Basis orthonormalization (stacr/oja.py:8-11).  QR stays a torch library call."""
from __future__ import annotations

import torch


def orthonormalize(matrix: torch.Tensor) -> torch.Tensor:
    """Orthonormal columns spanning ``matrix`` (reduced QR in fp32, returned in its dtype)."""
    q, _ = torch.linalg.qr(matrix.to(torch.float32), mode="reduced")
    return q.to(matrix.dtype)
