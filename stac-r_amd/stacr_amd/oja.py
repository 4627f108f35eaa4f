"""Basis orthonormalization and the persistent Oja basis (stacr/oja.py:8-106).

QR and SVD stay torch library calls; the Oja step's reductions (Y = XQ, X^T Y, Y^T Y) run in the
HIP kernel behind stacr_oja_step, so OjaBasis.update needs its basis on a ROCm GPU.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import kernels


def orthonormalize(matrix: torch.Tensor) -> torch.Tensor:
    """Orthonormal columns spanning ``matrix`` (reduced QR in fp32, returned in its dtype)."""
    q, _ = torch.linalg.qr(matrix.to(torch.float32), mode="reduced")
    return q.to(matrix.dtype)


@dataclass
class OjaBasis:
    """Persistent per-feature basis updated from streamed activations (stacr/oja.py:15-106).

    ``update`` rebinds ``basis`` to a new tensor, so a reference handed out by ``shared`` stays
    valid for the activations that used it.
    """

    features: int
    rank: int
    dtype: torch.dtype = torch.float32
    device: torch.device | str = "cpu"
    initialized: bool = False

    def __post_init__(self) -> None:
        self.rank = max(1, min(int(self.rank), int(self.features)))
        self.basis = torch.empty(self.features, self.rank, device=self.device, dtype=self.dtype)
        self._views: dict[torch.dtype, torch.Tensor] = {}
        self.reset_random(seed=0)
        self.initialized = False

    def _invalidate(self) -> None:
        self._views = {}

    def reset_random(self, seed: int = 0) -> None:
        """QR of a seeded CPU normal draw (same draw as the reference for a given seed)."""
        gen = torch.Generator(device="cpu")
        gen.manual_seed(int(seed))
        draw = torch.randn(self.features, self.rank, generator=gen, dtype=torch.float32)
        self.basis = orthonormalize(draw.to(device=self.basis.device, dtype=self.dtype))
        self._invalidate()
        self.initialized = True

    def initialize_from_batch(self, activations: torch.Tensor, centre: bool = False) -> None:
        """Top-``rank`` right singular vectors of the (uncentred by default) batch."""
        x = activations.reshape(-1, activations.shape[-1]).detach().to(torch.float32)
        if centre:
            x = x - x.mean(dim=0, keepdim=True)
        if x.shape[0] < self.rank:
            self.reset_random(seed=0)
            return
        _, _, vh = torch.linalg.svd(x, full_matrices=False)
        self.basis = orthonormalize(vh[: self.rank].t().contiguous()).to(device=self.basis.device, dtype=self.dtype)
        self._invalidate()
        self.initialized = True

    @torch.no_grad()
    def update(self, activations: torch.Tensor, lr: float = 0.01) -> None:
        """One Oja subspace step, then re-orthonormalization (stacr/oja.py:64-81)."""
        if not self.initialized:
            self.initialize_from_batch(activations)
            return
        x = activations.reshape(-1, activations.shape[-1]).detach().to(self.basis.device)
        if x.numel() == 0:
            return
        if x.dtype not in kernels.DTYPE_CODES:
            x = x.to(torch.float32)
        _, stepped = kernels.oja_step(x, self.basis, float(lr))
        self.basis = orthonormalize(stepped).to(dtype=self.dtype)
        self._invalidate()

    def snapshot(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        out = self.basis.detach()
        if dtype is not None:
            out = out.to(dtype=dtype)
        return out.clone()

    def shared(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """Basis of the current version, one tensor per dtype until the next update."""
        target = self.basis.dtype if dtype is None else dtype
        cached = self._views.get(target)
        if cached is None:
            cached = self.basis.detach() if target == self.basis.dtype else self.basis.detach().to(dtype=target)
            self._views[target] = cached
        return cached
