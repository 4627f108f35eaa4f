"""Orthonormalization and the persistent Oja basis (interface of stacr/oja.py:8-106).

The Oja step's reductions (Y = XQ, X^T Y, Y^T Y and the stepped basis) run in the HIP kernels
behind stacr_oja_step, so `OjaBasis.update` needs its basis on a ROCm GPU; the QR after it runs in
the QR kernels (stacr_qr, stacr_qr_tall) up to 16 columns, torch's QR beyond.  SVD stays a torch call.

The basis is versioned: every change installs a new tensor (never an in-place write) and bumps
the version, so a tensor handed out by `shared` stays valid for the activations that used it,
and the per-dtype casts `shared` hands out are cached for one version only.
"""
from __future__ import annotations

import torch

from . import kernels


def orthonormalize(matrix: torch.Tensor) -> torch.Tensor:
    """Orthonormal columns spanning ``matrix``: reduced QR in fp32 (LAPACK's Householder signs),
    returned in its dtype.  On a ROCm GPU the QR kernels (stacr_qr, or stacr_qr_tall past 8192
    elements) for up to 16 columns; otherwise torch's QR."""
    m = matrix.to(torch.float32)
    if m.is_cuda and m.dim() == 2 and m.shape[1] <= m.shape[0]:
        try:
            q, _ = kernels.qr(m)
            return q.to(matrix.dtype)
        except NotImplementedError:
            pass
    q, _ = torch.linalg.qr(m, mode="reduced")
    return q.to(matrix.dtype)


def _seeded_orthonormal(features: int, rank: int, seed: int) -> torch.Tensor:
    """QR of an fp32 normal draw from a CPU generator seeded with `seed` (reproducible anywhere)."""
    draw = torch.randn(features, rank, generator=torch.Generator(device="cpu").manual_seed(int(seed)),
                       dtype=torch.float32)
    return orthonormalize(draw)


def _top_right_singular_vectors(x: torch.Tensor, rank: int) -> torch.Tensor:
    """features x rank: the leading right singular vectors of the fp32 rows of `x`."""
    _, _, vh = torch.linalg.svd(x, full_matrices=False)
    return vh[:rank].t().contiguous()


class OjaBasis:
    """A features x rank orthonormal basis tracked from streamed activations.

    Starts as a seeded random orthonormal basis and uninitialized: the first `update` fits it to
    that batch (SVD), later ones take one Oja step and re-orthonormalize.
    """

    def __init__(self, features: int, rank: int, dtype: torch.dtype = torch.float32,
                 device: torch.device | str = "cpu", initialized: bool = False):
        self.features = int(features)
        self.rank = max(1, min(int(rank), self.features))
        self.dtype = dtype
        self.device = device
        self.version = 0
        self._casts: dict[torch.dtype, torch.Tensor] = {}
        self.reset_random(seed=0)
        self.initialized = False  # a fresh basis is always fitted by its first update

    def _install(self, basis: torch.Tensor) -> None:
        self.basis = basis.to(device=self.device, dtype=self.dtype)
        self.version += 1
        self._casts = {}

    def reset_random(self, seed: int = 0) -> None:
        """Seeded random orthonormal basis (QR of a CPU fp32 normal draw); marks it initialized."""
        self._install(_seeded_orthonormal(self.features, self.rank, seed))
        self.initialized = True

    def initialize_from_batch(self, activations: torch.Tensor, centre: bool = False) -> None:
        """Fit the leading right singular vectors of the batch (uncentred unless `centre`): the
        reconstruction C Q^T adds no mean back, so the mean direction belongs in the basis.  A
        batch with fewer rows than the rank falls back to the seed-0 random basis."""
        x = activations.reshape(-1, activations.shape[-1]).detach().to(torch.float32)
        if centre:
            x = x - x.mean(dim=0, keepdim=True)
        if x.shape[0] < self.rank:
            self.reset_random(seed=0)
            return
        self._install(orthonormalize(_top_right_singular_vectors(x, self.rank)))
        self.initialized = True

    @torch.no_grad()
    def update(self, activations: torch.Tensor, lr: float = 0.01) -> None:
        """Fit on the first call, then one Oja step Q + lr (X^T Y / n - Q Y^T Y / n), Y = X Q, in fp32
        on the GPU, followed by re-orthonormalization."""
        if not self.initialized:
            self.initialize_from_batch(activations)
            return
        rows = activations.reshape(-1, activations.shape[-1]).detach()
        if rows.numel() == 0:
            return
        rows = rows.to(self.basis.device)
        if rows.dtype not in kernels.DTYPE_CODES:
            rows = rows.to(torch.float32)
        _, stepped = kernels.oja_step(rows, self.basis, float(lr))
        self._install(orthonormalize(stepped))

    def snapshot(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """A private copy of the current basis (in `dtype` if given)."""
        return self.basis.detach().to(dtype=dtype or self.basis.dtype).clone()

    def shared(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """The current version's basis in `dtype`, one tensor per dtype until the next change, so
        many saved activations can reference it without a copy each."""
        want = dtype or self.basis.dtype
        if want not in self._casts:
            self._casts[want] = self.basis.detach() if want == self.basis.dtype else self.basis.detach().to(want)
        return self._casts[want]


__all__ = ["orthonormalize", "OjaBasis"]
