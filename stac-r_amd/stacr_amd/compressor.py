"""Saved-tensor compressor: the storage-only path (interface of stacr/compressor.py:13-140).

``stacr_saved_tensors(STACRCompressor(...))`` installs PyTorch saved-tensor hooks.  ``pack``
replaces an eligible saved activation X (floating point, >= 2 dims, not a parameter or a view of
one, wide and large enough) by its rank-r coefficients C = X Q, the shared basis Q and the
top-k residual entries of X - rnd(C Q^T) over the whole tensor; ``unpack`` hands autograd the
dense tensor rnd(C Q^T) + residual.  Both run in the HIP kernels: the save kernels (projection,
residual and exact global top-k in one call, stacr/compressor.py:108-119 and
stacr/residual.py:23-33) and the reconstruction kernels (stacr/compressor.py:127-133,
stacr/residual.py:13-20).  The basis per (feature size, device) is an OjaBasis whose update is
the HIP Oja step.  Tensors must be ROCm GPU tensors in fp32, bf16 or fp16; anything else raises.

As in the reference this path rebuilds a dense activation in backward; the factor-native layer
(STACRLinear via apply_stacr) is the measured method.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any

import torch

from . import kernels
from .oja import OjaBasis


@dataclass
class STACRConfig:
    """Options of the saved-tensor compressor (stacr/compressor.py:13-25); apply_stacr also takes
    it (a dataclass config is used as given)."""

    rank: int = 8
    residual_budget: float = 0.005
    min_features: int = 128
    min_numel: int = 4096
    oja_lr: float = 0.01
    update_interval: int = 1
    warmup_steps: int = 0
    residual_mode: str = "topk"
    post_warmup_mode: str = "full"
    turbo_after_step: int | None = None
    basis_dtype: str = "float32"


@dataclass
class SparseResidual:
    """Flat indices into a tensor of `shape` and the values kept there (stacr/residual.py:8-20)."""

    shape: tuple[int, ...]
    indices: torch.Tensor
    values: torch.Tensor

    def dense(self, *, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        out = torch.zeros(self.shape, device=device, dtype=dtype)
        if self.indices.numel() > 0:
            out.view(-1)[self.indices.to(device=device, dtype=torch.long)] = self.values.to(device=device,
                                                                                            dtype=dtype)
        return out


@dataclass
class PackedActivation:
    shape: tuple[int, ...]
    dtype: torch.dtype
    coeff: torch.Tensor
    basis: torch.Tensor
    residual: SparseResidual | None


def _topk_budget(numel: int, budget: float) -> float:
    """The budget whose global k is the reference's max(1, min(n, round(budget n)))
    (stacr/residual.py:30); the kernels' global k is round(budget n)."""
    if numel > 0 and round(float(budget) * numel) < 1:
        return 1.0 / numel
    return float(budget)


def _empty_residual(shape, device, dtype) -> SparseResidual:
    return SparseResidual(tuple(shape), torch.empty(0, device=device, dtype=torch.long),
                          torch.empty(0, device=device, dtype=dtype))


def select_topk_residual(residual: torch.Tensor, budget: float) -> SparseResidual:
    """The largest-magnitude entries of `residual` under a fractional budget, over the whole
    tensor (stacr/residual.py:23-33): the global top-k of the save kernels run on `residual`
    with a zero basis.  Indices are ascending; ties at the cut go to the lowest index."""
    residual = residual.detach()
    if budget <= 0 or residual.numel() == 0:
        return _empty_residual(residual.shape, residual.device, residual.dtype)
    x2d = residual.reshape(-1, residual.shape[-1]) if residual.dim() > 0 else residual.reshape(1, 1)
    zero = torch.zeros(x2d.shape[1], 1, device=residual.device, dtype=residual.dtype)
    _, idx, values, _ = kernels.save(x2d, zero, mode="global_topk", budget=_topk_budget(residual.numel(), budget),
                                     chunk_rows=x2d.shape[0], bits=0)
    return SparseResidual(tuple(residual.shape), idx.to(torch.long), values)


def _basis_dtype(name: str, activation_dtype: torch.dtype) -> torch.dtype:
    spec = str(name).lower()
    if spec in ("auto", "activation"):
        return activation_dtype
    if spec in ("float16", "fp16", "half"):
        return torch.float16
    if spec in ("bfloat16", "bf16"):
        return torch.bfloat16
    return torch.float32


class STACRCompressor:
    """Saved-tensor compressor with persistent Oja bases keyed by feature size and device."""

    def __init__(self, config: STACRConfig | None = None):
        self.config = config or STACRConfig()
        self.step = 0
        self._bases: dict[tuple[int, torch.device], OjaBasis] = {}

    def set_step(self, step: int) -> None:
        self.step = int(step)

    def advance(self) -> None:
        self.step += 1

    def _basis_for(self, tensor: torch.Tensor) -> OjaBasis:
        features = int(tensor.shape[-1])
        key = (features, tensor.device)
        if key not in self._bases:
            dtype = _basis_dtype(self.config.basis_dtype, tensor.dtype)
            self._bases[key] = OjaBasis(features, self.config.rank, dtype=dtype, device=tensor.device)
        return self._bases[key]

    @staticmethod
    def is_parameter(tensor: torch.Tensor) -> bool:
        """True for weights and biases (a parameter, a leaf that requires grad, or a view of one:
        linear autograd saves the transposed weight), which are never compressed."""
        if isinstance(tensor, torch.nn.Parameter) or (tensor.requires_grad and tensor.is_leaf):
            return True
        base = getattr(tensor, "_base", None)
        return base is not None and STACRCompressor.is_parameter(base)

    def should_compress(self, tensor: torch.Tensor) -> bool:
        return (tensor.is_floating_point() and tensor.dim() >= 2 and not self.is_parameter(tensor)
                and int(tensor.shape[-1]) >= int(self.config.min_features)
                and tensor.numel() >= int(self.config.min_numel))

    def _effective_residual_mode(self) -> str:
        if self.config.turbo_after_step is not None and self.step >= int(self.config.turbo_after_step):
            return "none"
        return self.config.residual_mode

    def pack(self, tensor: torch.Tensor) -> Any:
        if not self.should_compress(tensor) or self.step < int(self.config.warmup_steps):
            return tensor
        x = tensor.detach()
        x2d = x.reshape(-1, x.shape[-1])
        basis_state = self._basis_for(x)
        if self.step % max(1, int(self.config.update_interval)) == 0:
            basis_state.update(x2d, lr=float(self.config.oja_lr))
        basis = basis_state.shared(dtype=x.dtype)
        residual = None
        if self._effective_residual_mode() != "none":
            budget = float(self.config.residual_budget)
            if budget <= 0:
                coeff = kernels.save(x2d, basis, mode="global_topk", budget=0.0, chunk_rows=x2d.shape[0], bits=0)[0]
                residual = _empty_residual(x.shape, x.device, x.dtype)
            else:
                coeff, idx, values, _ = kernels.save(x2d, basis, mode="global_topk",
                                                     budget=_topk_budget(x.numel(), budget),
                                                     chunk_rows=x2d.shape[0], bits=0)
                residual = SparseResidual(tuple(x.shape), idx.to(torch.long), values)
        else:
            coeff = kernels.save(x2d, basis, mode="global_topk", budget=0.0, chunk_rows=x2d.shape[0], bits=0)[0]
        return PackedActivation(tuple(x.shape), x.dtype, coeff, basis, residual)

    def unpack(self, packed: Any) -> torch.Tensor:
        if not isinstance(packed, PackedActivation):
            return packed
        res = None
        if packed.residual is not None:
            res = (packed.residual.indices, packed.residual.values)
        recon = kernels.reconstruct(packed.coeff, packed.basis, res)
        return recon.reshape(packed.shape).to(dtype=packed.dtype)


@contextmanager
def stacr_saved_tensors(compressor: STACRCompressor):
    """Context manager for PyTorch saved-tensor hooks (stacr/compressor.py:136-140)."""
    with torch.autograd.graph.saved_tensors_hooks(compressor.pack, compressor.unpack):
        yield compressor


__all__ = ["STACRConfig", "STACRCompressor", "PackedActivation", "SparseResidual", "select_topk_residual",
           "stacr_saved_tensors"]
