"""Saved-tensor compressor: the storage-only path (interface of stacr/compressor.py:13-140 and
stacr/residual.py:8-33).

``stacr_saved_tensors(STACRCompressor(...))`` installs PyTorch saved-tensor hooks.  ``pack``
replaces an eligible saved activation X by its factors: rank-r coefficients C = X Q on a basis
kept per (feature size, device), and the top-k entries of the residual X - rnd(C Q^T) over the
whole tensor; ``unpack`` hands autograd the dense tensor rnd(C Q^T) + residual.

How the pieces are arranged here:
* eligibility is a table of named gates (`_GATES`); `skip_reason` names the first one a tensor
  fails, `should_compress` is "no gate failed";
* the compressor's schedule is a phase computed from the step (`"warmup"`: pass everything
  through, `"turbo"`: coefficients only, `"full"`: coefficients and residual);
* bases live in a `_BasisBank` that creates an `OjaBasis` on first use and steps it on the update
  interval (the step itself is the HIP Oja kernel);
* a pack is one library call: the save kernels project, form the residual and take the exact
  global top-k in the same call (chunk = the whole tensor, values kept in the activation dtype);
  the unpack is the reconstruction kernel (stacr_reconstruct).
Tensors must be ROCm GPU tensors in fp32, bf16 or fp16; anything else raises.

As in the reference this path rebuilds a dense activation in backward; the factor-native layer
(STACRLinear via apply_stacr) is the measured method.
"""
from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from typing import Any, Callable

import torch

from . import kernels
from .oja import OjaBasis


@dataclass
class STACRConfig:
    """Options of the saved-tensor compressor (field names and defaults of stacr/compressor.py:13-25);
    apply_stacr also takes it (a dataclass config is used as given)."""

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
    """Entries kept from a residual of `shape`: flat (row-major) indices and their values
    (stacr/residual.py:8-20)."""

    shape: tuple[int, ...]
    indices: torch.Tensor
    values: torch.Tensor

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= int(s)
        return n

    def dense(self, *, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
        """A zero tensor of `shape` holding the values at their flat indices."""
        flat = torch.zeros(self.numel, device=device, dtype=dtype)
        if self.indices.numel():
            flat.scatter_(0, self.indices.to(device=device, dtype=torch.long), self.values.to(device=device, dtype=dtype))
        return flat.view(self.shape)

    @classmethod
    def empty(cls, shape, device, dtype) -> "SparseResidual":
        return cls(tuple(shape), torch.zeros(0, device=device, dtype=torch.long),
                   torch.zeros(0, device=device, dtype=dtype))


@dataclass
class PackedActivation:
    shape: tuple[int, ...]
    dtype: torch.dtype
    coeff: torch.Tensor
    basis: torch.Tensor
    residual: SparseResidual | None


def _reference_k_budget(numel: int, budget: float) -> float:
    """The budget whose global k under the kernels' rule round(budget n) is the reference's
    max(1, min(n, round(budget n))) (stacr/residual.py:30): only the round-to-zero case differs."""
    budget = float(budget)
    return 1.0 / numel if numel and round(budget * numel) == 0 else budget


def _as_rows(t: torch.Tensor) -> torch.Tensor:
    return t.reshape(1, 1) if t.dim() == 0 else t.reshape(-1, t.shape[-1])


def _global_topk(rows: torch.Tensor, basis: torch.Tensor, budget: float):
    """(coeff, flat indices int64, values) of one save call: the projection on `basis` and the
    exact top-k of the residual over every element (budget 0: coefficients only)."""
    coeff, idx, values, _ = kernels.save(rows, basis, mode="global_topk", budget=budget, chunk_rows=rows.shape[0],
                                         bits=0)
    if idx is None:
        return coeff, None, None
    return coeff, idx.to(torch.long), values


def select_topk_residual(residual: torch.Tensor, budget: float) -> SparseResidual:
    """The largest-magnitude entries of `residual` under a fractional budget, over the whole
    tensor (stacr/residual.py:23-33): the save kernels' global top-k on `residual` against a zero
    basis (so the residual they form is `residual` itself).  Indices ascend; ties at the cut go to
    the lowest index."""
    residual = residual.detach()
    if budget <= 0 or residual.numel() == 0:
        return SparseResidual.empty(residual.shape, residual.device, residual.dtype)
    rows = _as_rows(residual)
    zero_basis = rows.new_zeros(rows.shape[1], 1)
    _, idx, values = _global_topk(rows, zero_basis, _reference_k_budget(residual.numel(), budget))
    return SparseResidual(tuple(residual.shape), idx, values)


# basis_dtype option -> basis dtype; "auto" / "activation" follow the activation, anything else is fp32
_BASIS_DTYPE_NAMES = {"float16": torch.float16, "fp16": torch.float16, "half": torch.float16,
                      "bfloat16": torch.bfloat16, "bf16": torch.bfloat16}
_FOLLOW_ACTIVATION = ("auto", "activation")


def _resolve_basis_dtype(spec: str, activation: torch.dtype) -> torch.dtype:
    key = str(spec).lower()
    if key in _FOLLOW_ACTIVATION:
        return activation
    return _BASIS_DTYPE_NAMES.get(key, torch.float32)


def _is_weight_like(t: torch.Tensor) -> bool:
    """A parameter, a leaf that requires grad, or a view of either (linear autograd saves the
    transposed weight): tensors whose compression would make G W approximate."""
    while t is not None:
        if isinstance(t, torch.nn.Parameter) or (t.is_leaf and t.requires_grad):
            return True
        t = getattr(t, "_base", None)
    return False


# (reason, test that fails the gate): a tensor is compressed only if no gate fails
_GATES: tuple[tuple[str, Callable[[STACRConfig, torch.Tensor], bool]], ...] = (
    ("not floating point", lambda cfg, t: not t.is_floating_point()),
    ("fewer than 2 dimensions", lambda cfg, t: t.dim() < 2),
    ("parameter or a view of one", lambda cfg, t: _is_weight_like(t)),
    ("too few features", lambda cfg, t: int(t.shape[-1]) < int(cfg.min_features)),
    ("too few elements", lambda cfg, t: t.numel() < int(cfg.min_numel)),
)


class _BasisBank:
    """One OjaBasis per (feature size, device), created on first use in the configured dtype."""

    def __init__(self, config: STACRConfig):
        self.config = config
        self.by_key: dict[tuple[int, torch.device], OjaBasis] = {}

    def get(self, x: torch.Tensor) -> OjaBasis:
        key = (int(x.shape[-1]), x.device)
        basis = self.by_key.get(key)
        if basis is None:
            basis = OjaBasis(key[0], self.config.rank, dtype=_resolve_basis_dtype(self.config.basis_dtype, x.dtype),
                             device=x.device)
            self.by_key[key] = basis
        return basis

    def refreshed(self, x: torch.Tensor, rows: torch.Tensor, step: int) -> OjaBasis:
        """The basis for `x`, stepped on `rows` when `step` falls on the update interval."""
        basis = self.get(x)
        if step % max(1, int(self.config.update_interval)) == 0:
            basis.update(rows, lr=float(self.config.oja_lr))
        return basis


class STACRCompressor:
    """Saved-tensor compressor with persistent Oja bases keyed by feature size and device."""

    def __init__(self, config: STACRConfig | None = None):
        self.config = config or STACRConfig()
        self.step = 0
        self._bank = _BasisBank(self.config)

    @property
    def _bases(self) -> dict:
        return self._bank.by_key

    def set_step(self, step: int) -> None:
        self.step = int(step)

    def advance(self) -> None:
        self.set_step(self.step + 1)

    def phase(self) -> str:
        """"warmup" before warmup_steps, "turbo" from turbo_after_step on (or with residual mode
        "none"), else "full"."""
        cfg = self.config
        if self.step < int(cfg.warmup_steps):
            return "warmup"
        turbo = cfg.turbo_after_step is not None and self.step >= int(cfg.turbo_after_step)
        return "turbo" if turbo or cfg.residual_mode == "none" else "full"

    @staticmethod
    def is_parameter(tensor: torch.Tensor) -> bool:
        return _is_weight_like(tensor)

    def skip_reason(self, tensor: torch.Tensor) -> str | None:
        for reason, fails in _GATES:
            if fails(self.config, tensor):
                return reason
        return None

    def should_compress(self, tensor: torch.Tensor) -> bool:
        return self.skip_reason(tensor) is None

    def pack(self, tensor: torch.Tensor) -> Any:
        phase = self.phase()
        if phase == "warmup" or not self.should_compress(tensor):
            return tensor
        x = tensor.detach()
        rows = _as_rows(x)
        basis = self._bank.refreshed(x, rows, self.step).shared(dtype=x.dtype)
        budget = float(self.config.residual_budget) if phase == "full" else 0.0
        coeff, idx, values = _global_topk(rows, basis, _reference_k_budget(x.numel(), budget) if budget > 0 else 0.0)
        if phase != "full":
            residual = None
        elif idx is None:
            residual = SparseResidual.empty(x.shape, x.device, x.dtype)
        else:
            residual = SparseResidual(tuple(x.shape), idx, values)
        return PackedActivation(tuple(x.shape), x.dtype, coeff, basis, residual)

    def unpack(self, packed: Any) -> torch.Tensor:
        if not isinstance(packed, PackedActivation):
            return packed
        entries = None if packed.residual is None else (packed.residual.indices, packed.residual.values)
        dense = kernels.reconstruct(packed.coeff, packed.basis, entries)
        return dense.reshape(packed.shape).to(dtype=packed.dtype)


@contextmanager
def stacr_saved_tensors(compressor: STACRCompressor):
    """Installs `compressor`'s pack / unpack as PyTorch saved-tensor hooks for the block
    (stacr/compressor.py:136-140)."""
    with torch.autograd.graph.saved_tensors_hooks(compressor.pack, compressor.unpack):
        yield compressor


__all__ = ["STACRConfig", "STACRCompressor", "PackedActivation", "SparseResidual", "select_topk_residual",
           "stacr_saved_tensors"]
