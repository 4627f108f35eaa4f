"""Analytical saved-byte estimate for a STAC-R factor payload (stacr/memory.py:21-73)."""
from __future__ import annotations

import math

import torch


def dtype_bytes(dtype: torch.dtype) -> int:
    return torch.empty((), dtype=dtype).element_size()


def dense_bytes(shape: tuple[int, ...], dtype: torch.dtype) -> int:
    n = 1
    for dim in shape:
        if isinstance(dim, bool) or int(dim) != dim or dim < 0:
            raise ValueError("Shape dimensions must be nonnegative integers")
        n *= int(dim)
    return n * dtype_bytes(dtype)


def stacr_stored_bytes(shape: tuple[int, ...], rank: int, dtype: torch.dtype = torch.float16,
                       residual_budget: float = 0.005, index_bytes: int = 4, include_basis: bool = False, *,
                       coeff_bits: int | None = None, residual_bits: int | None = None,
                       basis_dtype: torch.dtype | None = None, include_scales: bool = True) -> int:
    """Coefficient + residual (+ basis) bytes; unspecified widths keep the activation dtype and an
    explicit 4/8-bit width adds a 4-byte per-tensor scale (residual_bits=0 stores a unit scale)."""
    dense_bytes(shape, dtype)
    if isinstance(rank, bool) or int(rank) != rank or rank < 1:
        raise ValueError("rank must be a positive integer")
    if not math.isfinite(residual_budget) or not 0 <= residual_budget <= 1:
        raise ValueError("residual_budget must be between 0 and 1")
    if index_bytes not in (2, 4, 8):
        raise ValueError("index_bytes must be 2, 4, or 8")
    if coeff_bits not in (None, 0, 4, 8) or residual_bits not in (None, 0, 4, 8):
        raise ValueError("Bit widths must be None, 0, 4, or 8")
    if len(shape) == 0:
        return dense_bytes(shape, dtype)
    feats = int(shape[-1])
    if feats == 0:
        return 0
    rows = math.prod(int(d) for d in shape[:-1])
    rank = min(int(rank), feats)
    vb = dtype_bytes(dtype)
    n_coeff = rows * rank
    coeff = math.ceil(n_coeff * coeff_bits / 8) if coeff_bits else n_coeff * vb
    if include_scales and coeff_bits and n_coeff:
        coeff += 4
    n_res = int(round(float(residual_budget) * rows * feats))
    res_values = math.ceil(n_res * residual_bits / 8) if residual_bits else n_res * vb
    residual = n_res * index_bytes + res_values
    if include_scales and residual_bits is not None and n_res:
        residual += 4
    basis = feats * rank * dtype_bytes(basis_dtype or dtype) if include_basis else 0
    return int(coeff + residual + basis)
