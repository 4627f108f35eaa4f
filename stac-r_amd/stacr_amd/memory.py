"""Analytical byte counts of a STAC-R factor payload (interface of stacr/memory.py:8-82).

A payload is three stored channels: the coefficients (rows x rank), the sparse residual (k flat
indices plus k values, k = round(budget * rows * features)) and, optionally, one basis
(features x rank).  Each value channel is priced by `_channel_bytes`: values kept in the
activation dtype, or packed at 4 / 8 bits with one 4-byte per-tensor scale.  An explicit width
of 0 on the residual means "unquantized values with a unit scale tensor", as the projection
engine saves it.  The function names, argument order, defaults and error messages are the
reference's, so callers and their tests keep working.
"""
from __future__ import annotations

import math

import torch

_SCALE_BYTES = 4
_BIT_WIDTHS = (None, 0, 4, 8)


def dtype_bytes(dtype: torch.dtype) -> int:
    """Bytes of one element of `dtype`."""
    return int(dtype.itemsize)


def _element_count(shape) -> int:
    count = 1
    for dim in shape:
        if isinstance(dim, bool) or int(dim) != dim or dim < 0:
            raise ValueError("Shape dimensions must be nonnegative integers")
        count *= int(dim)
    return count


def dense_bytes(shape: tuple[int, ...], dtype: torch.dtype) -> int:
    """Bytes of a dense tensor of `shape` and `dtype`."""
    return _element_count(shape) * dtype_bytes(dtype)


def _channel_bytes(count: int, bits: int | None, element_bytes: int, scale_bytes: int) -> int:
    """Bytes of `count` stored values: packed to `bits` when that is 4 or 8, otherwise kept at
    `element_bytes`; `scale_bytes` is added when the channel is non-empty."""
    if not count:
        return 0
    body = math.ceil(count * bits / 8) if bits else count * element_bytes
    return body + scale_bytes


def stacr_stored_bytes(shape: tuple[int, ...], rank: int, dtype: torch.dtype = torch.float16,
                       residual_budget: float = 0.005, index_bytes: int = 4, include_basis: bool = False, *,
                       coeff_bits: int | None = None, residual_bits: int | None = None,
                       basis_dtype: torch.dtype | None = None, include_scales: bool = True) -> int:
    """Stored factor bytes for an activation of `shape` (parameters and workspaces excluded).

    Widths left as None keep the activation dtype; 4 / 8 adds a 4-byte per-tensor scale when
    `include_scales`; residual_bits=0 keeps the values unquantized with a unit scale.  The basis
    is counted once, in `basis_dtype` (default: the activation dtype), when `include_basis`.
    """
    total = _element_count(shape)
    if isinstance(rank, bool) or int(rank) != rank or rank < 1:
        raise ValueError("rank must be a positive integer")
    if not math.isfinite(residual_budget) or not 0 <= residual_budget <= 1:
        raise ValueError("residual_budget must be between 0 and 1")
    if index_bytes not in (2, 4, 8):
        raise ValueError("index_bytes must be 2, 4, or 8")
    if coeff_bits not in _BIT_WIDTHS or residual_bits not in _BIT_WIDTHS:
        raise ValueError("Bit widths must be None, 0, 4, or 8")
    elem = dtype_bytes(dtype)
    if not shape:
        return total * elem  # a scalar is stored as it is
    features = int(shape[-1])
    if features == 0:
        return 0
    rows = _element_count(shape[:-1])
    rank = min(int(rank), features)
    coeff_scale = _SCALE_BYTES if include_scales and coeff_bits else 0
    coeff = _channel_bytes(rows * rank, coeff_bits, elem, coeff_scale)
    entries = int(round(float(residual_budget) * rows * features))
    residual_scale = _SCALE_BYTES if include_scales and residual_bits is not None else 0
    residual = entries * index_bytes + _channel_bytes(entries, residual_bits, elem, residual_scale)
    basis = features * rank * dtype_bytes(basis_dtype or dtype) if include_basis else 0
    return int(coeff + residual + basis)


def saved_surface_predictor(saved_bytes: float, baseline_peak_bytes: float) -> float:
    """Replaceable saved-surface bytes (clamped at 0) as a fraction of the baseline peak."""
    if not math.isfinite(baseline_peak_bytes) or baseline_peak_bytes <= 0:
        raise ValueError("baseline_peak_bytes must be finite and positive")
    if not math.isfinite(saved_bytes):
        raise ValueError("saved_bytes must be finite")
    return max(0.0, float(saved_bytes)) / float(baseline_peak_bytes)


__all__ = ["dtype_bytes", "dense_bytes", "stacr_stored_bytes", "saved_surface_predictor"]
