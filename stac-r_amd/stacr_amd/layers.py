"""Drop-in STACRLinear / STACRFunction whose save and weight gradient run in HIP kernels.

Same public surface and observable contract as stacr/layers.py:
  * STACRFunction.apply(x, weight, bias, basis, budget, residual_bits, chunk_rows, transposed,
    residual_mode="chunk_topk", residual_block_size=16, residual_sample_ratio=0.1)
    (stacr/layers.py:112-126); saved tensors [coeff, weight, q] + [idx, data, scale]
    (:149-152); ctx.has_residual, residual_bits, residual_len (:153-155).
  * forward output and grad_input are the native dense ops (:129-132, :168-171); grad_bias is
    g.sum(0) in G's dtype (:197-198), so all three stay bit-equal to nn.Linear / Conv1D.
  * coeff, residual selection and quantization come from one stacr_save call; grad_weight from
    stacr_weight_grad.  Indices are saved in ascending flat order (the reference leaves the
    order of torch.topk(sorted=False) unspecified; readers only use them as a set).
  * STACRLinear(weight, bias, **options), from_linear, set_step, step, stored_bytes with the
    reference's validation and schedule (stacr/layers.py:202-473).
  * Selectors "uniform", "block_sparse" and "sampled" run as their own HIP kernels on the
    save's coefficients (stacr_select_uniform / stacr_select_block_sparse / stacr_select_threshold),
    and their values are quantized with quantize_values as in the reference (:146).
"""
from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn
from torch.nn import functional as F

from . import kernels
from .adaptive_checkpointing import get_global_recomputation_guard
from .oja import orthonormalize
from .quant import QuantizedValues, quantize_values

RESIDUAL_MODES = {"chunk_topk", "topk", "global_topk", "uniform", "none", "block_sparse", "sampled"}
TOPK_SELECTORS = {"chunk_topk", "topk", "global_topk"}


def _check_selector(mode: str) -> None:
    if mode not in RESIDUAL_MODES:
        raise ValueError(f"Unknown residual_mode: {mode!r}")


def _select_residual(x, coeff, basis, budget, chunk_rows, mode, block_size=16, sample_ratio=0.1):
    """(flat indices, values in x's dtype) of the selected residual, or (None, None)
    (stacr/layers.py:44-101), on a given projection ``coeff``.  Indices ascend."""
    _check_selector(mode)
    if mode == "none" or budget <= 0 or x.numel() == 0:
        return None, None
    q = basis.to(x.dtype)
    coeff = coeff.to(x.dtype)
    rows, features = x.shape
    if mode in TOPK_SELECTORS or (mode == "block_sparse" and features % block_size):
        sel = "global_topk" if mode == "global_topk" else "chunk_topk"
        _, idx, data, _ = kernels.save(x, q, mode=sel, budget=float(budget), chunk_rows=int(chunk_rows), bits=0,
                                       coeff=coeff)
        return idx, data
    k_total = int(round(budget * x.numel()))
    if k_total == 0:
        return None, None
    if mode == "uniform":
        return kernels.select_uniform(x, coeff, q, k_total)
    if mode == "block_sparse":
        return kernels.select_block_sparse(x, coeff, q, float(budget), int(chunk_rows), int(block_size))
    return kernels.select_sampled(x, coeff, q, float(budget), float(sample_ratio), k_total)


class STACRFunction(torch.autograd.Function):
    """Exact linear forward and input gradient; weight gradient from the saved factors.

    grad_W = (G^T C) Q^T + G^T R_sparse.  The saved basis is the version passed in; a later
    forward rebinds the layer's basis instead of mutating it.
    """

    @staticmethod
    def forward(ctx, x, weight, bias, basis, budget, residual_bits, chunk_rows, transposed,
                residual_mode="chunk_topk", residual_block_size=16, residual_sample_ratio=0.1):
        d_in = basis.shape[0]
        x2d = x.reshape(-1, d_in)
        if transposed:
            out2d = x2d.mm(weight) if bias is None else torch.addmm(bias, x2d, weight)
        else:
            out2d = F.linear(x2d, weight, bias)
        budget = float(budget)
        mode = residual_mode
        _check_selector(mode)
        bits = int(residual_bits)
        if mode == "none":
            mode, budget = "chunk_topk", 0.0
        with torch.autocast(device_type=x.device.type, enabled=False):
            activation, q = x2d.to(out2d.dtype), basis.to(out2d.dtype)
            fused = mode in TOPK_SELECTORS or (mode == "block_sparse" and d_in % int(residual_block_size))
            if fused:  # projection, selection and quantization in one stacr_save call
                sel = "global_topk" if mode == "global_topk" else "chunk_topk"
                coeff, idx, data, scale = kernels.save(activation, q, mode=sel, budget=budget,
                                                       chunk_rows=int(chunk_rows), bits=bits)
                length = int(idx.numel()) if idx is not None else 0
            else:  # projection, then the selector's kernels, then quantize_values
                coeff, _, _, _ = kernels.save(activation, q, mode="chunk_topk", budget=0.0,
                                              chunk_rows=int(chunk_rows), bits=0)
                idx, val = _select_residual(activation, coeff, q, budget, int(chunk_rows), mode,
                                            int(residual_block_size), float(residual_sample_ratio))
                data = scale = None
                if idx is not None:
                    packed = quantize_values(val, bits)
                    data, scale, bits, length = packed.data, packed.scale, packed.bits, packed.length
        saved = [coeff, weight, q]
        if idx is not None:
            saved += [idx, data, scale]
        ctx.save_for_backward(*saved)
        ctx.has_residual = idx is not None
        ctx.residual_bits = bits if idx is not None else 0
        ctx.residual_len = length if idx is not None else 0
        ctx.leading, ctx.in_features = x.shape[:-1], d_in
        ctx.out_features, ctx.transposed = out2d.shape[1], bool(transposed)
        ctx.input_dtype = x.dtype
        ctx.bias_dtype = None if bias is None else bias.dtype
        ctx.arg_count = len(ctx.needs_input_grad)
        return out2d.reshape(*ctx.leading, ctx.out_features)

    @staticmethod
    def backward(ctx, grad_out):
        coeff, weight, q, *residual = ctx.saved_tensors
        g2d = grad_out.reshape(-1, ctx.out_features)
        grad_input = grad_weight = grad_bias = None
        with torch.autocast(device_type=g2d.device.type, enabled=False):
            if ctx.needs_input_grad[0]:
                w = weight.to(g2d.dtype)
                grad_input = g2d.mm(w.t() if ctx.transposed else w)
                grad_input = grad_input.reshape(*ctx.leading, ctx.in_features).to(ctx.input_dtype)
            if ctx.needs_input_grad[1]:
                res = tuple(residual) if ctx.has_residual and residual[0].numel() else None
                grad_weight, _ = kernels.weight_grad(g2d, coeff, q, res, ctx.residual_bits, ctx.transposed,
                                                     weight.dtype)
            if ctx.needs_input_grad[2]:
                grad_bias = g2d.sum(0).to(ctx.bias_dtype)
        return (grad_input, grad_weight, grad_bias) + (None,) * (ctx.arg_count - 3)


_BASIS_DTYPES = {
    "float32": torch.float32, "fp32": torch.float32,
    "float16": torch.float16, "fp16": torch.float16,
    "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
}


def _positive_int(name: str, value) -> None:
    if isinstance(value, bool) or int(value) != value or value < 1:
        raise ValueError(f"{name} must be a positive integer")


def _optional_nonneg_int(name: str, value) -> None:
    if value is not None and (isinstance(value, bool) or int(value) != value or value < 0):
        raise ValueError(f"{name} must be a nonnegative integer")


class STACRLinear(nn.Module):
    """Linear projection whose saved input is compressed; parameters are unchanged.

    Call set_step (or stacr_amd.set_step) with the optimizer step before each training forward.
    Eval, no-grad and frozen-weight calls use the exact native op.  Turbo (step >=
    turbo_after_step) freezes the basis and drops the residual; the weights keep training.
    """

    def __init__(self, weight: nn.Parameter, bias: nn.Parameter | None, *, rank: int = 8,
                 residual_budget: float = 0.005, residual_bits: int = 8, oja_lr: float = 0.01,
                 update_interval: int = 1, warmup_steps: int = 0, freeze_after_warmup: bool = False,
                 turbo_after_step: int | None = None, chunk_rows: int = 512, basis_dtype: str = "float32",
                 transposed: bool = False, residual_mode: str = "chunk_topk", residual_block_size: int = 16,
                 residual_sample_ratio: float = 0.1):
        super().__init__()
        # validation order and messages follow stacr/layers.py:232-270
        if not isinstance(weight, nn.Parameter) or weight.ndim != 2 or not weight.is_floating_point():
            raise ValueError("weight must be a floating-point 2-D Parameter")
        for name, value in (("rank", rank), ("update_interval", update_interval), ("chunk_rows", chunk_rows),
                            ("residual_block_size", residual_block_size)):
            _positive_int(name, value)
        if not math.isfinite(residual_budget) or not 0 <= residual_budget <= 1:
            raise ValueError("residual_budget must be between 0 and 1")
        if residual_bits not in (0, 4, 8):
            raise ValueError("residual_bits must be 0, 4, or 8")
        if not math.isfinite(oja_lr) or oja_lr < 0:
            raise ValueError("oja_lr must be finite and nonnegative")
        _optional_nonneg_int("warmup_steps", warmup_steps)
        _optional_nonneg_int("turbo_after_step", turbo_after_step)
        if residual_mode not in RESIDUAL_MODES:
            raise ValueError(f"residual_mode must be one of {sorted(RESIDUAL_MODES)}")
        if not math.isfinite(residual_sample_ratio) or not 0 < residual_sample_ratio <= 1:
            raise ValueError("residual_sample_ratio must be in (0, 1]")
        if basis_dtype in ("auto", "activation"):
            basis_torch_dtype = weight.dtype
        elif basis_dtype in _BASIS_DTYPES:
            basis_torch_dtype = _BASIS_DTYPES[basis_dtype]
        else:
            raise ValueError(f"Unknown basis_dtype: {basis_dtype!r}")
        self.weight, self.bias = weight, bias
        self.transposed = bool(transposed)
        self.in_features = int(weight.shape[0] if transposed else weight.shape[1])
        self.out_features = int(weight.shape[1] if transposed else weight.shape[0])
        if bias is not None and (bias.ndim != 1 or bias.numel() != self.out_features):
            raise ValueError("bias shape must match the output feature count")
        self.rank = min(int(rank), self.in_features)
        self.residual_budget, self.residual_bits = float(residual_budget), int(residual_bits)
        self.oja_lr, self.update_interval = float(oja_lr), int(update_interval)
        self.warmup_steps, self.freeze_after_warmup = int(warmup_steps), bool(freeze_after_warmup)
        self.turbo_after_step, self.chunk_rows = turbo_after_step, int(chunk_rows)
        self.residual_mode, self.residual_block_size = residual_mode, int(residual_block_size)
        self.residual_sample_ratio = float(residual_sample_ratio)
        dev = weight.device
        self.register_buffer("basis", torch.zeros(self.in_features, self.rank, dtype=basis_torch_dtype, device=dev))
        self.register_buffer("basis_ready", torch.zeros((), dtype=torch.bool, device=dev))
        self.register_buffer("_step", torch.zeros((), dtype=torch.int64, device=dev))
        self.register_buffer("_last_update_step", torch.full((), -1, dtype=torch.int64, device=dev))

    @classmethod
    def from_linear(cls, module: nn.Module, **options) -> "STACRLinear":
        """Wrap an nn.Linear or a Transformers Conv1D (weight stored in x out)."""
        transposed = type(module).__name__ == "Conv1D"
        if not transposed and not isinstance(module, nn.Linear):
            raise TypeError("from_linear requires nn.Linear or Transformers Conv1D")
        layer = cls(module.weight, getattr(module, "bias", None), transposed=transposed, **options)
        layer.train(module.training)
        return layer

    @property
    def step(self) -> int:
        return int(self._step.item())

    @step.setter
    def step(self, value: int) -> None:
        self.set_step(value)

    def set_step(self, step: int) -> None:
        if isinstance(step, bool) or int(step) != step or step < 0:
            raise ValueError("step must be a nonnegative integer")
        self._step.fill_(int(step))

    def _turbo(self) -> bool:
        return self.turbo_after_step is not None and self.step >= int(self.turbo_after_step)

    @torch.no_grad()
    def _refresh_basis(self, x2d: torch.Tensor) -> None:
        """SVD init on the first batch, then one Oja step per update interval
        (stacr/layers.py:323-354).  The basis tensor is rebound, never mutated in place.
        The Oja step's reductions run in stacr_oja_step; SVD and QR stay library calls."""
        if not x2d.numel():
            return
        step = self.step
        ready = bool(self.basis_ready)
        if ready and int(self._last_update_step.item()) == step:
            return
        target = self.basis.dtype
        with torch.autocast(device_type=x2d.device.type, enabled=False):
            if not ready:
                sample = x2d.detach().float()
                if sample.shape[0] >= self.rank:
                    _, _, vh = torch.linalg.svd(sample, full_matrices=False)
                    init = vh[: self.rank].t().contiguous()
                else:
                    gen = torch.Generator(device="cpu").manual_seed(0)
                    init = torch.randn(self.in_features, self.rank, generator=gen).to(sample.device)
                self.basis = orthonormalize(init).to(target)
                self.basis_ready.fill_(True)
                self._last_update_step.fill_(step)
                return
            if self.freeze_after_warmup and step >= self.warmup_steps:
                return
            if self._turbo() or step % self.update_interval:
                return
            # Y = XQ, X^T Y and Y^T Y in the HIP reduction (X read once more in its own dtype)
            _, stepped = kernels.oja_step(x2d.detach(), self.basis, self.oja_lr)
            self.basis = orthonormalize(stepped).to(target)
            self._last_update_step.fill_(step)

    def _native(self, x: torch.Tensor) -> torch.Tensor:
        if self.transposed:
            flat = x.reshape(-1, self.in_features)
            out = flat.mm(self.weight) if self.bias is None else torch.addmm(self.bias, flat, self.weight)
            return out.reshape(*x.shape[:-1], self.out_features)
        return F.linear(x, self.weight, self.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.ndim < 1 or x.shape[-1] != self.in_features:
            raise ValueError(f"Expected last input dimension {self.in_features}, got {tuple(x.shape)}")
        if not self.training or not torch.is_grad_enabled() or not self.weight.requires_grad or x.numel() == 0:
            return self._native(x)
        guard = get_global_recomputation_guard()
        replay = guard.replay_layer(self) if guard.is_recomputing else None
        if replay is not None:
            basis, budget = replay
        else:
            if not guard.is_recomputing or not bool(self.basis_ready):
                self._refresh_basis(x.reshape(-1, self.in_features))
            basis = self.basis
            budget = 0.0 if self._turbo() else self.residual_budget
            guard.record_layer(self, (basis, budget))
        return STACRFunction.apply(x, self.weight, self.bias, basis, budget, self.residual_bits, self.chunk_rows,
                                   self.transposed, self.residual_mode, self.residual_block_size,
                                   self.residual_sample_ratio)

    def stored_bytes(self, rows: int, value_bytes: int = 2) -> dict[str, Any]:
        """Saved-factor bytes for one forward of ``rows`` rows (stacr/layers.py:402-473).

        Counts follow the selectors' rounding; "sampled" reports an upper bound.  ``basis``
        includes the persistent basis and the saved cast when value and basis widths differ.
        """
        if isinstance(rows, bool) or int(rows) != rows or rows < 0 or value_bytes not in (2, 4, 8):
            raise ValueError("rows must be a nonnegative integer and value_bytes must be 2, 4, or 8")
        rows = int(rows)
        d = self.in_features
        budget = 0.0 if self._turbo() or self.residual_mode == "none" else self.residual_budget
        count = int(round(budget * rows * d))
        starts = range(0, rows, self.chunk_rows)
        if self.residual_mode == "block_sparse" and d % self.residual_block_size == 0 and count:
            count = sum(
                max(1, int(round(budget * min(self.chunk_rows, rows - s) * d / self.residual_block_size)))
                * self.residual_block_size
                for s in starts
            )
        elif self.residual_mode in ("chunk_topk", "topk", "block_sparse") and count:
            count = min(count, sum(max(1, int(round(budget * min(self.chunk_rows, rows - s) * d))) for s in starts))
        index_bytes = 4 if rows * d < 2**31 - 1 else 8
        if self.residual_bits == 4:
            value_store = (count + 1) // 2
        elif self.residual_bits == 8:
            value_store = count
        else:
            value_store = count * value_bytes
        residual = count * index_bytes + value_store + (4 if count else 0)
        coeff = rows * self.rank * value_bytes
        persistent = self.basis.numel() * self.basis.element_size()
        cast = self.basis.numel() * value_bytes if self.basis.element_size() != value_bytes and rows else 0
        basis = persistent + cast
        return {
            "coeff": coeff,
            "residual": residual,
            "basis": basis,
            "total": coeff + residual + basis,
            "persistent_basis": persistent,
            "saved_basis_cast": cast,
            "residual_count": count,
            "residual_count_is_upper_bound": self.residual_mode == "sampled",
        }


__all__ = ["RESIDUAL_MODES", "STACRFunction", "STACRLinear", "QuantizedValues", "_select_residual"]
