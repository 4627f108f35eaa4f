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
            census = None
            if fused:  # projection, selection and quantization in one stacr_save call
                sel = "global_topk" if mode == "global_topk" else "chunk_topk"
                coeff, idx, data, scale, census = kernels.save_with_census(activation, q, mode=sel, budget=budget,
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
        ctx.save_for_backward(*saved)  # the reference's six (or three) saved tensors
        ctx.has_residual = idx is not None
        # the save's entry census (an intermediate kept on ctx, outside the saved tensors): the
        # backward skips its own count of the entries
        ctx.census = census if idx is not None else None
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
                                                     weight.dtype, census=ctx.census)
            if ctx.needs_input_grad[2]:
                grad_bias = g2d.sum(0).to(ctx.bias_dtype)
        return (grad_input, grad_weight, grad_bias) + (None,) * (ctx.arg_count - 3)


_BASIS_DTYPES = {
    "float32": torch.float32, "fp32": torch.float32,
    "float16": torch.float16, "fp16": torch.float16,
    "bfloat16": torch.bfloat16, "bf16": torch.bfloat16,
}
_FOLLOW_WEIGHT_DTYPE = ("auto", "activation")


def _is_int(value) -> bool:
    return not isinstance(value, bool) and int(value) == value


def _finite(value) -> bool:
    return math.isfinite(value)


# Option checks in the order a caller meets them, with the reference's messages (callers catch the
# ValueError; the first failing check names the option).  Each entry: (options, test, message).
_OPTION_CHECKS = (
    (("rank", "update_interval", "chunk_rows", "residual_block_size"),
     lambda v: _is_int(v) and v >= 1, "{} must be a positive integer"),
    (("residual_budget",), lambda v: _finite(v) and 0 <= v <= 1, "residual_budget must be between 0 and 1"),
    (("residual_bits",), lambda v: v in (0, 4, 8), "residual_bits must be 0, 4, or 8"),
    (("oja_lr",), lambda v: _finite(v) and v >= 0, "oja_lr must be finite and nonnegative"),
    (("warmup_steps", "turbo_after_step"), lambda v: v is None or (_is_int(v) and v >= 0),
     "{} must be a nonnegative integer"),
    (("residual_mode",), lambda v: v in RESIDUAL_MODES, f"residual_mode must be one of {sorted(RESIDUAL_MODES)}"),
    (("residual_sample_ratio",), lambda v: _finite(v) and 0 < v <= 1, "residual_sample_ratio must be in (0, 1]"),
)


def _check_options(options: dict) -> None:
    for names, ok, message in _OPTION_CHECKS:
        for name in names:
            if not ok(options[name]):
                raise ValueError(message.format(name))


def _chunk_sizes(rows: int, chunk_rows: int):
    return (min(chunk_rows, rows - start) for start in range(0, rows, chunk_rows))


class STACRLinear(nn.Module):
    """Linear projection whose saved input is compressed; the parameters are unchanged.

    Call set_step (or stacr_amd.set_step) with the optimizer step before each training forward;
    every call within one step shares that step's basis, checkpoint replay included.  Eval,
    no-grad and frozen-weight calls run the exact native op.  Turbo (step >= turbo_after_step)
    freezes the basis and drops the residual; the weights keep training.

    Basis schedule (stacr/layers.py:323-354): the first training forward fits the basis to its
    batch (SVD of the fp32 rows; a seeded random basis when there are fewer rows than the rank);
    afterwards one Oja step (stacr_oja_step, then QR) per `update_interval` steps, skipped under
    Turbo and, with `freeze_after_warmup`, from `warmup_steps` on.  The basis buffer is rebound,
    never written in place, so a forward still awaiting its backward keeps its version.
    """

    def __init__(self, weight: nn.Parameter, bias: nn.Parameter | None, *, rank: int = 8,
                 residual_budget: float = 0.005, residual_bits: int = 8, oja_lr: float = 0.01,
                 update_interval: int = 1, warmup_steps: int = 0, freeze_after_warmup: bool = False,
                 turbo_after_step: int | None = None, chunk_rows: int = 512, basis_dtype: str = "float32",
                 transposed: bool = False, residual_mode: str = "chunk_topk", residual_block_size: int = 16,
                 residual_sample_ratio: float = 0.1):
        super().__init__()
        if not (isinstance(weight, nn.Parameter) and weight.ndim == 2 and weight.is_floating_point()):
            raise ValueError("weight must be a floating-point 2-D Parameter")
        _check_options(dict(rank=rank, update_interval=update_interval, chunk_rows=chunk_rows,
                            residual_block_size=residual_block_size, residual_budget=residual_budget,
                            residual_bits=residual_bits, oja_lr=oja_lr, warmup_steps=warmup_steps,
                            turbo_after_step=turbo_after_step, residual_mode=residual_mode,
                            residual_sample_ratio=residual_sample_ratio))
        if basis_dtype in _FOLLOW_WEIGHT_DTYPE:
            store_dtype = weight.dtype
        elif basis_dtype in _BASIS_DTYPES:
            store_dtype = _BASIS_DTYPES[basis_dtype]
        else:
            raise ValueError(f"Unknown basis_dtype: {basis_dtype!r}")
        self.transposed = bool(transposed)
        # nn.Linear keeps (out, in); Conv1D keeps (in, out)
        self.out_features, self.in_features = (int(d) for d in (weight.shape[::-1] if transposed else weight.shape))
        if bias is not None and (bias.ndim != 1 or bias.numel() != self.out_features):
            raise ValueError("bias shape must match the output feature count")
        self.weight, self.bias = weight, bias
        self.rank = min(int(rank), self.in_features)
        self.residual_budget = float(residual_budget)
        self.residual_bits = int(residual_bits)
        self.oja_lr = float(oja_lr)
        self.update_interval = int(update_interval)
        self.warmup_steps = int(warmup_steps)
        self.freeze_after_warmup = bool(freeze_after_warmup)
        self.turbo_after_step = turbo_after_step
        self.chunk_rows = int(chunk_rows)
        self.residual_mode = residual_mode
        self.residual_block_size = int(residual_block_size)
        self.residual_sample_ratio = float(residual_sample_ratio)
        on = {"device": weight.device}
        self.register_buffer("basis", torch.zeros(self.in_features, self.rank, dtype=store_dtype, **on))
        self.register_buffer("basis_ready", torch.zeros((), dtype=torch.bool, **on))
        self.register_buffer("_step", torch.zeros((), dtype=torch.int64, **on))
        self.register_buffer("_last_update_step", torch.full((), -1, dtype=torch.int64, **on))

    @classmethod
    def from_linear(cls, module: nn.Module, **options) -> "STACRLinear":
        """Wrap an nn.Linear, or a Transformers Conv1D (weight kept as in x out)."""
        conv1d = type(module).__name__ == "Conv1D"
        if not (conv1d or isinstance(module, nn.Linear)):
            raise TypeError("from_linear requires nn.Linear or Transformers Conv1D")
        layer = cls(module.weight, getattr(module, "bias", None), transposed=conv1d, **options)
        return layer.train(module.training)

    # ---------------------------------------------------------------- step and schedule
    # Host mirrors of the one-element buffers _step, basis_ready and _last_update_step, so a
    # training step does not read them back from the GPU (each read waits for every queued
    # kernel): a mirror holds the value, the tensor and its in-place version counter (host
    # metadata), and is trusted only while both still match, so a write from outside (fill_,
    # load_state_dict's copy_, a move to another device) forces one fresh read.
    def _host_value(self, name: str):
        t = getattr(self, name)
        cached = self.__dict__.get("_host_" + name)
        if cached is not None and cached[1] is t and cached[2] == t._version:
            return cached[0]
        v = t.item()
        self.__dict__["_host_" + name] = (v, t, t._version)
        return v

    def _fill(self, name: str, value) -> None:
        """Sets the buffer `name` (bool or int64) to `value` and its mirror with it."""
        t = getattr(self, name)
        t.fill_(value)
        self.__dict__["_host_" + name] = (bool(value) if t.dtype == torch.bool else int(value), t, t._version)

    @property
    def step(self) -> int:
        return int(self._host_value("_step"))

    @step.setter
    def step(self, value: int) -> None:
        self.set_step(value)

    def set_step(self, step: int) -> None:
        if not _is_int(step) or step < 0:
            raise ValueError("step must be a nonnegative integer")
        self._fill("_step", int(step))

    def _turbo(self) -> bool:
        after = self.turbo_after_step
        return after is not None and self.step >= int(after)

    def _basis_action(self, step: int) -> str | None:
        """What this step's first training forward does to the basis: "fit", "oja" or None."""
        if not bool(self._host_value("basis_ready")):
            return "fit"
        if int(self._host_value("_last_update_step")) == step:
            return None  # already refreshed for this step (micro-batches, recomputation)
        frozen = self.freeze_after_warmup and step >= self.warmup_steps
        if frozen or self._turbo() or step % self.update_interval:
            return None
        return "oja"

    def _install_basis(self, basis: torch.Tensor, step: int) -> None:
        self.basis = basis.to(self.basis.dtype)  # rebind: an outstanding forward keeps its version
        self._fill("basis_ready", True)
        self._fill("_last_update_step", step)

    @torch.no_grad()
    def _refresh_basis(self, x2d: torch.Tensor) -> None:
        if not x2d.numel():
            return
        step = self.step
        action = self._basis_action(step)
        if action is None:
            return
        with torch.autocast(device_type=x2d.device.type, enabled=False):
            if action == "fit":
                rows = x2d.detach().float()
                if rows.shape[0] >= self.rank:
                    start = torch.linalg.svd(rows, full_matrices=False)[2][: self.rank].t().contiguous()
                else:
                    seeded = torch.Generator(device="cpu").manual_seed(0)
                    start = torch.randn(self.in_features, self.rank, generator=seeded).to(rows.device)
                self._install_basis(orthonormalize(start), step)
            else:  # Y = XQ, X^T Y, Y^T Y and the stepped basis in the HIP reduction; QR in torch
                _, stepped = kernels.oja_step(x2d.detach(), self.basis, self.oja_lr)
                self._install_basis(orthonormalize(stepped), step)

    # ---------------------------------------------------------------- forward
    def _native(self, x: torch.Tensor) -> torch.Tensor:
        if not self.transposed:
            return F.linear(x, self.weight, self.bias)
        flat = x.reshape(-1, self.in_features)
        out = torch.addmm(self.bias, flat, self.weight) if self.bias is not None else flat.mm(self.weight)
        return out.reshape(*x.shape[:-1], self.out_features)

    def _compresses(self, x: torch.Tensor) -> bool:
        return self.training and torch.is_grad_enabled() and self.weight.requires_grad and x.numel() > 0

    def _factor_state(self, x: torch.Tensor):
        """(basis, budget) this forward saves with: recorded state when a checkpointed region is
        recomputed, otherwise this step's (possibly refreshed) basis and the Turbo-aware budget."""
        guard = get_global_recomputation_guard()
        if guard.is_recomputing:
            replayed = guard.replay_layer(self)
            if replayed is not None:
                return replayed
            if not bool(self._host_value("basis_ready")):
                self._refresh_basis(x.reshape(-1, self.in_features))
        else:
            self._refresh_basis(x.reshape(-1, self.in_features))
        state = (self.basis, 0.0 if self._turbo() else self.residual_budget)
        guard.record_layer(self, state)
        return state

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.ndim < 1 or x.shape[-1] != self.in_features:
            raise ValueError(f"Expected last input dimension {self.in_features}, got {tuple(x.shape)}")
        if not self._compresses(x):
            return self._native(x)
        basis, budget = self._factor_state(x)
        return STACRFunction.apply(x, self.weight, self.bias, basis, budget, self.residual_bits, self.chunk_rows,
                                   self.transposed, self.residual_mode, self.residual_block_size,
                                   self.residual_sample_ratio)

    # ---------------------------------------------------------------- accounting
    def _saved_entries(self, rows: int, budget: float) -> int:
        """Residual entries one forward of `rows` rows saves, with each selector's rounding
        (stacr/layers.py:25-40, 51-54, 81-88); "sampled" is capped at round(budget * n)."""
        d = self.in_features
        whole = int(round(budget * rows * d))
        if not whole:
            return 0
        block = self.residual_block_size
        if self.residual_mode == "block_sparse" and d % block == 0:
            return sum(max(1, int(round(budget * n * d / block))) * block for n in _chunk_sizes(rows, self.chunk_rows))
        if self.residual_mode in ("chunk_topk", "topk", "block_sparse"):
            per_chunk = sum(max(1, int(round(budget * n * d))) for n in _chunk_sizes(rows, self.chunk_rows))
            return min(whole, per_chunk)
        return whole

    def stored_bytes(self, rows: int, value_bytes: int = 2) -> dict[str, Any]:
        """Saved-factor bytes for one forward of `rows` rows (weights and workspaces excluded).

        `basis` counts the persistent basis plus the cast a forward saves when the value width
        differs from the basis width; "sampled" reports an upper bound on its entries.
        """
        if not _is_int(rows) or rows < 0 or value_bytes not in (2, 4, 8):
            raise ValueError("rows must be a nonnegative integer and value_bytes must be 2, 4, or 8")
        rows = int(rows)
        budget = 0.0 if self._turbo() or self.residual_mode == "none" else self.residual_budget
        entries = self._saved_entries(rows, budget)
        index_bytes = 4 if rows * self.in_features < 2**31 - 1 else 8
        value_store = {4: (entries + 1) // 2, 8: entries}.get(self.residual_bits, entries * value_bytes)
        residual = entries * index_bytes + value_store + (4 if entries else 0)
        coeff = rows * self.rank * value_bytes
        persistent = self.basis.numel() * self.basis.element_size()
        cast = self.basis.numel() * value_bytes if rows and self.basis.element_size() != value_bytes else 0
        return {
            "coeff": coeff,
            "residual": residual,
            "basis": persistent + cast,
            "total": coeff + residual + persistent + cast,
            "persistent_basis": persistent,
            "saved_basis_cast": cast,
            "residual_count": entries,
            "residual_count_is_upper_bound": self.residual_mode == "sampled",
        }


__all__ = ["RESIDUAL_MODES", "STACRFunction", "STACRLinear", "QuantizedValues", "_select_residual"]
