"""Adaptive-engine save / weight-gradient path on the HIP kernels.

Mirrors the STAC-R branch of the reference's adaptive engine (stacr/adaptive.py) and its helpers:
  * quantize_int8 / dequantize_int8 / quantize_int4 / dequantize_int4 (:44-135): per-tensor, the
    scale computed and kept in the tensor's own dtype, with the reference's fp32 / fp64 redo when
    that scale underflows to zero;
  * _choose_index_dtype (:138-159), compress_indices / decompress_indices with the CSR and delta
    formats (stacr/index_compression.py:118-345);
  * STACRFunction's "topk" save (:1333-1572) with coefficient and residual quantization and index
    compression (:1962-2052), and its STAC-R backward (:2256-2470); the low-rank-only route
    (STACRLowRankOnlyFunction, :2551-2686) is residual_mode "none".
Every arithmetic step runs in libstacr_amd.so.  Stable sorting of unsorted index lists (only
needed when a caller hands compress_indices an unsorted list; the HIP save emits ascending
indices) uses torch's sort.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import Enum
from typing import Optional, Union

import torch

from . import _lib
from .kernels import _ptr, _stream, dtype_code, require_gpu

_SCALE_DTYPES = {_lib.DTYPE_F32: torch.float32, _lib.DTYPE_BF16: torch.bfloat16, _lib.DTYPE_F16: torch.float16,
                 _lib.SCALE_F64: torch.float64}
_SCALE_CODES = {v: k for k, v in _SCALE_DTYPES.items()}


# ---------------------------------------------------------------- scale records
def _scale_record_to_tensor(rec: torch.Tensor) -> torch.Tensor:
    """The reference's scale tensor, shape (1,), in the dtype the record names (reads 4 bytes back)."""
    code = int(rec.view(torch.int32)[2].item())
    return rec.view(torch.float64)[:1].to(_SCALE_DTYPES[code])


def _tensor_to_scale_record(scale: torch.Tensor) -> torch.Tensor:
    rec = torch.zeros(16, dtype=torch.uint8, device=scale.device)
    rec.view(torch.float64)[0] = scale.reshape(-1)[0].to(torch.float64)
    rec.view(torch.int32)[2] = _SCALE_CODES[scale.dtype]
    return rec


def _quantize_record(values: torch.Tensor, bits: int):
    require_gpu(values, "values")
    flat = values.reshape(-1).contiguous()
    n = flat.numel()
    device = flat.device
    data = torch.empty(n if bits == 8 else (n + 1) // 2, dtype=torch.int8 if bits == 8 else torch.uint8, device=device)
    rec = torch.empty(16, dtype=torch.uint8, device=device)
    ws = torch.empty(4, dtype=torch.uint8, device=device)
    L = _lib.load()
    _lib.check(L.stacr_adaptive_quantize(_ptr(flat), dtype_code(flat.dtype), n, int(bits), _ptr(data), _ptr(rec),
                                         _ptr(ws), 4, _stream(device)), "stacr_adaptive_quantize")
    return data, rec


def _dequantize_record(data: torch.Tensor, rec: torch.Tensor, bits: int, n: int, out_dtype: torch.dtype):
    out = torch.empty(n, dtype=out_dtype, device=data.device)
    L = _lib.load()
    _lib.check(L.stacr_adaptive_dequantize(_ptr(data), int(bits), _ptr(rec), int(n), _ptr(out), dtype_code(out_dtype),
                                           _stream(data.device)), "stacr_adaptive_dequantize")
    return out


# ---------------------------------------------------------------- public quantizers
def quantize_int8(tensor: torch.Tensor):
    """(int8 tensor of tensor's shape, scale (1,)) as stacr/adaptive.py:44-76."""
    if tensor.numel() == 0:
        return tensor.to(torch.int8), torch.ones(1, device=tensor.device, dtype=tensor.dtype)
    data, rec = _quantize_record(tensor, 8)
    return data.reshape(tensor.shape), _scale_record_to_tensor(rec)


def dequantize_int8(quantized: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """quantized.to(scale.dtype) * scale (stacr/adaptive.py:79-90)."""
    if quantized.numel() == 0 or scale.dtype == torch.float64:
        return quantized.to(scale.dtype) * scale
    rec = _tensor_to_scale_record(scale)
    out = _dequantize_record(quantized.reshape(-1).contiguous(), rec, 8, quantized.numel(), scale.dtype)
    return out.reshape(quantized.shape)


def quantize_int4(tensor: torch.Tensor):
    """(packed uint8, scale (1,), orig_len) as stacr/adaptive.py:93-120."""
    orig_len = tensor.numel()
    if orig_len == 0:
        return tensor.to(torch.uint8), torch.ones(1, device=tensor.device, dtype=tensor.dtype), 0
    data, rec = _quantize_record(tensor, 4)
    return data, _scale_record_to_tensor(rec), orig_len


def dequantize_int4(packed: torch.Tensor, scale: torch.Tensor, orig_len: int) -> torch.Tensor:
    """(nibble - 8).to(scale.dtype) * scale for the first orig_len entries (stacr/adaptive.py:123-131)."""
    if orig_len == 0:
        return packed.to(scale.dtype)
    if scale.dtype == torch.float64:
        low, high = packed & 0x0F, (packed >> 4) & 0x0F
        q = torch.stack([low, high], dim=1).reshape(-1)[:orig_len].to(torch.int8) - 8
        return q.to(scale.dtype) * scale
    rec = _tensor_to_scale_record(scale)
    return _dequantize_record(packed.contiguous(), rec, 4, orig_len, scale.dtype)


# ---------------------------------------------------------------- index dtypes and codecs
def _choose_index_dtype(total_elements: int) -> torch.dtype:
    """int16 below 32768 elements, int32 up to 2^31, else int64 (stacr/adaptive.py:138-159)."""
    if total_elements < 32768:
        return torch.int16
    if total_elements <= 2**31:
        return torch.int32
    return torch.int64


def _choose_col_dtype(n: int) -> torch.dtype:
    """stacr/index_compression.py:118-130."""
    if n < 32768:
        return torch.int16
    if n <= 2**31:
        return torch.int32
    return torch.int64


class IndexCompressionMode(Enum):
    NONE = "none"
    CSR = "csr"
    DELTA = "delta"


@dataclass
class CompressedIndices:
    """Same fields as stacr/index_compression.py:57-83."""

    mode: IndexCompressionMode
    row_ptrs: Optional[torch.Tensor] = None
    col_indices: Optional[torch.Tensor] = None
    delta_base: Optional[torch.Tensor] = None
    sort_indices: Optional[torch.Tensor] = None
    nnz: int = 0
    B_flat: int = 0
    N: int = 0
    original_dtype: torch.dtype = torch.int32

    def memory_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in (self.row_ptrs, self.col_indices, self.delta_base,
                                                          self.sort_indices) if t is not None)


def _csr_encode(sorted_idx: torch.Tensor, b_flat: int, n: int):
    nnz = sorted_idx.numel()
    device = sorted_idx.device
    ptr = torch.empty(b_flat + 1, dtype=torch.int32 if nnz < 2**31 else torch.int64, device=device)
    cols = torch.empty(nnz, dtype=_choose_col_dtype(n), device=device)
    L = _lib.load()
    _lib.check(L.stacr_csr_encode(_ptr(sorted_idx), sorted_idx.element_size(), nnz, int(b_flat), int(n), _ptr(ptr),
                                  ptr.element_size(), _ptr(cols), cols.element_size(), _stream(device)),
               "stacr_csr_encode")
    return ptr, cols


def _delta_encode(sorted_idx: torch.Tensor, b_flat: int, n: int):
    nnz = sorted_idx.numel()
    device = sorted_idx.device
    L = _lib.load()
    base = torch.empty(1, dtype=torch.int32 if b_flat * n <= 2**31 else torch.int64, device=device)
    if nnz > 1:
        mx = torch.empty(1, dtype=torch.int64, device=device)
        _lib.check(L.stacr_delta_max(_ptr(sorted_idx), sorted_idx.element_size(), nnz, _ptr(mx), _stream(device)),
                   "stacr_delta_max")
        max_delta = int(mx.item())  # the width choice is a host decision, as in the reference
        ddt = torch.int16 if max_delta <= 32767 else (torch.int32 if max_delta < 2**31 else torch.int64)
        deltas = torch.empty(nnz - 1, dtype=ddt, device=device)
    else:
        deltas = torch.empty(0, dtype=torch.int16, device=device)
    _lib.check(L.stacr_delta_encode(_ptr(sorted_idx), sorted_idx.element_size(), nnz, _ptr(base), base.element_size(),
                                    _ptr(deltas), deltas.element_size() if deltas.numel() else 2, _stream(device)),
               "stacr_delta_encode")
    return base, deltas


def compress_indices(flat_indices: torch.Tensor, B_flat: int, N: int, mode: Union[str, IndexCompressionMode] = "csr",
                     preserve_order: bool = True) -> CompressedIndices:
    """stacr/index_compression.py:133-269 with the HIP encoders."""
    if isinstance(mode, str):
        mode = IndexCompressionMode(mode)
    require_gpu(flat_indices, "indices")
    device = flat_indices.device
    original_dtype = flat_indices.dtype
    nnz = flat_indices.numel()
    if nnz == 0:
        return CompressedIndices(
            mode=mode,
            row_ptrs=torch.zeros(B_flat + 1, dtype=torch.int32, device=device) if mode == IndexCompressionMode.CSR
            else None,
            col_indices=torch.tensor([], dtype=_choose_col_dtype(N), device=device),
            nnz=0, B_flat=B_flat, N=N, original_dtype=original_dtype)
    if mode == IndexCompressionMode.NONE:
        return CompressedIndices(mode=mode, col_indices=flat_indices, nnz=nnz, B_flat=B_flat, N=N,
                                 original_dtype=original_dtype)
    flat = flat_indices.reshape(-1)
    if mode == IndexCompressionMode.CSR:
        sort_idx = torch.argsort(torch.div(flat.long(), N, rounding_mode="floor"), stable=True)
        ptr, cols = _csr_encode(flat[sort_idx].contiguous(), B_flat, N)
        unsort = torch.argsort(sort_idx) if preserve_order else None
        return CompressedIndices(mode=mode, row_ptrs=ptr, col_indices=cols, sort_indices=unsort, nnz=nnz,
                                 B_flat=B_flat, N=N, original_dtype=original_dtype)
    if mode == IndexCompressionMode.DELTA:
        sorted_indices, sort_idx = torch.sort(flat)
        base, deltas = _delta_encode(sorted_indices.contiguous(), B_flat, N)
        unsort = torch.argsort(sort_idx) if preserve_order else None
        return CompressedIndices(mode=mode, col_indices=deltas, delta_base=base, sort_indices=unsort, nnz=nnz,
                                 B_flat=B_flat, N=N, original_dtype=original_dtype)
    raise ValueError(f"Unknown compression mode: {mode}")


def decompress_indices(compressed: CompressedIndices, restore_order: bool = True) -> torch.Tensor:
    """stacr/index_compression.py:272-345 with the HIP decoders."""
    mode = compressed.mode
    if compressed.col_indices is not None:
        device = compressed.col_indices.device
    elif compressed.delta_base is not None:
        device = compressed.delta_base.device
    else:
        device = torch.device("cpu")
    if compressed.nnz == 0:
        return torch.tensor([], dtype=compressed.original_dtype, device=device)
    if mode == IndexCompressionMode.NONE:
        return compressed.col_indices.to(compressed.original_dtype)
    out = torch.empty(compressed.nnz, dtype=compressed.original_dtype, device=device)
    L = _lib.load()
    if mode == IndexCompressionMode.CSR:
        ptr, cols = compressed.row_ptrs, compressed.col_indices
        if cols.numel() != compressed.nnz:
            raise ValueError(f"CSR col_indices has {cols.numel()} elements but nnz={compressed.nnz}")
        _lib.check(L.stacr_csr_decode(_ptr(ptr), ptr.element_size(), _ptr(cols), cols.element_size(),
                                      int(compressed.B_flat), int(compressed.N), int(compressed.nnz), _ptr(out),
                                      out.element_size(), _stream(device)), "stacr_csr_decode")
    elif mode == IndexCompressionMode.DELTA:
        base, deltas = compressed.delta_base, compressed.col_indices
        ws_bytes = ctypes.c_size_t()
        _lib.check(L.stacr_delta_decode_workspace_bytes(int(compressed.nnz), ctypes.byref(ws_bytes)),
                   "stacr_delta_decode")
        ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
        _lib.check(L.stacr_delta_decode(_ptr(base), base.element_size(), _ptr(deltas),
                                        deltas.element_size() if deltas.numel() else 2, int(compressed.nnz),
                                        _ptr(out), out.element_size(), _ptr(ws), ws_bytes.value, _stream(device)),
                   "stacr_delta_decode")
    else:
        raise ValueError(f"Unknown compression mode: {mode}")
    if restore_order and compressed.sort_indices is not None:
        out = out[compressed.sort_indices]
    return out


# ---------------------------------------------------------------- the adaptive save
def residual_plan(rows: int, feats: int, budget: float, chunk_rows: int = 512):
    """(k, k_saved, index_bytes) of the adaptive "topk" mode (stacr/adaptive.py:1357-1365,1524)."""
    k, ks, ib = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
    _lib.check(_lib.load().stacr_adaptive_residual_plan(int(rows), int(feats), float(budget), int(chunk_rows),
                                                        ctypes.byref(k), ctypes.byref(ks), ctypes.byref(ib)),
               "stacr_adaptive_residual_plan")
    return int(k.value), int(ks.value), int(ib.value)


def save(x2d: torch.Tensor, basis: torch.Tensor, budget: float, chunk_rows: int = 512,
         coeff: torch.Tensor | None = None):
    """coefficients, indices, values (activation dtype) and the energy vector of one adaptive save.

    energy (fp32, device): [residual energy, |X|^2, |C|^2, mean c_j^2 per rank ...].
    """
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    basis = basis.to(x2d.dtype).contiguous()
    rows, feats = x2d.shape
    rank = basis.shape[1]
    dt = dtype_code(x2d.dtype)
    k, k_saved, ib = residual_plan(rows, feats, budget, chunk_rows)
    device = x2d.device
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_adaptive_save_workspace_bytes(rows, feats, rank, dt, float(budget), int(chunk_rows),
                                                     ctypes.byref(ws_bytes)), "stacr_adaptive_save")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
    idx_dtype = {2: torch.int16, 4: torch.int32, 8: torch.int64}[ib]
    idx = torch.empty(k_saved, dtype=idx_dtype, device=device)
    values = torch.empty(k_saved, dtype=x2d.dtype, device=device)
    energy = torch.zeros(3 + rank, dtype=torch.float32, device=device)
    out_coeff = None
    if coeff is None:
        out_coeff = torch.empty(rows, rank, dtype=x2d.dtype, device=device)
    else:
        coeff = coeff.to(x2d.dtype).contiguous()
    _lib.check(L.stacr_adaptive_save(_ptr(x2d), _ptr(basis), dt, rows, feats, rank, float(budget), int(chunk_rows),
                                     _ptr(coeff), _ptr(out_coeff), _ptr(idx), ib, _ptr(values), _ptr(energy),
                                     _ptr(ws), ws_bytes.value, _stream(device)), "stacr_adaptive_save")
    return (coeff if coeff is not None else out_coeff), (idx if k > 0 else None), (values if k > 0 else None), energy


# ---------------------------------------------------------------- the autograd Function
class STACRFunction(torch.autograd.Function):
    """The adaptive engine's STAC-R Function for residual_mode "topk" / "none".

    forward(x, weight, bias, basis, config, layer_state) -> x @ weight^T + bias.  ``config`` keys
    (defaults of stacr/adaptive.py): residual_mode ("topk"), residual_budget (0.01), chunk_size
    (512), quantize_coefficients (False), quantize_residuals (False), residual_quantize_bits (8),
    index_compression ("none" | "csr" | "delta").  ``layer_state`` (dict or None) receives
    last_residual_energy and last_coeff_energy_by_rank as the reference records them.
    Saved tensors follow stacr/adaptive.py:2026-2052: [coefficients(_q), weight, (coeff_scale),
    (bias), (residual values, then row_ptrs+cols | deltas+base | indices, then (residual_scale))].
    """

    @staticmethod
    def forward(ctx, x, weight, bias, basis, config, layer_state=None):
        config = dict(config or {})
        in_features = weight.shape[1]
        leading = x.shape[:-1]
        x2d = x.reshape(-1, in_features)
        w = weight if weight.dtype == x2d.dtype else weight.to(x2d.dtype)
        out = x2d.mm(w.t())
        if bias is not None:
            out = out + (bias if bias.dtype == out.dtype else bias.to(out.dtype)).unsqueeze(0)
        mode = config.get("residual_mode", "topk")
        if mode not in ("topk", "none"):
            raise NotImplementedError(f"adaptive residual_mode {mode!r} has no HIP kernel (topk and none do)")
        budget = float(config.get("residual_budget", 0.01)) if mode == "topk" else 0.0
        chunk = int(config.get("chunk_size", 512))
        basis_c = basis if basis.dtype == x2d.dtype else basis.to(x2d.dtype)
        coeff, idx, values, energy = save(x2d, basis_c, budget, chunk)
        if layer_state is not None:
            e = energy.tolist()
            layer_state["last_residual_energy"] = e[0]
            layer_state["last_coeff_energy_by_rank"] = e[3:3 + basis.shape[1]] if coeff.numel() else None
        b_flat = x2d.shape[0]
        tensors = []
        coeff_scale = None
        if config.get("quantize_coefficients", False):
            if int(config.get("quantize_bits", 8)) != 8:
                raise ValueError("Only int8 coefficient quantization supported")
            coeff_q, coeff_scale = quantize_int8(coeff)
            tensors.append(coeff_q)
        else:
            tensors.append(coeff)
        tensors.append(weight)
        if coeff_scale is not None:
            tensors.append(coeff_scale)
        if bias is not None:
            tensors.append(bias)
        ctx.index_compression_mode = config.get("index_compression", "none")
        ctx.index_compression_nnz = 0
        ctx.residual_bits = int(config.get("residual_quantize_bits", 8))
        ctx.quantize_residuals = bool(config.get("quantize_residuals", False))
        ctx.residual_orig_len = None
        ctx.has_residual = idx is not None
        if idx is not None:
            values_to_save = values
            if ctx.index_compression_mode != "none" and idx.numel():
                comp = compress_indices(idx, b_flat, in_features, ctx.index_compression_mode, preserve_order=False)
                ctx.index_compression_nnz = comp.nnz
                ctx.index_compression_original_dtype = comp.original_dtype
                packed = [comp.row_ptrs, comp.col_indices] if comp.mode == IndexCompressionMode.CSR else \
                    [comp.col_indices, comp.delta_base]
            else:
                packed = [idx]
            residual_scale = None
            if ctx.quantize_residuals:
                if ctx.residual_bits == 8:
                    values_to_save, residual_scale = quantize_int8(values)
                elif ctx.residual_bits == 4:
                    values_to_save, residual_scale, ctx.residual_orig_len = quantize_int4(values)
                else:
                    raise ValueError(f"Unsupported residual_quantize_bits: {ctx.residual_bits}")
            tensors.append(values_to_save)
            tensors.extend(packed)
            if residual_scale is not None:
                tensors.append(residual_scale)
        ctx.save_for_backward(*tensors)
        ctx.quantize_coefficients = coeff_scale is not None
        ctx.has_bias = bias is not None
        ctx.leading_shape = leading
        # the backward must see the basis C was projected on: keep a private copy unless the
        # dtype cast above already made one (a caller may update its basis in place meanwhile)
        ctx.basis = basis_c.detach().clone() if basis_c is basis else basis_c.detach()
        ctx.b_flat, ctx.in_features = b_flat, in_features
        return out.reshape(*leading, weight.shape[0])

    @staticmethod
    def backward(ctx, grad_output):
        from . import kernels

        saved = ctx.saved_tensors
        coeff_saved, weight = saved[0], saved[1]
        i = 2
        if ctx.quantize_coefficients:
            coefficients = dequantize_int8(coeff_saved, saved[i])
            i += 1
        else:
            coefficients = coeff_saved
        bias = None
        if ctx.has_bias:
            bias = saved[i]
            i += 1
        g2d = grad_output.reshape(-1, grad_output.shape[-1])
        compute = g2d.dtype
        residual = None
        if ctx.has_residual:
            values = saved[i]
            i += 1
            if ctx.index_compression_mode != "none" and ctx.index_compression_nnz > 0:
                a, b = saved[i], saved[i + 1]
                i += 2
                if ctx.index_compression_mode == "csr":
                    comp = CompressedIndices(IndexCompressionMode.CSR, row_ptrs=a, col_indices=b,
                                             nnz=ctx.index_compression_nnz, B_flat=ctx.b_flat, N=ctx.in_features,
                                             original_dtype=ctx.index_compression_original_dtype)
                else:
                    comp = CompressedIndices(IndexCompressionMode.DELTA, col_indices=a, delta_base=b,
                                             nnz=ctx.index_compression_nnz, B_flat=ctx.b_flat, N=ctx.in_features,
                                             original_dtype=ctx.index_compression_original_dtype)
                indices = decompress_indices(comp, restore_order=False)
            else:
                indices = saved[i]
                i += 1
            if ctx.quantize_residuals:
                scale = saved[i]
                if values.numel():
                    values = dequantize_int8(values, scale) if ctx.residual_bits == 8 else \
                        dequantize_int4(values, scale, ctx.residual_orig_len or 0)
                else:
                    values = values.to(scale.dtype)
            if indices.numel():
                residual = (indices.to(torch.int64 if indices.dtype == torch.int64 else torch.int32).contiguous(),
                            values.to(compute).contiguous(), None)
        grad_input = grad_weight = grad_bias = None
        if ctx.needs_input_grad[0]:
            w = weight if weight.dtype == g2d.dtype else weight.to(g2d.dtype)
            grad_input = g2d.mm(w).reshape(*ctx.leading_shape, ctx.in_features)
        if ctx.needs_input_grad[1]:
            grad_weight, _ = kernels.weight_grad(g2d, coefficients.to(compute), ctx.basis.to(compute), residual, 0,
                                                 False, weight.dtype)
        if bias is not None and ctx.needs_input_grad[2]:
            grad_bias = g2d.sum(0)
            if grad_bias.dtype != bias.dtype:
                grad_bias = grad_bias.to(bias.dtype)
        return grad_input, grad_weight, grad_bias, None, None, None
