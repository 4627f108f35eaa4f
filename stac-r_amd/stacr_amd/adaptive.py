"""The adaptive engine (stacr/adaptive.py, stacr/index_compression.py) on the HIP kernels.

Kernel-facing helpers, each one library call or a short chain of them:
  * quantize_int8 / dequantize_int8 / quantize_int4 / dequantize_int4 (:44-135): per-tensor, the
    scale computed and kept in the tensor's own dtype, with the reference's fp32 / fp64 redo when
    that scale underflows to zero;
  * _choose_index_dtype (:138-159), compress_indices / decompress_indices with the CSR and delta
    formats (stacr/index_compression.py:118-345);
  * save: the "topk" save (:1333-1572): coefficients, energies and the chunked top-k selection.
The engine built on them: STACRConfig (:599-977), the autograd Functions STACRFunction
(:1045-2470) and STACRLowRankOnlyFunction (:2551-2686) with the reference's
(input, weight, bias, basis, config, step_counter, layer_state) signature, the layer
STACRLinear (:2689-3727; alias AdaptiveSTACRLinear), set_stacr_runtime_state (:3730) and
apply_adaptive_stacr (:3839-3902).  Stable sorting of unsorted index lists (only when a caller
hands compress_indices an unsorted list; the HIP save emits ascending indices) uses torch's sort;
SVD, QR and the rank / refresh policy are host library calls.
"""
from __future__ import annotations

import copy
import ctypes
import json
import math
import threading
import warnings
from dataclasses import asdict, dataclass
from enum import Enum
from typing import Optional, Union

import torch
from torch import nn

from . import _lib
from .kernels import _ptr, _stream, dtype_code, require_gpu
from .rank_controller import BasisRefreshTrigger, basis_update_outlook, select_active_rank, should_update_basis

_SCALE_DTYPES = {_lib.DTYPE_F32: torch.float32, _lib.DTYPE_BF16: torch.bfloat16, _lib.DTYPE_F16: torch.float16,
                 _lib.SCALE_F64: torch.float64}
_SCALE_CODES = {v: k for k, v in _SCALE_DTYPES.items()}


# ---------------------------------------------------------------- scale records
def _record_code(rec: torch.Tensor) -> torch.Tensor:
    """The dtype code of a scale record, as a (1,) device tensor (not read back)."""
    return rec.view(torch.int32)[2:3]


def _scale_from_record(rec: torch.Tensor, code: int) -> torch.Tensor:
    """The reference's scale tensor, shape (1,), in the dtype `code` names (a device-side cast)."""
    return rec.view(torch.float64)[:1].to(_SCALE_DTYPES[int(code)])


def _scale_record_to_tensor(rec: torch.Tensor) -> torch.Tensor:
    """The reference's scale tensor, shape (1,), in the dtype the record names (reads 4 bytes back)."""
    return _scale_from_record(rec, int(_record_code(rec).item()))


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


def save_y(x2d: torch.Tensor, full_basis: torch.Tensor, rank: int, budget: float, chunk_rows: int = 512):
    """save() on the first `rank` columns of `full_basis` (feats x q_cols, the activation dtype), also
    returning Y = X full_basis (rows x q_cols fp32) when the projection pass could write it, else None
    (stacr_adaptive_save_y): (coeff, idx, values, energy, Y or None)."""
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    full = full_basis.to(x2d.dtype).contiguous()
    rows, feats = x2d.shape
    q_cols = full.shape[1]
    dt = dtype_code(x2d.dtype)
    k, k_saved, ib = residual_plan(rows, feats, budget, chunk_rows)
    device = x2d.device
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_adaptive_save_y_workspace_bytes(rows, feats, q_cols, rank, dt, float(budget), int(chunk_rows),
                                                       ctypes.byref(ws_bytes)), "stacr_adaptive_save_y")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
    idx = torch.empty(k_saved, dtype={2: torch.int16, 4: torch.int32, 8: torch.int64}[ib], device=device)
    values = torch.empty(k_saved, dtype=x2d.dtype, device=device)
    energy = torch.zeros(3 + rank, dtype=torch.float32, device=device)
    coeff = torch.empty(rows, rank, dtype=x2d.dtype, device=device)
    y = torch.empty(rows, q_cols, dtype=torch.float32, device=device)
    written = ctypes.c_int(0)
    _lib.check(L.stacr_adaptive_save_y(_ptr(x2d), _ptr(full), dt, rows, feats, q_cols, int(rank), float(budget),
                                       int(chunk_rows), None, _ptr(coeff), _ptr(idx), ib, _ptr(values), _ptr(energy),
                                       _ptr(y), ctypes.byref(written), _ptr(ws), ws_bytes.value, _stream(device)),
               "stacr_adaptive_save_y")
    return coeff, (idx if k > 0 else None), (values if k > 0 else None), energy, (y if written.value else None)


def block_sparse_plan(rows: int, feats: int, budget: float, chunk_rows: int = 512, block_size: int = 16):
    """(k_blocks, max entries, index bytes, workspace bytes) of the adaptive block_sparse selector."""
    kb, mx, ib, ws = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int(), ctypes.c_size_t()
    _lib.check(_lib.load().stacr_adaptive_block_sparse_plan(int(rows), int(feats), float(budget), int(chunk_rows),
                                                            int(block_size), ctypes.byref(kb), ctypes.byref(mx),
                                                            ctypes.byref(ib), ctypes.byref(ws)),
               "stacr_adaptive_block_sparse_plan")
    return int(kb.value), int(mx.value), int(ib.value), int(ws.value)


def select_block_sparse(x2d: torch.Tensor, coeff: torch.Tensor, basis: torch.Tensor, budget: float,
                        chunk_rows: int = 512, block_size: int = 16):
    """(flat indices, residual values) of the adaptive block_sparse selector (stacr/adaptive.py:1788-1938),
    ascending, or (None, None) when the budget keeps no entry.  Every column of the kept blocks is
    stored; when feats % block_size != 0 the count depends on which row-end blocks were kept and is
    read back from the device (one read, as the reference's boolean mask also syncs)."""
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    coeff = coeff.to(x2d.dtype).contiguous()
    basis = basis.to(x2d.dtype).contiguous()
    rows, feats = x2d.shape
    k_blocks, max_entries, ib, ws_bytes = block_sparse_plan(rows, feats, budget, chunk_rows, block_size)
    if k_blocks == 0:
        return None, None
    device = x2d.device
    idx = torch.empty(max_entries, dtype={2: torch.int16, 4: torch.int32, 8: torch.int64}[ib], device=device)
    values = torch.empty(max_entries, dtype=x2d.dtype, device=device)
    count = torch.empty((), dtype=torch.int64, device=device)
    ws = torch.empty(max(1, ws_bytes), dtype=torch.uint8, device=device)
    _lib.check(_lib.load().stacr_adaptive_select_block_sparse(
        _ptr(x2d), _ptr(coeff), _ptr(basis), dtype_code(x2d.dtype), rows, feats, basis.shape[1], float(budget),
        int(chunk_rows), int(block_size), _ptr(idx), ib, _ptr(values), _ptr(count), _ptr(ws), ws_bytes,
        _stream(device)), "stacr_adaptive_select_block_sparse")
    if feats % block_size:
        n = int(count.item())
        idx, values = idx[:n], values[:n]
    return idx, values


# ================================================================ configuration
_CONFIG_CHOICES = {
    "residual_mode": ("none", "topk", "threshold", "block_sparse", "adaptive_threshold", "sparse_only"),
    "update_trigger": ("fixed", "adaptive", "hybrid"),
    "streaming_algorithm": ("oja",),
    "backward_mode": ("dense", "sparse"),
    "rank_mode": ("fixed", "variance", "sensitivity"),
    "basis_sharing": ("none", "every_2", "every_3", "every_4", "all"),
    "index_compression": ("none", "csr", "delta"),
    "adaptive_layer_rank": ("none", "heuristic"),
    "residual_schedule": ("none", "linear", "cosine"),
    "post_warmup_residual_mode": ("full", "none", "threshold"),
    "refresh_trigger": ("off", "fixed", "residual_energy", "hybrid"),
}
_POSITIVE_INTS = ("rank", "update_interval", "chunk_size", "residual_block_size", "rank_min", "rank_max",
                  "rank_adjust_interval", "refresh_period", "randomized_svd_threshold")
_NONNEGATIVE_INTS = ("warmup_steps", "residual_warmup_steps", "min_adaptation_steps", "randomized_svd_oversampling",
                     "randomized_svd_niter")
_UNIT_FRACTIONS = ("residual_budget", "residual_start", "residual_end", "rank_variance_threshold",
                   "streaming_topk_sample_ratio", "skip_residual_energy_threshold")
_NONNEGATIVE_REALS = ("oja_learning_rate", "energy_threshold", "residual_threshold", "adaptive_oja_scale",
                      "adaptive_oja_max_lr", "lazy_update_threshold", "refresh_energy_threshold",
                      "rank_sensitivity_low", "rank_sensitivity_high", "rank_step_fraction")
# fields the layer does not hand to its Function (the Function then uses its own chunk default of
# 512 rows, as stacr/adaptive.py's to_dict omits chunk_size)
_NOT_IN_FUNCTION_CONFIG = ("chunk_size", "joint_qk")


def _resolve_basis_dtype(value: object, auto_detect_amp: bool = True) -> torch.dtype:
    """torch dtype named by `value`: "auto" is fp16 while GPU autocast is on, else fp32
    (stacr/adaptive.py:162-198)."""
    if isinstance(value, torch.dtype):
        return value
    if not isinstance(value, str):
        return torch.float32
    name = value.lower()
    if name == "auto":
        amp = auto_detect_amp and torch.cuda.is_available() and torch.is_autocast_enabled()
        return torch.float16 if amp else torch.float32
    for dtype, names in ((torch.float32, ("float32", "fp32", "torch.float32")),
                         (torch.float16, ("float16", "fp16", "half", "torch.float16")),
                         (torch.bfloat16, ("bfloat16", "bf16", "torch.bfloat16"))):
        if name in names:
            return dtype
    raise ValueError(f"Unsupported basis dtype: {value}. Use 'auto', 'float32', 'float16', or 'bfloat16'.")


@dataclass
class STACRConfig:
    """Adaptive-engine configuration: the reference's fields, defaults and validation
    (stacr/adaptive.py:599-977), so configs and checkpoints written for it load here.

    Every residual_mode runs on the HIP kernels ("topk" and its streaming form, "threshold",
    "adaptive_threshold", "block_sparse" (the default), "none", "sparse_only", and the warmup
    baseline), with or without basis sharing between layers.
    """

    method: str = "stacr"
    rank: int = 32
    # residual channel
    residual_mode: str = "block_sparse"
    residual_budget: float = 0.005
    residual_threshold: float = 0.1
    # basis update schedule
    update_trigger: str = "hybrid"
    update_interval: int = 100
    energy_threshold: float = 0.05
    streaming_algorithm: str = "oja"
    oja_learning_rate: float = 0.01
    warmup_steps: int = 0
    freeze_basis_after_warmup: bool = True
    # quantization
    quantize_coefficients: bool = True
    quantize_bits: int = 8
    quantize_residuals: bool = True
    residual_quantize_bits: int = 4
    # basis initialization
    randomized_svd_threshold: int = 1024
    randomized_svd_oversampling: int = 4
    randomized_svd_niter: int = 2
    adaptive_oja_lr: bool = False
    adaptive_oja_scale: float = 5.0
    adaptive_oja_max_lr: float = 0.1
    basis_dtype: str = "auto"
    use_random_qr_init: bool = False
    min_adaptation_steps: int = 50
    allow_unadapted_random_qr: bool = False
    backward_mode: str = "sparse"
    residual_block_size: int = 16
    use_mgs: bool = False
    lazy_update_threshold: float = 0.01
    lazy_update_enabled: bool = True
    use_fused_kernel: bool = False
    streaming_topk: bool = False
    streaming_topk_sample_ratio: float = 0.1
    chunk_size: int = 512
    # runtime rank
    rank_mode: str = "fixed"
    rank_variance_threshold: float = 0.95
    rank_min: int = 4
    rank_max: int = 64
    rank_adjust_interval: int = 100
    rank_sensitivity_low: float = 0.03
    rank_sensitivity_high: float = 0.10
    rank_step_fraction: float = 0.125
    basis_sharing: str = "none"
    basis_sharing_group: Optional[int] = None
    joint_qk: bool = False
    cpu_offload: bool = False
    index_compression: str = "none"
    skip_residual_enabled: bool = False
    skip_residual_energy_threshold: float = 0.05
    buffer_reuse: bool = False
    adaptive_layer_rank: str = "none"
    residual_schedule: str = "none"
    residual_start: float = 0.05
    residual_end: float = 0.001
    post_warmup_residual_mode: str = "full"
    residual_warmup_steps: int = 0
    post_warmup_residual_threshold: float = 0.1
    refresh_trigger: str = "off"
    refresh_period: int = 1000
    refresh_energy_threshold: float = 0.1
    cache_basis_per_optimizer_step: bool = False
    oja_update_per_optimizer_step: bool = False
    enable_low_rank_only_fast_path: bool = True

    def __post_init__(self):
        """Reject unsupported settings before any model is changed (messages as the reference's)."""
        for name, accepted in _CONFIG_CHOICES.items():
            if getattr(self, name) not in accepted:
                raise ValueError(f"{name} must be one of {sorted(accepted)}")
        for names, ok, message in (
                (_POSITIVE_INTS, lambda v: _is_int(v) and v >= 1, "{} must be a positive integer"),
                (_NONNEGATIVE_INTS, lambda v: _is_int(v) and v >= 0, "{} must be a nonnegative integer"),
                (_UNIT_FRACTIONS, lambda v: math.isfinite(v) and 0 <= v <= 1, "{} must be between 0 and 1")):
            for name in names:
                if not ok(getattr(self, name)):
                    raise ValueError(message.format(name))
        if self.quantize_bits != 8 or self.residual_quantize_bits not in (4, 8):
            raise ValueError("Coefficient quantization requires 8 bits; residual quantization requires 4 or 8")
        if self.rank_min > self.rank_max:
            raise ValueError("rank_min cannot exceed rank_max")
        if self.rank_sensitivity_low > self.rank_sensitivity_high:
            raise ValueError("rank_sensitivity_low cannot exceed rank_sensitivity_high")
        for name in _NONNEGATIVE_REALS:
            value = getattr(self, name)
            if not math.isfinite(value) or value < 0:
                raise ValueError(f"{name} must be finite and nonnegative")
        _resolve_basis_dtype(self.basis_dtype)
        if self.basis_sharing != "none" and self.rank_mode != "fixed":
            raise ValueError("Basis sharing requires rank_mode='fixed'")

    def get_layer_rank(self, layer_idx: int, base_rank: int, num_layers: int = 12) -> int:
        """Per-layer rank: the base rank, or under "heuristic" 1.0 / 0.7 / 0.4 of it for the first /
        middle / last third of the layers, at least 8 (stacr/adaptive.py:932-959)."""
        if self.adaptive_layer_rank != "heuristic":
            return base_rank
        third = num_layers // 3
        factor = 1.0 if layer_idx < third else (0.7 if layer_idx < 2 * third else 0.4)
        return max(8, int(base_rank * factor))

    def get_residual_budget(self, step: int, total_steps: int) -> float:
        """Residual budget at `step` of `total_steps` under the residual schedule."""
        return _scheduled_budget(self.residual_schedule, self.residual_budget, self.residual_start,
                                 self.residual_end, step / max(1, total_steps))

    def to_dict(self) -> dict:
        """The options a layer hands its autograd Function."""
        out = asdict(self)
        for name in _NOT_IN_FUNCTION_CONFIG:
            out.pop(name)
        if isinstance(out["basis_dtype"], torch.dtype):
            out["basis_dtype"] = str(out["basis_dtype"])
        return out


class BasisPool:
    """The bases that the layers of a sharing group use when basis_sharing is on (the interface of
    stacr/adaptive.py:271-381): one tensor per (group, in_features, rank), all zeros until a member
    of the group fits it.  An update installs a new tensor rather than writing into the old one, so
    a forward that took the previous basis keeps it for its backward and its recomputation."""

    def __init__(self):
        self._lock = threading.Lock()
        self._bases: dict = {}

    def get_or_create_basis(self, group_id: int, in_features: int, rank: int, device, dtype: torch.dtype):
        key = (group_id, in_features, rank)
        with self._lock:
            basis = self._bases.get(key)
            if basis is None:
                basis = torch.zeros(in_features, rank, dtype=dtype, device=device)
            elif basis.device != torch.device(device) or basis.dtype != dtype:
                basis = basis.to(device=device, dtype=dtype)
            self._bases[key] = basis
            return basis

    def update_basis(self, group_id: int, in_features: int, rank: int, new_basis: torch.Tensor) -> None:
        fresh = new_basis.detach().clone()
        with self._lock:
            self._bases[(group_id, in_features, rank)] = fresh

    def is_initialized(self, group_id: int, in_features: int, rank: int) -> bool:
        """Whether a member has fitted the group's basis (it is no longer all zeros)."""
        with self._lock:
            basis = self._bases.get((group_id, in_features, rank))
        return basis is not None and bool(basis.abs().sum().item() > 0)

    def clear(self) -> None:
        with self._lock:
            self._bases.clear()


_BASIS_POOL = BasisPool()


def get_basis_pool() -> BasisPool:
    """The process-wide pool of shared bases."""
    return _BASIS_POOL


_SHARING_GROUP = {"all": lambda i: 0, "every_2": lambda i: i // 2, "every_3": lambda i: i // 3,
                  "every_4": lambda i: i // 4}


def _is_int(value) -> bool:
    return not isinstance(value, bool) and int(value) == value


def _scheduled_budget(schedule: str, fixed: float, start: float, end: float, progress: float) -> float:
    if schedule == "linear":
        return start - (start - end) * progress
    if schedule == "cosine":
        return end + 0.5 * (start - end) * (1 + math.cos(math.pi * progress))
    return fixed


def profile_layer_spectrum(activations: torch.Tensor, threshold: float = 0.95, return_full: bool = False) -> dict:
    """The smallest rank whose squared singular values reach `threshold` of the total energy
    (stacr/adaptive.py:980-1042); singular values are a library call."""
    with torch.no_grad():
        rows = activations.reshape(-1, activations.shape[-1]) if activations.dim() > 2 else activations
        if rows.numel() == 0:
            out = {"adaptive_rank": 1, "total_energy": 0.0, "energy_at_rank": 0.0}
            if return_full:
                out["spectrum"] = []
            return out
        sv = torch.linalg.svdvals(rows.float())
        energy = sv * sv
        total = energy.sum().item()
        if total < 1e-12:
            out = {"adaptive_rank": 1, "total_energy": total, "energy_at_rank": 0.0}
        else:
            captured = torch.cumsum(energy, dim=0) / total
            rank = max(1, min(int((captured < threshold).sum().item()) + 1, sv.numel()))
            out = {"adaptive_rank": rank, "total_energy": total, "energy_at_rank": captured[rank - 1].item()}
        if return_full:
            out["spectrum"] = sv.cpu().numpy()
        return out


# ================================================================ the autograd Functions
def _is_recomputing() -> bool:
    from .adaptive_checkpointing import get_global_recomputation_guard

    return get_global_recomputation_guard().is_recomputing


def _dense_output(x2d: torch.Tensor, weight: torch.Tensor, bias):
    """X W^T (+ b) as the adaptive engine forms it: the product in X's dtype, then the bias added."""
    out = x2d.mm((weight if weight.dtype == x2d.dtype else weight.to(x2d.dtype)).t())
    if bias is not None:
        out = out + (bias if bias.dtype == out.dtype else bias.to(out.dtype)).unsqueeze(0)
    return out


def _residual_plan(config: dict, layer_state: dict, step_counter) -> tuple[str, float, Optional[float]]:
    """(effective residual mode, budget, energy-skip threshold or None) for this forward
    (stacr/adaptive.py:1080-1132): the post-warmup Turbo switch and the budget schedule."""
    mode = config["residual_mode"]
    step = int(layer_state.get("_schedule_step", 0))
    post, warm = config.get("post_warmup_residual_mode", "full"), config.get("residual_warmup_steps", 0)
    turbo_gate = False
    if post != "full" and warm > 0 and step >= warm:
        if not layer_state.get("_turbo_switched", False):
            layer_state.update(_turbo_switched=True, _turbo_switch_step=step, _turbo_original_mode=mode,
                               _turbo_mode=post)
        if post == "none":
            mode = "none"
        elif post == "threshold":
            turbo_gate = True
    budget = float(config["residual_budget"])
    total = layer_state.get("total_steps")
    if config.get("residual_schedule", "none") != "none" and total is not None and total > 0:
        now = step_counter[0].item() if hasattr(step_counter[0], "item") else int(step_counter[0])
        budget = _scheduled_budget(config["residual_schedule"], budget, float(config.get("residual_start", 0.05)),
                                   float(config.get("residual_end", 0.001)), now / max(1, total))
    budget = max(0.0, min(1.0, budget))
    layer_state["current_residual_budget"] = budget
    if turbo_gate:
        gate = float(config.get("post_warmup_residual_threshold", 0.1))
    elif config.get("skip_residual_enabled", False):
        gate = float(config.get("skip_residual_energy_threshold", 0.05))
    else:
        gate = None
    return mode, budget, gate


def _select_above(x2d: torch.Tensor, coeff: torch.Tensor, basis: torch.Tensor, threshold):
    """(indices, values) of every residual with |r| > threshold, ascending, as the reference's
    `chunk_flat.abs() > threshold_val` + `nonzero` over the chunks (stacr/adaptive.py:1493-1517,
    1574-1622, 1762-1786): the threshold (a Python float, or a 0-dim tensor) is rounded to the
    activation dtype as torch's comparison does, and the strict comparison becomes the HIP
    selector's |r| >= t' with t' the next value of that dtype above it.  Indices in
    _choose_index_dtype(rows * feats)."""
    dt = x2d.dtype
    t = torch.as_tensor(threshold, device="cpu").to(dt)  # the dtype rounding of the comparison
    index_dtype = _choose_index_dtype(x2d.numel())
    tv = float(t)
    if tv == 0:
        t = torch.zeros((), dtype=dt)  # -0 compares as +0: one ulp above it is the smallest subnormal
    if tv != tv or tv == math.inf:  # nothing compares above NaN or +inf
        return torch.empty(0, dtype=index_dtype, device=x2d.device), torch.empty(0, dtype=dt, device=x2d.device)
    if tv < 0:
        # every residual but NaN passes (|r| >= 0); the selector's >= 0 gives exactly that
        nxt = torch.zeros((), dtype=torch.float32)
    else:
        # the next representable value above t in the activation dtype (t >= 0: one ulp up)
        ibits = {torch.float32: torch.int32, torch.bfloat16: torch.int16, torch.float16: torch.int16}[dt]
        nxt = (t.reshape(1).view(ibits) + 1).view(dt).float().reshape(())
    from .kernels import select_threshold
    idx, values = select_threshold(x2d, coeff, basis, nxt.to(x2d.device), None)
    return idx.to(index_dtype), values


def _sampled_threshold(x2d: torch.Tensor, coeff: torch.Tensor, basis: torch.Tensor, chunk_size: int,
                       sample_size: int, quantile: float) -> torch.Tensor:
    """The threshold the reference's sampling passes estimate (stacr/adaptive.py:1422-1470,
    1694-1738): per chunk of `chunk_size` rows, min(samples_per_chunk, chunk elements) positions
    from torch.randint on the activation's device (the global generator, drawn chunk by chunk in
    the reference's order), |r| there (one HIP gather for all chunks), then torch.quantile of
    those magnitudes (in fp32 for 16-bit types, rounded back to the activation dtype)."""
    from .kernels import sample_magnitudes
    rows, feats = x2d.shape
    per_chunk = max(1, (sample_size * chunk_size) // rows)
    positions = []
    for start in range(0, rows, chunk_size):
        n_el = (min(start + chunk_size, rows) - start) * feats
        n = min(per_chunk, n_el)
        if n > 0:
            positions.append(torch.randint(0, n_el, (n,), device=x2d.device) + start * feats)
    samples = sample_magnitudes(x2d, coeff, basis, torch.cat(positions))
    if samples.dtype in (torch.float16, torch.bfloat16):
        return torch.quantile(samples.float(), quantile).to(samples.dtype)
    return torch.quantile(samples, quantile)


def _record_energy(layer_state: dict, energy_host: list, rank: int, coeff_rows: int, schedule_step: int) -> None:
    layer_state["last_residual_energy"] = energy_host[0]
    layer_state["step"] = schedule_step
    layer_state["last_coeff_energy_by_rank"] = energy_host[3:3 + rank] if coeff_rows else None


def _offload(t: torch.Tensor) -> torch.Tensor:
    return t.to("cpu", non_blocking=True) if t.is_cuda else t


def _onload(t: torch.Tensor, device) -> torch.Tensor:
    return t.to(device) if t.device != device else t


def _basis_for_backward(basis_c: torch.Tensor, basis: torch.Tensor) -> torch.Tensor:
    """A private copy of the basis C was projected on (the layer may replace or refresh its basis
    before this backward runs); a dtype cast already made one."""
    return basis_c.detach().clone() if basis_c.data_ptr() == basis.data_ptr() else basis_c.detach()


class STACRFunction(torch.autograd.Function):
    """The adaptive engine's autograd Function (stacr/adaptive.py:1045-2470) on the HIP kernels.

    forward(input, weight, bias, basis, config, step_counter, layer_state): exact Y = X W^T + b;
    saves the full input during warmup (or without a basis), otherwise the coefficients C = X B
    (int8 per-tensor when quantize_coefficients), the selected residual (values, flat indices or
    their CSR / delta streams, optional int8 / int4 values) in the reference's tensor order, and
    the basis version.  The save is one stacr_adaptive_save call (projection, energies, chunked
    top-k with the adaptive k rules); the backward is one stacr_weight_grad call.
    """

    @staticmethod
    def forward(ctx, input_tensor, weight, bias, basis, config, step_counter, layer_state):
        mode, budget, gate = _residual_plan(config, layer_state, step_counter)
        schedule_step = int(layer_state.get("_schedule_step", 0))
        in_features = weight.shape[1]
        leading = input_tensor.shape[:-1]
        x2d = input_tensor.reshape(-1, in_features)
        b_flat = x2d.shape[0]
        output = _dense_output(x2d, weight, bias).reshape(*leading, weight.shape[0])
        ctx.leading_shape, ctx.has_bias = leading, bias is not None
        ctx.residual_shape, ctx.cpu_offload = (b_flat, in_features), False
        recomputing = _is_recomputing()

        # streaming top-k: the reference's fused route takes precedence when it runs (budget > 0)
        streaming = (mode == "topk" and config.get("streaming_topk", False)
                     and not (config.get("use_fused_kernel", False) and budget > 0))
        if config.get("use_fused_kernel", False):
            layer_state["b4_fused_kernel_route"] = "hip_save"

        quant_res = bool(config.get("quantize_residuals", False))
        res_bits = int(config.get("residual_quantize_bits", 8))
        ctx.quantize_residuals, ctx.residual_bits, ctx.residual_orig_len = quant_res, res_bits, None

        if mode == "sparse_only":  # top-k of the raw activation: the save with a zero basis
            zero = torch.zeros(in_features, 1, dtype=x2d.dtype, device=x2d.device)
            _, idx, values, _ = save(x2d, zero, budget, 512)
            tensors = [weight] + ([bias] if bias is not None else [])
            if idx is not None:
                stored, scale = _quantize_residual(values, quant_res, res_bits, ctx)
                tensors += [stored, idx] + ([scale] if scale is not None else [])
            ctx.save_for_backward(*tensors)
            ctx.stacr_mode, ctx.has_residual = "sparse_only", idx is not None
            if not recomputing:
                layer_state["last_residual_energy"] = 1.0
                layer_state["step"] = schedule_step
            return output

        if schedule_step < config["warmup_steps"] or basis is None or basis.numel() == 0:
            ctx.save_for_backward(*([x2d, weight] + ([bias] if bias is not None else [])))
            ctx.stacr_mode = "baseline"
            return output

        basis_c = basis if basis.dtype == x2d.dtype else basis.to(x2d.dtype)
        rank = basis_c.shape[1]
        chunk = int(config.get("chunk_size", 512))
        total = b_flat * in_features
        k_budget = min(int(total * budget), total)  # the k of "topk" and "adaptive_threshold"
        exact_topk = mode == "topk" and not streaming
        # The layer asks for Y = X B over its whole allocated basis when a post-forward Oja refresh may
        # follow on this X (its refresh then reads X once more instead of twice); the save computes
        # it in its projection pass.  Y serves the refresh only when B is exact in the activation
        # dtype (the refresh projects on B itself) and the saved basis is B's leading columns.
        full = layer_state.pop("_oja_y_request", None) if not recomputing else None
        y = None
        # basis_c = full[:, :rank] (a column slice keeps the data pointer and strides, whatever the layout)
        leading_cols = full is not None and basis_c.data_ptr() == full.data_ptr() and basis_c.stride() == full.stride()
        if (leading_cols and full.dtype == x2d.dtype and full.shape[0] == in_features
                and full.shape[1] >= rank):
            coeff, idx, values, energy, y = save_y(x2d, full, rank, budget if exact_topk else 0.0, chunk)
            layer_state["_oja_y"] = (y, full, x2d) if y is not None else None
        else:
            coeff, idx, values, energy = save(x2d, basis_c, budget if exact_topk else 0.0, chunk)
        # "adaptive_threshold" with k = 0 keeps no residual and computes no energy (it stays 0)
        no_energy = mode == "adaptive_threshold" and k_budget <= 0
        # The host reads of a forward: the energies (the rank controller, refresh triggers and skip
        # gate consume them every step, as in the reference) and the dtype code of each quantized
        # scale, fetched together in one transfer after every kernel is queued.  Only a skip gate
        # needs the energy first, to decide whether the residual is kept.
        energy_host = None
        if gate is not None and not no_energy and mode in ("topk", "block_sparse", "threshold", "adaptive_threshold"):
            energy_host = energy.tolist()
        skipped = energy_host is not None and energy_host[0] < gate
        if skipped:
            idx = values = None
        elif mode == "block_sparse":
            idx, values = select_block_sparse(x2d, coeff, basis_c, budget, chunk,
                                              int(config.get("residual_block_size", 16)))
        elif mode == "threshold":  # every |r| above the configured value (stacr/adaptive.py:1574-1622)
            idx, values = _select_above(x2d, coeff, basis_c, float(config["residual_threshold"]))
        elif mode == "adaptive_threshold" and k_budget > 0:  # (stacr/adaptive.py:1628-1786)
            thr = _sampled_threshold(x2d, coeff, basis_c, min(chunk, b_flat),
                                     min(100000, max(10000, total // 10)), 1.0 - budget)
            idx, values = _select_above(x2d, coeff, basis_c, thr)
        elif streaming and k_budget > 0:  # streaming top-k (stacr/adaptive.py:1416-1517)
            ratio = float(config.get("streaming_topk_sample_ratio", 0.1))
            thr = _sampled_threshold(x2d, coeff, basis_c, min(chunk, b_flat),
                                     min(100000, max(10000, int(total * ratio))), 1.0 - k_budget / total)
            idx, values = _select_above(x2d, coeff, basis_c, thr)

        coeff_rec = None
        if config.get("quantize_coefficients", False):
            if int(config.get("quantize_bits", 8)) != 8:
                raise ValueError(f"Only int8 coefficient quantization supported, got {config.get('quantize_bits')}")
            if coeff.numel():
                coeff_saved, rec = _quantize_record(coeff, 8)
                coeff_saved, coeff_rec = coeff_saved.reshape(coeff.shape), (rec,)
            else:
                coeff_saved, coeff_rec = quantize_int8(coeff)  # (no record: the reference's ones scale)
        else:
            coeff_saved = coeff
        ctx.index_compression_mode = config.get("index_compression", "none")
        ctx.index_compression_nnz, ctx.index_compression_B_flat = 0, b_flat
        ctx.index_compression_N, ctx.index_compression_original_dtype = in_features, torch.int32
        streams, stored, res_rec = [], None, None
        if idx is not None:
            # the save emits ascending flat indices, which is both the row order CSR needs and the
            # sorted order delta needs, so no permutation of the values is required
            streams = [idx]
            if ctx.index_compression_mode != "none" and idx.numel():
                if ctx.index_compression_mode == "csr":
                    streams = list(_csr_encode(idx, b_flat, in_features))
                else:
                    base, deltas = _delta_encode(idx, b_flat, in_features)
                    streams = [deltas, base]
                ctx.index_compression_nnz = idx.numel()
                ctx.index_compression_original_dtype = idx.dtype
            stored, res_rec = _quantize_residual_record(values, quant_res, res_bits, ctx)

        # the one transfer: energies (unless already read) and the records' dtype codes
        reads = [] if energy_host is not None or recomputing else [energy.to(torch.float64)]
        recs = [r for r in (coeff_rec, res_rec) if isinstance(r, tuple)]
        reads += [_record_code(r[0]).to(torch.float64) for r in recs]
        host = torch.cat(reads).tolist() if reads else []
        if energy_host is None and not recomputing:
            energy_host, host = host[:energy.numel()], host[energy.numel():]
        codes = {id(r): host[i] for i, r in enumerate(recs)}
        coeff_scale = None
        if coeff_rec is not None:
            coeff_scale = _scale_from_record(coeff_rec[0], codes[id(coeff_rec)]) if isinstance(coeff_rec, tuple) else coeff_rec
        res_scale = None
        if res_rec is not None:
            res_scale = _scale_from_record(res_rec[0], codes[id(res_rec)]) if isinstance(res_rec, tuple) else res_rec

        if not recomputing:
            if no_energy:
                energy_host = [0.0] + list(energy_host[1:])
            _record_energy(layer_state, energy_host, rank, coeff.shape[0], schedule_step)
            if skipped:
                layer_state["skipped_residuals"] = layer_state.get("skipped_residuals", 0) + 1
            if not config.get("use_fused_kernel", False):
                layer_state["b4_fused_kernel_route"] = "disabled"
                layer_state["b4_numerical_parity_error"] = None

        tensors = [coeff_saved, weight] + ([coeff_scale] if coeff_scale is not None else [])
        tensors += [bias] if bias is not None else []
        if idx is not None:
            tensors += [stored] + streams + ([res_scale] if res_scale is not None else [])
        first_residual = 2 + (coeff_scale is not None) + (bias is not None)
        if config.get("cpu_offload", False) and tensors[0].is_cuda:
            ctx.cpu_offload = True
            tensors[0] = _offload(tensors[0])
            for i in range(first_residual, len(tensors)):
                tensors[i] = _offload(tensors[i])
        ctx.save_for_backward(*tensors)
        ctx.stacr_mode, ctx.has_residual = "stacr", idx is not None
        ctx.quantize_coefficients = coeff_scale is not None
        ctx.backward_mode = config.get("backward_mode", "sparse")
        ctx.rank = rank
        ctx.basis = _basis_for_backward(basis_c, basis)
        ctx.basis_clone_skipped = False
        return output

    @staticmethod
    def backward(ctx, grad_output):
        saved = list(ctx.saved_tensors)
        g2d = grad_output.reshape(-1, grad_output.shape[-1])
        if ctx.stacr_mode == "baseline":
            x2d, weight = saved[0], saved[1]
            bias = saved[2] if ctx.has_bias else None
            return _baseline_grads(ctx, g2d, x2d, weight, bias)
        if ctx.stacr_mode == "sparse_only":
            weight, pos = saved[0], 1
            bias = saved[pos] if ctx.has_bias else None
            pos += ctx.has_bias
            residual = None
            if ctx.has_residual:
                values, idx = saved[pos], saved[pos + 1]
                pos += 2
                if ctx.quantize_residuals:
                    values = _dequantize_residual(values, saved[pos], ctx)
                residual = (idx, values)
            b_flat, in_features = ctx.residual_shape
            zero_c = torch.zeros(b_flat, 1, dtype=g2d.dtype, device=g2d.device)
            zero_q = torch.zeros(in_features, 1, dtype=g2d.dtype, device=g2d.device)
            return _factor_grads(ctx, g2d, weight, bias, zero_c, zero_q, residual)

        device = saved[1].device
        coeff_saved, weight = _onload(saved[0], device), saved[1]
        pos = 2
        if ctx.quantize_coefficients:
            coefficients = dequantize_int8(coeff_saved, saved[pos])
            pos += 1
        else:
            coefficients = coeff_saved
        bias = None
        if ctx.has_bias:
            bias, pos = saved[pos], pos + 1
        residual = None
        if ctx.has_residual:
            values = _onload(saved[pos], device)
            pos += 1
            if ctx.index_compression_mode != "none" and ctx.index_compression_nnz > 0:
                a, b = _onload(saved[pos], device), _onload(saved[pos + 1], device)
                pos += 2
                csr = ctx.index_compression_mode == "csr"
                comp = CompressedIndices(
                    IndexCompressionMode.CSR if csr else IndexCompressionMode.DELTA,
                    row_ptrs=a if csr else None, col_indices=b if csr else a, delta_base=None if csr else b,
                    nnz=ctx.index_compression_nnz, B_flat=ctx.index_compression_B_flat,
                    N=ctx.index_compression_N, original_dtype=ctx.index_compression_original_dtype)
                idx = decompress_indices(comp, restore_order=False)
            else:
                idx, pos = _onload(saved[pos], device), pos + 1
            if ctx.quantize_residuals:
                values = _dequantize_residual(values, _onload(saved[pos], device), ctx)
            residual = (idx, values)
        return _factor_grads(ctx, g2d, weight, bias, coefficients, ctx.basis, residual)


def _quantize_residual_record(values, quantize: bool, bits: int, ctx):
    """(stored values, (record,) or a scale tensor or None): as _quantize_residual, but a non-empty
    tensor's scale stays a device record whose dtype code the caller reads with its others."""
    if not quantize:
        return values, None
    if not values.numel():
        return _quantize_residual(values, quantize, bits, ctx)
    if bits not in (4, 8):
        raise ValueError(f"Unsupported residual_quantize_bits: {bits}")
    data, rec = _quantize_record(values, bits)
    if bits == 4:
        ctx.residual_orig_len = values.numel()
    else:
        data = data.reshape(values.shape)
    return data, (rec,)


def _quantize_residual(values, quantize: bool, bits: int, ctx):
    """(stored values, scale or None): int8 / int4 per-tensor codes after any index reordering."""
    if not quantize:
        return values, None
    if bits == 8:
        return quantize_int8(values)
    if bits == 4:
        packed, scale, ctx.residual_orig_len = quantize_int4(values)
        return packed, scale
    raise ValueError(f"Unsupported residual_quantize_bits: {bits}")


def _dequantize_residual(stored, scale, ctx):
    if not stored.numel():
        return stored.to(scale.dtype)
    if ctx.residual_bits == 8:
        return dequantize_int8(stored, scale)
    if ctx.residual_bits == 4:
        return dequantize_int4(stored, scale, ctx.residual_orig_len or 0)
    raise ValueError(f"Unsupported residual_quantize_bits: {ctx.residual_bits}")


def _input_and_bias_grads(ctx, g2d, weight, bias, in_features):
    grad_input = grad_bias = None
    if ctx.needs_input_grad[0]:
        w = weight if weight.dtype == g2d.dtype else weight.to(g2d.dtype)
        grad_input = g2d.mm(w).reshape(*ctx.leading_shape, in_features)
    if bias is not None and ctx.needs_input_grad[2]:
        grad_bias = g2d.sum(0)
        grad_bias = grad_bias if grad_bias.dtype == bias.dtype else grad_bias.to(bias.dtype)
    return grad_input, grad_bias


def _baseline_grads(ctx, g2d, x2d, weight, bias):
    grad_input, grad_bias = _input_and_bias_grads(ctx, g2d, weight, bias, weight.shape[1])
    grad_weight = None
    if ctx.needs_input_grad[1]:
        grad_weight = g2d.t().mm(x2d if x2d.dtype == g2d.dtype else x2d.to(g2d.dtype))
        grad_weight = grad_weight if grad_weight.dtype == weight.dtype else grad_weight.to(weight.dtype)
    return grad_input, grad_weight, grad_bias, None, None, None, None


def _factor_grads(ctx, g2d, weight, bias, coefficients, basis, residual):
    """grad_W = (G^T C) B^T + G^T R_s in one stacr_weight_grad call (fp32 accumulation, rounded once
    to the weight dtype); grad_input and grad_bias as native ops."""
    from . import kernels

    grad_input, grad_bias = _input_and_bias_grads(ctx, g2d, weight, bias, weight.shape[1])
    grad_weight = None
    if ctx.needs_input_grad[1]:
        compute = g2d.dtype
        res = None
        if residual is not None and residual[1].numel():
            idx, values = residual
            idx = idx.to(torch.int64 if idx.dtype == torch.int64 else torch.int32).contiguous()
            res = (idx, values.to(compute).contiguous(), None)
        grad_weight, _ = kernels.weight_grad(g2d, coefficients.to(compute), basis.to(compute), res, 0, False,
                                             weight.dtype)
    return grad_input, grad_weight, grad_bias, None, None, None, None


class STACRLowRankOnlyFunction(torch.autograd.Function):
    """The adaptive engine's residual-free route (stacr/adaptive.py:2551-2686): saves C = X B (not
    quantized) and the basis version; grad_W = (G^T C) B^T."""

    @staticmethod
    def forward(ctx, input_tensor, weight, bias, basis, config, step_counter, layer_state):
        del step_counter
        schedule_step = int(layer_state.get("_schedule_step", 0))
        effective = config.get("residual_mode", "topk")
        post, warm = config.get("post_warmup_residual_mode", "full"), int(config.get("residual_warmup_steps", 0))
        if post != "full" and warm > 0 and schedule_step >= warm:
            effective = {"none": "none", "threshold": "threshold"}.get(post, effective)
        if effective != "none":
            raise AssertionError(f"STACRLowRankOnlyFunction received effective_residual_mode={effective}; "
                                 "B1 route is only valid when residuals are truly off.")
        in_features = weight.shape[1]
        leading = input_tensor.shape[:-1]
        x2d = input_tensor.reshape(-1, in_features)
        output = _dense_output(x2d, weight, bias).reshape(*leading, weight.shape[0])
        basis_c = basis if basis.dtype == x2d.dtype else basis.to(x2d.dtype)
        coeff, _, _, energy = save(x2d, basis_c, 0.0, 512)
        if not _is_recomputing():
            _record_energy(layer_state, energy.tolist(), basis_c.shape[1], coeff.shape[0], schedule_step)
        tensors = [coeff, weight] + ([bias] if bias is not None else [])
        ctx.cpu_offload = bool(config.get("cpu_offload", False)) and coeff.is_cuda
        if ctx.cpu_offload:
            tensors[0] = _offload(tensors[0])
        ctx.save_for_backward(*tensors)
        ctx.leading_shape, ctx.has_bias, ctx.quantize_coefficients = leading, bias is not None, False
        ctx.basis = _basis_for_backward(basis_c, basis)
        return output

    @staticmethod
    def backward(ctx, grad_output):
        saved = ctx.saved_tensors
        weight = saved[1]
        coefficients = _onload(saved[0], weight.device)
        bias = saved[2] if ctx.has_bias else None
        g2d = grad_output.reshape(-1, grad_output.shape[-1])
        return _factor_grads(ctx, g2d, weight, bias, coefficients, ctx.basis, None)


# ================================================================ the adaptive layer
class _TransposedProjection(nn.Module):
    """nn.Linear-shaped view of a Transformers Conv1D (weight kept as in x out): `.weight` is the
    transposed parameter, so gradients reach the Conv1D's own parameter."""

    def __init__(self, module: nn.Module):
        super().__init__()
        self.source_weight = module.weight
        self.bias = getattr(module, "bias", None)
        self.in_features, self.out_features = module.weight.shape

    @property
    def weight(self):
        return self.source_weight.t()

    def forward(self, x):
        flat = x.reshape(-1, self.in_features)
        out = flat.mm(self.source_weight) if self.bias is None else torch.addmm(self.bias, flat, self.source_weight)
        return out.reshape(*x.shape[:-1], self.out_features)


def _initial_layer_state(rank: int, effective_rank: int, base_rank: int, layer_index, num_layers: int,
                         budget: float) -> dict:
    """Monitoring / scheduling record of one adaptive layer (keys of stacr/adaptive.py:2807-2849)."""
    return {
        "last_residual_energy": 0.0, "step": 0, "basis_updates": 0, "skipped_updates": 0,
        "skipped_recompute": 0, "frozen_updates": 0, "refresh_count_total": 0, "refresh_count_by_reason": {},
        "microbatch_cache_hits": 0, "microbatch_cache_misses": 0, "b1_route_step_count": 0,
        "b1_generic_fallback_count": 0, "active_rank": rank, "allocated_rank": rank,
        "last_coeff_energy_by_rank": None, "rank_reason_code_counts": {}, "rank_trajectory": [],
        "last_rank_reason": "fixed", "_last_rank_adjust_step": -1, "b4_fused_kernel_route": "disabled",
        "b4_fused_kernel_route_counts": {}, "b4_numerical_parity_error": None, "optimizer_step": 0,
        "microbatch_index": 0, "accum_steps": 1, "effective_rank": effective_rank, "base_rank": base_rank,
        "layer_index": layer_index, "num_layers": num_layers, "total_steps": None,
        "current_residual_budget": budget,
    }


def _padded_orthonormal(leading: torch.Tensor, rank: int) -> torch.Tensor:
    """`leading` (features x m, m < rank) completed to `rank` orthonormal columns with random
    directions (QR of the concatenation)."""
    extra = torch.randn(leading.shape[0], rank - leading.shape[1], device=leading.device, dtype=leading.dtype)
    q, _ = torch.linalg.qr(torch.cat([leading, extra], dim=1))
    return q[:, :rank]


class STACRLinear(nn.Module):
    """The adaptive engine's layer (stacr/adaptive.py:2689-3727): a drop-in for nn.Linear whose
    saved input is C = X B plus a sparse residual.

    Each training forward: on the first one the basis is fitted to the batch (SVD; randomized SVD
    above `randomized_svd_threshold` features; random QR with `use_random_qr_init`; the
    "variance" rank mode picks the rank from the batch's spectrum first); the active prefix rank
    comes from the rank controller; the forward runs the low-rank-only Function when residuals
    are off and the STAC-R Function otherwise; afterwards the step counter advances and the basis
    may take one Oja step (HIP reduction + QR) when the update / refresh policy says so.
    Checkpoint recomputation replays the original forward's basis version and schedule step.
    """

    def __init__(self, in_features: int, out_features: int, config: Optional[STACRConfig] = None, bias: bool = True,
                 layer_index: Optional[int] = None, num_layers: int = 12):
        super().__init__()
        self.in_features, self.out_features = int(in_features), int(out_features)
        self.config = config or STACRConfig()
        self.linear = nn.Linear(self.in_features, self.out_features, bias=bias)
        base = self.config.rank
        self.effective_rank = (self.config.get_layer_rank(layer_index, base, num_layers)
                               if layer_index is not None and self.config.adaptive_layer_rank != "none" else base)
        rank = min(self.effective_rank, self.in_features)
        self.basis_dtype = _resolve_basis_dtype(self.config.basis_dtype)
        self.layer_index, self.num_layers = layer_index, num_layers
        # basis sharing (stacr/adaptive.py:2735-2792): the group from the explicit group or the layer
        # index; the layer then keeps no basis of its own and reads and writes the pool's
        self.use_basis_sharing, self.basis_group_id = False, None
        sharing = self.config.basis_sharing
        if sharing != "none":
            if self.config.rank_mode != "fixed":
                warnings.warn("basis_sharing only supports rank_mode='fixed'; disabling basis sharing "
                              f"for rank_mode={self.config.rank_mode!r}.")
            elif self.config.basis_sharing_group is not None:
                self.use_basis_sharing, self.basis_group_id = True, self.config.basis_sharing_group
            elif layer_index is None:
                warnings.warn("basis_sharing enabled but layer_index not provided, disabling sharing")
            elif sharing in _SHARING_GROUP:
                self.use_basis_sharing, self.basis_group_id = True, _SHARING_GROUP[sharing](layer_index)
            else:
                warnings.warn(f"Unknown basis_sharing mode: {sharing}, using 'none'")
        if self.use_basis_sharing:
            self.basis = None
        else:
            self.register_buffer("basis", torch.zeros(self.in_features, rank, dtype=self.basis_dtype))
        self.register_buffer("_basis_initialized", torch.zeros(1, dtype=torch.bool), persistent=True)
        self.register_buffer("step_counter", torch.zeros(1, dtype=torch.long))
        self.register_buffer("_runtime_state", torch.empty(0, dtype=torch.uint8))
        self.register_buffer("_shared_basis_state", torch.empty(0))
        self.layer_state = _initial_layer_state(rank, self.effective_rank, base, layer_index, num_layers,
                                                self.config.residual_budget)
        self._layer_id = id(self)

    @classmethod
    def from_linear(cls, module: nn.Module, config: Optional[STACRConfig] = None, *, layer_index=None,
                    num_layers: int = 12) -> "STACRLinear":
        """Wrap an nn.Linear or a Transformers Conv1D, keeping its parameters (and so the
        optimizer's references to them)."""
        conv1d = type(module).__name__ == "Conv1D" and getattr(module, "weight", None) is not None \
            and module.weight.dim() == 2
        if not (conv1d or isinstance(module, nn.Linear)):
            raise TypeError("Expected nn.Linear or Transformers Conv1D")
        in_f, out_f = module.weight.shape if conv1d else module.weight.shape[::-1]
        with torch.random.fork_rng(devices=[]):  # the placeholder nn.Linear must not move the caller's RNG
            layer = cls(in_f, out_f, copy.deepcopy(config), bias=getattr(module, "bias", None) is not None,
                        layer_index=layer_index, num_layers=num_layers)
        layer.to(module.weight.device)
        layer.linear = _TransposedProjection(module) if conv1d else module
        return layer.train(module.training)

    # ---------------------------------------------------------------- persistent state
    # Host mirrors of the one-element buffers step_counter and _basis_initialized, so the forward
    # does not read them back from the GPU: a mirror holds the value, the tensor and its in-place
    # version counter (host metadata), and is trusted only while both still match, so a write from
    # outside (fill_, load_state_dict's copy_, a move to another device) forces one fresh read.
    def _host_value(self, name: str):
        t = getattr(self, name)
        cached = self.__dict__.get("_host_" + name)
        if cached is not None and cached[1] is t and cached[2] == t._version:
            return cached[0]
        v = t.item()
        self.__dict__["_host_" + name] = (v, t, t._version)
        return v

    def _set_host_value(self, name: str, value) -> None:
        t = getattr(self, name)
        self.__dict__["_host_" + name] = (value, t, t._version)

    @property
    def basis_initialized(self) -> bool:
        return bool(self._host_value("_basis_initialized"))

    @basis_initialized.setter
    def basis_initialized(self, value: bool) -> None:
        self._basis_initialized.fill_(bool(value))
        self._set_host_value("_basis_initialized", bool(value))

    def _save_to_state_dict(self, destination, prefix, keep_vars):
        plain = {k: v for k, v in self.layer_state.items() if isinstance(v, (str, int, float, bool, list, dict,
                                                                             type(None)))}
        cfg = asdict(self.config)
        if isinstance(cfg["basis_dtype"], torch.dtype):
            cfg["basis_dtype"] = str(cfg["basis_dtype"])
        blob = json.dumps({"layer_state": plain, "config": cfg, "effective_rank": self.effective_rank}).encode()
        self._runtime_state = torch.tensor(list(blob), dtype=torch.uint8, device=self.step_counter.device)
        if self.use_basis_sharing and self.basis_initialized:
            self._shared_basis_state = self.effective_basis.detach()
        super()._save_to_state_dict(destination, prefix, keep_vars)

    def _load_from_state_dict(self, state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                              error_msgs):
        runtime_key, shared_key = prefix + "_runtime_state", prefix + "_shared_basis_state"
        blob = state_dict.get(runtime_key)
        if blob is not None and blob.numel():
            payload = json.loads(bytes(blob.cpu().tolist()).decode("utf-8"))
            self.layer_state.update(payload["layer_state"])
            self.config = STACRConfig(**payload["config"])
            self.effective_rank = payload["effective_rank"]
            self._runtime_state = torch.empty_like(blob, device=self.step_counter.device)
        else:
            state_dict[runtime_key] = self._runtime_state
        if shared_key in state_dict:
            shared = state_dict[shared_key]
            self._shared_basis_state = torch.empty_like(shared, device=self.step_counter.device)
            if shared.numel() and self.use_basis_sharing:
                get_basis_pool().update_basis(self.basis_group_id, self.in_features, shared.shape[1],
                                              shared.to(self.linear.weight.device))
        else:
            state_dict[shared_key] = self._shared_basis_state
        stored = state_dict.get(prefix + "basis")
        if stored is not None and self.basis is not None and stored.shape != self.basis.shape:
            self.basis = torch.empty_like(stored, device=self.basis.device)
        super()._load_from_state_dict(state_dict, prefix, local_metadata, strict, missing_keys, unexpected_keys,
                                      error_msgs)
        flag = prefix + "_basis_initialized"
        # checkpoints from before the flag existed: a non-zero stored basis means it was fitted
        if flag in missing_keys and stored is not None and stored.numel() and bool(torch.any(stored != 0)):
            self._basis_initialized.fill_(True)
            missing_keys.remove(flag)

    # ---------------------------------------------------------------- runtime scheduling
    def set_runtime_state(self, optimizer_step: Optional[int] = None, microbatch_index: int = 0,
                          accum_steps: int = 1) -> None:
        """Inject the training loop's optimizer step and micro-batch position."""
        st = self.layer_state
        if optimizer_step is None:
            st.pop("_optimizer_step_runtime", None)
        else:
            st["_optimizer_step_runtime"] = st["optimizer_step"] = int(optimizer_step)
        st["_microbatch_index_runtime"] = st["microbatch_index"] = int(microbatch_index)
        st["_accum_steps_runtime"] = st["accum_steps"] = max(1, int(accum_steps))

    def _use_optimizer_step_schedule(self) -> bool:
        c = self.config
        return bool(c.oja_update_per_optimizer_step or c.cache_basis_per_optimizer_step
                    or c.refresh_trigger != "off" or c.post_warmup_residual_mode != "full")

    def _get_schedule_step(self) -> int:
        runtime = self.layer_state.get("_optimizer_step_runtime") if self._use_optimizer_step_schedule() else None
        return int(runtime) if runtime is not None else int(self._host_value("step_counter"))

    _get_forward_schedule_step = _get_schedule_step

    def _get_microbatch_index(self) -> int:
        return int(self.layer_state.get("_microbatch_index_runtime", 0))

    def _get_accum_steps(self) -> int:
        return max(1, int(self.layer_state.get("_accum_steps_runtime", 1)))

    def _record_update_reason(self, reason: Optional[str]) -> None:
        if reason:
            self.layer_state["_pending_update_reason"] = reason

    def _consume_update_reason(self) -> Optional[str]:
        return self.layer_state.pop("_pending_update_reason", None)

    def _should_use_low_rank_only_route(self, schedule_step: int) -> bool:
        return self.config.enable_low_rank_only_fast_path and self._residual_off(schedule_step)

    def _residual_off(self, schedule_step: int) -> bool:
        c = self.config
        if schedule_step < c.warmup_steps or not self.basis_initialized:
            return False
        return c.residual_mode == "none" or (c.post_warmup_residual_mode == "none" and c.residual_warmup_steps > 0
                                             and schedule_step >= c.residual_warmup_steps)

    # ---------------------------------------------------------------- ranks
    def get_effective_rank(self) -> int:
        """The allocated basis rank (the configured rank until the basis is fitted)."""
        return self.basis.shape[1] if self.basis_initialized else min(self.effective_rank, self.in_features)

    def get_active_rank(self) -> int:
        active = self.layer_state.get("active_rank")
        return self.get_effective_rank() if active is None else max(1, min(int(active), self.get_effective_rank()))

    def _select_active_rank(self, schedule_step: int, allocated_rank: int) -> int:
        return select_active_rank(self.config.to_dict(), self.layer_state, schedule_step, allocated_rank,
                                  self.use_basis_sharing)

    @property
    def effective_basis(self) -> Optional[torch.Tensor]:
        """The layer's basis, or with sharing its group's basis from the pool."""
        if self.use_basis_sharing:
            return get_basis_pool().get_or_create_basis(self.basis_group_id, self.in_features, self._basis_rank(),
                                                        self.linear.weight.device, self.basis_dtype)
        return self.basis

    def _basis_rank(self) -> int:
        return self.basis.shape[1] if self.basis is not None else min(self.effective_rank, self.in_features)

    # ---------------------------------------------------------------- basis maintenance
    def _set_basis(self, basis: torch.Tensor) -> None:
        """Install `basis` as the layer's own, or with sharing as its group's."""
        if self.use_basis_sharing:
            get_basis_pool().update_basis(self.basis_group_id, self.in_features, basis.shape[1],
                                          basis.to(device=self.linear.weight.device, dtype=self.basis_dtype))
        else:
            self.basis = basis.to(device=self.basis.device, dtype=self.basis.dtype)

    def _install_basis(self, basis: torch.Tensor) -> None:
        self._set_basis(basis)
        self.basis_initialized = True
        allocated = basis.shape[1]
        self.layer_state["allocated_rank"] = allocated
        self.layer_state["active_rank"] = min(self.layer_state.get("active_rank", allocated), allocated)

    def _resize_basis(self, rank: int) -> None:
        fresh = torch.zeros(self.in_features, rank, dtype=self.basis_dtype, device=self.basis.device)
        self._buffers["basis"] = fresh

    def _init_basis_from_batch(self, input_2d: torch.Tensor) -> None:
        """Fit the basis to the first training batch (stacr/adaptive.py:3116-3309)."""
        cfg = self.config
        with torch.no_grad(), torch.autocast(device_type=input_2d.device.type, enabled=False):
            rows, feats = input_2d.shape
            target = self._basis_rank()
            if cfg.rank_mode == "variance" and cfg.use_random_qr_init:
                warnings.warn("rank_mode='variance' is incompatible with use_random_qr_init; "
                              "using configured rank for random-QR init.")
            elif cfg.rank_mode == "variance":
                if input_2d.numel() == 0:
                    warnings.warn("Empty batch during basis init, using rank_min")
                    chosen = cfg.rank_min
                else:
                    spectrum = profile_layer_spectrum(input_2d, threshold=cfg.rank_variance_threshold)
                    chosen = max(cfg.rank_min, min(spectrum["adaptive_rank"], cfg.rank_max))
                chosen = min(chosen, rows, feats)
                target = self.effective_rank = chosen
                self.layer_state.update(effective_rank=chosen, allocated_rank=chosen, active_rank=chosen)
                self._resize_basis(chosen)
            if cfg.use_random_qr_init:
                target = max(1, min(target, feats))
                draw = torch.randn(feats, target, device=input_2d.device,
                                   dtype=torch.float32 if self.basis_dtype in (torch.float16, torch.bfloat16)
                                   else self.basis_dtype)
                self._install_basis(torch.linalg.qr(draw)[0])
                return
            x = input_2d.float() if input_2d.dtype in (torch.float16, torch.bfloat16) else input_2d
            try:
                if feats > cfg.randomized_svd_threshold:
                    q = min(target + cfg.randomized_svd_oversampling, rows, feats)
                    _, _, v = torch.svd_lowrank(x, q=q, niter=cfg.randomized_svd_niter)
                    leading = v[:, :min(v.shape[1], target)]
                else:
                    vh = torch.linalg.svd(x, full_matrices=False)[2]
                    leading = vh[:min(vh.shape[0], target)].t()
            except RuntimeError as exc:
                warnings.warn(f"SVD failed for basis init ({exc}), using random orthonormal basis")
                self._install_basis(torch.linalg.qr(torch.randn(feats, target, device=x.device, dtype=x.dtype))[0])
                return
            if leading.shape[1] < target:
                leading = _padded_orthonormal(leading, target)
            self._install_basis(leading)

    def _should_update_basis(self) -> bool:
        return should_update_basis(self.config.to_dict(), self.layer_state, self._get_schedule_step(),
                                   self._get_microbatch_index(), self._get_accum_steps(), self.layer_index,
                                   self.num_layers)

    def _update_basis_oja(self, input_2d: torch.Tensor) -> None:
        """One Oja step on this batch (stacr_oja_step: Y = XB, X^T Y, Y^T Y in fp32 on the GPU), then
        QR, with the residual-energy-scaled rate when adaptive_oja_lr (stacr/adaptive.py:3311-3395)."""
        from . import kernels

        cfg, st = self.config, self.layer_state
        lr = cfg.oja_learning_rate
        if cfg.adaptive_oja_lr:
            lr = min(lr * (1.0 + st.get("last_residual_energy", 0.0) * cfg.adaptive_oja_scale), cfg.adaptive_oja_max_lr)
        with torch.no_grad(), torch.autocast(device_type=input_2d.device.type, enabled=False):
            rows = input_2d.detach()
            if rows.dtype not in kernels.DTYPE_CODES:
                rows = rows.float()
            current = self.effective_basis
            # Y = X B from this forward's save, when it was computed on this X and this basis
            given = st.pop("_oja_y", None)
            stepped = None
            if given is not None and given[1] is current and given[2].data_ptr() == rows.data_ptr() \
                    and given[2].shape == rows.shape:
                try:
                    _, stepped = kernels.oja_step_given_y(rows, current, given[0], float(lr))
                    st["oja_given_y_steps"] = st.get("oja_given_y_steps", 0) + 1
                except NotImplementedError:
                    stepped = None
            if stepped is None:
                _, stepped = kernels.oja_step(rows, current, float(lr))
            try:
                q, r = kernels.qr(stepped)
            except NotImplementedError:
                q, r = torch.linalg.qr(stepped)
            if cfg.use_mgs:  # Gram-Schmidt's factor has a positive diagonal: the same Q up to column signs
                q = q * torch.sign(torch.diagonal(r)).where(torch.diagonal(r) != 0, torch.ones_like(q[0]))
            self._set_basis(q[:, :current.shape[1]].to(self.basis_dtype))
        st["basis_updates"] += 1
        st["last_oja_lr"] = lr
        if cfg.cache_basis_per_optimizer_step and self._get_accum_steps() > 1:
            st["microbatch_cache_misses"] = st.get("microbatch_cache_misses", 0) + 1
        reason = self._consume_update_reason()
        if reason is not None:
            st["last_update_reason"] = reason
            if reason.startswith("refresh_"):
                st["refresh_count_total"] = st.get("refresh_count_total", 0) + 1
                by_reason = st.setdefault("refresh_count_by_reason", {})
                by_reason[reason] = int(by_reason.get(reason, 0)) + 1
                st["_last_refresh_schedule_step"] = self._get_schedule_step()
            else:
                st["_last_non_refresh_schedule_step"] = self._get_schedule_step()

    # ---------------------------------------------------------------- forward
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.training or not torch.is_grad_enabled() or not self.linear.weight.requires_grad \
                or x.numel() == 0:
            return self.linear(x)
        from .adaptive_checkpointing import get_global_recomputation_guard

        st, cfg = self.layer_state, self.config
        sparse_only = cfg.residual_mode == "sparse_only"
        guard = get_global_recomputation_guard()
        recomputing = guard.is_recomputing
        if (not sparse_only and not self.basis_initialized and self.use_basis_sharing
                and get_basis_pool().is_initialized(self.basis_group_id, self.in_features, self._basis_rank())):
            self.basis_initialized = True  # another member of the group fitted the shared basis
        if not sparse_only and not self.basis_initialized and not recomputing:
            self._init_basis_from_batch(x.reshape(-1, self.in_features))
        step_tensor = self.step_counter
        if recomputing:  # the counter already advanced past the forward being recomputed
            step_tensor = self.step_counter.new_tensor([max(int(self._host_value("step_counter")) - 1, 0)])
            st["skipped_recompute"] = st.get("skipped_recompute", 0) + 1
        schedule_step = self._get_forward_schedule_step()
        st["_schedule_step"] = schedule_step

        basis = None if sparse_only or not self.basis_initialized else self.effective_basis
        if basis is not None:
            allocated = basis.shape[1]
            st["allocated_rank"] = allocated
            if recomputing:
                active = max(1, min(int(st.get("active_rank", allocated)), allocated))
            elif cfg.rank_mode == "fixed":
                active = allocated
                st["last_rank_reason"] = "fixed"
            else:
                active = self._select_active_rank(schedule_step, allocated)
            if not recomputing:
                st["active_rank"] = active
            if active < allocated:
                basis = basis[:, :active]
        elif not recomputing:
            st["active_rank"] = self.get_effective_rank()

        replay = guard.replay_layer(self) if recomputing else None
        if replay is not None:
            basis, schedule_step, recorded = replay
            st["_schedule_step"] = schedule_step
            step_tensor = self.step_counter.new_tensor([recorded])
        elif not recomputing:
            guard.record_layer(self, (basis, schedule_step, int(self._host_value("step_counter"))))

        config_dict = cfg.to_dict()
        residual_off = basis is not None and not sparse_only and self._residual_off(schedule_step)
        st.pop("_oja_y", None)
        st.pop("_oja_y_request", None)
        if basis is not None and not recomputing and not residual_off and self.basis_initialized:
            outlook = basis_update_outlook(config_dict, schedule_step, self._get_microbatch_index(),
                                           self._get_accum_steps(), self.layer_index, self.num_layers)
            full = self.effective_basis
            # Y over more columns than the saved rank moves the save to its wide projection pass
            # (slower below 2048 features), so that is done only for a certain refresh
            if outlook == "certain" or (outlook == "maybe" and full.shape[1] == basis.shape[1]):
                st["_oja_y_request"] = full
        fast = residual_off and cfg.enable_low_rank_only_fast_path
        fn = STACRLowRankOnlyFunction if fast else STACRFunction
        output = fn.apply(x, self.linear.weight, self.linear.bias, basis, config_dict, step_tensor, st)
        if not recomputing:
            if fast:
                st["b1_route_step_count"] = st.get("b1_route_step_count", 0) + 1
            elif residual_off:
                st["b1_generic_fallback_count"] = st.get("b1_generic_fallback_count", 0) + 1
            steps = int(self._host_value("step_counter"))
            self.step_counter += 1
            self._set_host_value("step_counter", steps + 1)
            if not sparse_only and self.basis_initialized and self._should_update_basis():
                self._update_basis_oja(x.reshape(-1, self.in_features))
        return output

    def extra_repr(self) -> str:
        out = f"in_features={self.in_features}, out_features={self.out_features}, rank={self.config.rank}"
        if self.config.rank_mode != "fixed":
            out += f", rank_mode={self.config.rank_mode}"
            if self.basis_initialized and self.get_effective_rank() != self.config.rank:
                out += f", effective_rank={self.get_effective_rank()}"
            if self.basis_initialized and self.get_active_rank() != self.get_effective_rank():
                out += f", active_rank={self.get_active_rank()}"
        return out + f", residual_mode={self.config.residual_mode}, update_interval={self.config.update_interval}"


# ================================================================ model-level API
def set_stacr_runtime_state(model: nn.Module, optimizer_step: int, microbatch_index: int = 0,
                            accum_steps: int = 1) -> None:
    """Hand the optimizer step and micro-batch position to every adaptive layer of `model`
    (stacr/adaptive.py:3730-3744)."""
    for module in model.modules():
        if isinstance(module, STACRLinear):
            module.set_runtime_state(optimizer_step=optimizer_step, microbatch_index=microbatch_index,
                                     accum_steps=accum_steps)


_ADAPTIVE_SELECTION = ("surface", "min_features", "target_names", "target_pattern", "extra_names", "exclude_names",
                       "trainable_only")


def apply_adaptive_stacr(model: nn.Module, config=None, **options) -> list:
    """Wrap the selected projections of `model` with adaptive layers in place and return them
    (stacr/adaptive.py:3839-3902).  Takes a STACRConfig or a dict plus overrides; selection options
    are apply_stacr's.  Every layer is built before the model is touched."""
    from .surgery import select_target_names

    values = asdict(config) if isinstance(config, STACRConfig) else dict(config or {})
    values.update(options)
    selection = {k: values.pop(k) for k in _ADAPTIVE_SELECTION if k in values}
    allow_empty = values.pop("allow_empty", False)
    cfg = STACRConfig(**values)
    if cfg.joint_qk:
        raise ValueError("joint_qk requires the attention protocol adapter; it is not a generic linear "
                         "selection option")
    if not cfg.use_random_qr_init and (cfg.allow_unadapted_random_qr or cfg.min_adaptation_steps != 50):
        raise ValueError("Random-QR adaptation controls require use_random_qr_init=True")
    if cfg.use_random_qr_init and not cfg.allow_unadapted_random_qr and cfg.freeze_basis_after_warmup \
            and cfg.warmup_steps < cfg.min_adaptation_steps:
        raise ValueError("Random-QR initialization needs warmup_steps >= min_adaptation_steps before freezing; "
                         "set allow_unadapted_random_qr=True for an explicit random-basis control")
    names = select_target_names(model, **selection)
    if "" in names:
        raise ValueError("Use AdaptiveSTACRLinear.from_linear(model, config) for a standalone module")
    if not names and not allow_empty and selection.get("surface") != "none":
        raise ValueError("No trainable projections matched the adaptive STAC-R selection")
    built: dict[int, STACRLinear] = {}
    plan = []
    for index, name in enumerate(names):
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name)
        module = getattr(parent, leaf)
        if id(module) not in built:
            layer = STACRLinear.from_linear(module, cfg, layer_index=index, num_layers=len(names))
            layer.source_name = name
            built[id(module)] = layer
        plan.append((parent, leaf, built[id(module)]))
    for parent, leaf, layer in plan:
        setattr(parent, leaf, layer)
    return list(built.values())


AdaptiveSTACRConfig = STACRConfig
AdaptiveSTACRLinear = STACRLinear
