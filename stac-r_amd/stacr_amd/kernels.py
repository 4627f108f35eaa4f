"""Tensor-level calls into the HIP library (PyTorch supplies device memory and the stream).

Every function here requires ROCm GPU tensors and raises otherwise: the save and weight-gradient
arithmetic has no CPU implementation in this package.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib

DTYPE_CODES = {torch.float32: _lib.DTYPE_F32, torch.bfloat16: _lib.DTYPE_BF16, torch.float16: _lib.DTYPE_F16}
MODE_CODES = {"chunk_topk": _lib.MODE_CHUNK_TOPK, "topk": _lib.MODE_CHUNK_TOPK,
              "global_topk": _lib.MODE_GLOBAL_TOPK}


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"stacr_amd supports float32, bfloat16 and float16 tensors, got {dtype}") from None


def require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"stacr_amd: {name} must be a ROCm GPU tensor; the save/backward path runs only in the "
            f"HIP kernels (got device {t.device})"
        )


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr() if t is not None and t.numel() else None)


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def residual_plan(rows: int, feats: int, mode: str, budget: float, chunk_rows: int):
    """(k_total, k_saved, index_bytes) per the reference's k rules (stacr/layers.py:25-27,33,51-53)."""
    if mode not in MODE_CODES:
        raise ValueError(f"residual_mode {mode!r} has no HIP selection kernel")
    kt, ks, ib = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int()
    L = _lib.load()
    _lib.check(L.stacr_residual_plan(int(rows), int(feats), MODE_CODES[mode], float(budget), int(chunk_rows),
                                     ctypes.byref(kt), ctypes.byref(ks), ctypes.byref(ib)), "stacr_residual_plan")
    return int(kt.value), int(ks.value), int(ib.value)


def _outputs(k: int, bits: int, dtype: torch.dtype, index_bytes: int, device):
    idx = torch.empty(k, dtype=torch.int32 if index_bytes == 4 else torch.int64, device=device)
    if bits == 8:
        data = torch.empty(k, dtype=torch.int8, device=device)
    elif bits == 4:
        data = torch.empty((k + 1) // 2, dtype=torch.uint8, device=device)
    else:
        data = torch.empty(k, dtype=dtype, device=device)
    scale = torch.empty((), dtype=torch.float32, device=device)
    return idx, data, scale


def save(x2d: torch.Tensor, q: torch.Tensor, *, mode: str, budget: float, chunk_rows: int, bits: int,
         coeff: torch.Tensor | None = None):
    """One save pass.  Returns (coeff, idx, data, scale); the last three are None without residual.

    x2d: rows x feats activation (cast to the compute dtype), q: feats x rank basis in that dtype.
    With ``coeff`` given, only selection and quantization run (stacr_select_residual).
    """
    return _save(x2d, q, mode, budget, chunk_rows, bits, coeff, False)[:4]


def save_with_census(x2d: torch.Tensor, q: torch.Tensor, *, mode: str, budget: float, chunk_rows: int, bits: int):
    """save() plus the entry census the weight gradient can take instead of counting the entries
    (stacr_save_census): (coeff, idx, data, scale, census or None when this save writes none)."""
    return _save(x2d, q, mode, budget, chunk_rows, bits, None, True)


def _save(x2d, q, mode, budget, chunk_rows, bits, coeff, want_census):
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    q = q.contiguous()
    if q.dtype != x2d.dtype:
        raise TypeError("basis must be cast to the activation dtype")
    rows, feats = x2d.shape
    rank = q.shape[1]
    dt = dtype_code(x2d.dtype)
    k_total, k_saved, ib = residual_plan(rows, feats, mode, budget, chunk_rows)
    device = x2d.device
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_save_workspace_bytes(rows, feats, rank, dt, MODE_CODES[mode], float(budget),
                                            int(chunk_rows), int(bits), ctypes.byref(ws_bytes)), "stacr_save")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
    stream = _stream(device)
    if k_total > 0:
        idx, data, scale = _outputs(k_saved, bits, x2d.dtype, ib, device)
    else:
        idx = data = scale = None
    census = None
    if coeff is None and want_census and k_total > 0:
        coeff = torch.empty(rows, rank, dtype=x2d.dtype, device=device)
        cb = ctypes.c_size_t()
        _lib.check(L.stacr_save_census_bytes(rows, feats, ctypes.byref(cb)), "stacr_save_census_bytes")
        census = torch.empty(cb.value // 4, dtype=torch.int32, device=device)
        written = ctypes.c_int(0)
        _lib.check(L.stacr_save_census(_ptr(x2d), _ptr(q), dt, rows, feats, rank, MODE_CODES[mode], float(budget),
                                       int(chunk_rows), int(bits), _ptr(coeff), _ptr(idx), ib, _ptr(data),
                                       _ptr(scale), _ptr(ws), ws_bytes.value, _ptr(census), cb.value,
                                       ctypes.byref(written), stream), "stacr_save_census")
        if not written.value:
            census = None
    elif coeff is None:
        coeff = torch.empty(rows, rank, dtype=x2d.dtype, device=device)
        _lib.check(L.stacr_save(_ptr(x2d), _ptr(q), dt, rows, feats, rank, MODE_CODES[mode], float(budget),
                                int(chunk_rows), int(bits), _ptr(coeff), _ptr(idx), ib, _ptr(data), _ptr(scale),
                                _ptr(ws), ws_bytes.value, stream), "stacr_save")
    else:
        coeff = coeff.contiguous()
        if k_total > 0:
            _lib.check(L.stacr_select_residual(_ptr(x2d), _ptr(coeff), _ptr(q), dt, rows, feats, rank,
                                               MODE_CODES[mode], float(budget), int(chunk_rows), int(bits),
                                               _ptr(idx), ib, _ptr(data), _ptr(scale), _ptr(ws), ws_bytes.value,
                                               stream), "stacr_select_residual")
    return coeff, idx, data, scale, census


def _factor_args(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor):
    require_gpu(x2d, "activation")
    x2d, coeff, q = x2d.contiguous(), coeff.contiguous(), q.contiguous()
    if coeff.dtype != x2d.dtype or q.dtype != x2d.dtype:
        raise TypeError("coefficients and basis must be cast to the activation dtype")
    rows, feats = x2d.shape
    total = rows * feats
    ib = 4 if total < 2**31 - 1 else 8
    return x2d, coeff, q, rows, feats, q.shape[1], dtype_code(x2d.dtype), ib


def _index_tensor(n: int, ib: int, device):
    return torch.empty(n, dtype=torch.int32 if ib == 4 else torch.int64, device=device)


def select_uniform(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, k: int):
    """(idx, values) of the "uniform" selector: positions floor(i * total / k) (stacr/layers.py:89-98)."""
    x2d, coeff, q, rows, feats, rank, dt, ib = _factor_args(x2d, coeff, q)
    idx = _index_tensor(k, ib, x2d.device)
    values = torch.empty(k, dtype=x2d.dtype, device=x2d.device)
    _lib.check(_lib.load().stacr_select_uniform(_ptr(x2d), _ptr(coeff), _ptr(q), dt, rows, feats, rank, int(k),
                                                _ptr(idx), ib, _ptr(values), _stream(x2d.device)),
               "stacr_select_uniform")
    return idx, values


def select_block_sparse(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, budget: float, chunk_rows: int,
                        block_size: int):
    """(idx, values) of the "block_sparse" selector (stacr/layers.py:81-88); feats % block_size == 0."""
    x2d, coeff, q, rows, feats, rank, dt, ib = _factor_args(x2d, coeff, q)
    L = _lib.load()
    cf, cl, n, ws_bytes = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64(), ctypes.c_size_t()
    _lib.check(L.stacr_block_sparse_plan(rows, feats, float(budget), int(chunk_rows), int(block_size), ctypes.byref(cf),
                                         ctypes.byref(cl), ctypes.byref(n), ctypes.byref(ws_bytes)),
               "stacr_block_sparse_plan")
    idx = _index_tensor(n.value, ib, x2d.device)
    values = torch.empty(n.value, dtype=x2d.dtype, device=x2d.device)
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=x2d.device)
    _lib.check(L.stacr_select_block_sparse(_ptr(x2d), _ptr(coeff), _ptr(q), dt, rows, feats, rank, float(budget),
                                           int(chunk_rows), int(block_size), _ptr(idx), ib, _ptr(values), _ptr(ws),
                                           ws_bytes.value, _stream(x2d.device)), "stacr_select_block_sparse")
    return idx, values


def sample_magnitudes(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, positions: torch.Tensor):
    """|r| at the given flat positions (int64), in the activation dtype."""
    x2d, coeff, q, rows, feats, rank, dt, _ = _factor_args(x2d, coeff, q)
    positions = positions.to(device=x2d.device, dtype=torch.int64).contiguous()
    out = torch.empty(positions.numel(), dtype=x2d.dtype, device=x2d.device)
    _lib.check(_lib.load().stacr_sample_magnitudes(_ptr(x2d), _ptr(coeff), _ptr(q), dt, rows, feats, rank,
                                                   _ptr(positions), positions.numel(), _ptr(out),
                                                   _stream(x2d.device)), "stacr_sample_magnitudes")
    return out


def select_sampled(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, budget: float, sample_ratio: float,
                   k_total: int):
    """(idx, values) of the "sampled" selector (stacr/layers.py:55-66).

    The sample positions come from torch.randint with the reference's seeded generator on the
    activation's device and the threshold from torch.quantile (library calls, as in the
    reference); the magnitude gather and the ordered, capped compaction are HIP kernels.  One
    device-to-host read of the selected count sizes the outputs (the reference's nonzero syncs
    the same way).
    """
    x2d, coeff, q, rows, feats, _, _, _ = _factor_args(x2d, coeff, q)
    device = x2d.device
    total = rows * feats
    generator = torch.Generator(device=device).manual_seed(0)
    sample_n = max(1024, int(total * sample_ratio))
    positions = torch.randint(total, (sample_n,), device=device, generator=generator)
    sample = sample_magnitudes(x2d, coeff, q, positions)
    threshold = torch.quantile(sample.float(), 1.0 - budget)
    return select_threshold(x2d, coeff, q, threshold, k_total)


def select_threshold(x2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, threshold: torch.Tensor,
                     cap: int | None):
    """The first ``cap`` flat positions with |r| >= threshold (an fp32 device scalar, compared in
    the activation dtype), ascending, with their residual values.  ``cap`` None selects every
    passing position (a count-only call sizes the outputs first)."""
    x2d, coeff, q, rows, feats, rank, dt, ib = _factor_args(x2d, coeff, q)
    device = x2d.device
    L = _lib.load()
    threshold = threshold.to(device=device, dtype=torch.float32).reshape(()).contiguous()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_threshold_workspace_bytes(rows, feats, ctypes.byref(ws_bytes)), "stacr_threshold_workspace_bytes")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
    count = torch.zeros((), dtype=torch.int64, device=device)

    def call(c, idx, values):
        _lib.check(L.stacr_select_threshold(_ptr(x2d), _ptr(coeff), _ptr(q), dt, rows, feats, rank, _ptr(threshold),
                                            int(c), _ptr(idx), ib, _ptr(values), _ptr(count), _ptr(ws),
                                            ws_bytes.value, _stream(device)), "stacr_select_threshold")
        return int(count.item())

    if cap is None:
        cap = call(0, None, None)  # cap 0: the count of every passing entry, nothing written
    if cap == 0:
        return _index_tensor(0, ib, device), torch.empty(0, dtype=x2d.dtype, device=device)
    idx = _index_tensor(cap, ib, device)
    values = torch.empty(cap, dtype=x2d.dtype, device=device)
    n = min(call(cap, idx, values), cap)
    if n < cap:
        idx, values = idx[:n].clone(), values[:n].clone()
    return idx, values


def quantize(values: torch.Tensor, bits: int):
    """(data, scale) of quantize_values for bits 4/8 (stacr/quant.py:49-65)."""
    require_gpu(values, "values")
    flat = values.reshape(-1).contiguous()
    n = flat.numel()
    data = torch.empty(n if bits == 8 else (n + 1) // 2, dtype=torch.int8 if bits == 8 else torch.uint8,
                       device=flat.device)
    scale = torch.empty((), dtype=torch.float32, device=flat.device)
    ws = torch.empty(4, dtype=torch.uint8, device=flat.device)
    L = _lib.load()
    _lib.check(L.stacr_quantize_values(_ptr(flat), dtype_code(flat.dtype), n, int(bits), _ptr(data), _ptr(scale),
                                       _ptr(ws), 4, _stream(flat.device)), "stacr_quantize_values")
    return data, scale


def oja_step(x2d: torch.Tensor, q: torch.Tensor, lr: float):
    """One Oja step in fp32 (stacr/layers.py:346-348, stacr/oja.py:73-79).

    x2d: rows x feats activation in its own dtype; q: feats x rank basis (cast to fp32 here).
    Returns (update, out) with update = X^T Y / N - Q (Y^T Y / N), Y = X Q, out = Q + lr * update,
    both feats x rank fp32.  The caller re-orthonormalizes ``out``.
    """
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    q32 = q.to(device=x2d.device, dtype=torch.float32).contiguous()
    rows, feats = x2d.shape
    rank = q32.shape[1]
    if q32.shape[0] != feats:
        raise ValueError(f"basis has {q32.shape[0]} rows, activation has {feats} features")
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_oja_workspace_bytes(rows, feats, rank, ctypes.byref(ws_bytes)), "stacr_oja_workspace_bytes")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=x2d.device)
    update = torch.empty(feats, rank, dtype=torch.float32, device=x2d.device)
    out = torch.empty_like(update)
    _lib.check(L.stacr_oja_step(_ptr(x2d), dtype_code(x2d.dtype), rows, feats, _ptr(q32), rank, float(lr),
                                _ptr(update), _ptr(out), _ptr(ws), ws_bytes.value, _stream(x2d.device)),
               "stacr_oja_step")
    return update, out


def oja_step_given_y(x2d: torch.Tensor, q: torch.Tensor, y: torch.Tensor, lr: float):
    """oja_step with Y = X Q supplied (rows x rank fp32, e.g. the save's own projection), so X is
    read once (stacr_oja_step_given_y).  Raises NotImplementedError for shapes the one-pass form
    does not take (see the header); oja_step serves those."""
    require_gpu(x2d, "activation")
    x2d = x2d.contiguous()
    q32 = q.to(device=x2d.device, dtype=torch.float32).contiguous()
    rows, feats = x2d.shape
    rank = q32.shape[1]
    if q32.shape[0] != feats:
        raise ValueError(f"basis has {q32.shape[0]} rows, activation has {feats} features")
    if y.shape != (rows, rank) or y.dtype != torch.float32:
        raise ValueError(f"Y must be {rows} x {rank} fp32, got {tuple(y.shape)} {y.dtype}")
    y = y.contiguous()
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_oja_workspace_bytes(rows, feats, rank, ctypes.byref(ws_bytes)), "stacr_oja_workspace_bytes")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=x2d.device)
    update = torch.empty(feats, rank, dtype=torch.float32, device=x2d.device)
    out = torch.empty_like(update)
    _lib.check(L.stacr_oja_step_given_y(_ptr(x2d), dtype_code(x2d.dtype), rows, feats, _ptr(q32), rank, _ptr(y),
                                        float(lr), _ptr(update), _ptr(out), _ptr(ws), ws_bytes.value,
                                        _stream(x2d.device)), "stacr_oja_step_given_y")
    return update, out


# rows * cols up to which the one-workgroup kernel (stacr_qr, limit 32768) runs; larger matrices take
# stacr_qr_tall, which is faster from here on (measured: 2048 x 16 in 33 us against 58 us)
QR_REGISTER_ELEMS = 8192


def qr(a: torch.Tensor):
    """Reduced QR (Q, R) of a tall GPU matrix in fp32, LAPACK's sign convention (as
    torch.linalg.qr): one workgroup (stacr_qr) up to 8192 elements, the tall route (stacr_qr_tall:
    fp64 CholeskyQR with LAPACK's signs, or LAPACK's Householder QR where that is not exact enough)
    past it.  Raises NotImplementedError for more than 16 columns."""
    require_gpu(a, "matrix")
    if a.dim() != 2:
        raise ValueError(f"qr takes a matrix, got {a.dim()} dimensions")
    rows, cols = a.shape
    if cols > rows:
        raise ValueError(f"qr takes a tall matrix, got {rows} x {cols}")
    if cols > 16:
        raise NotImplementedError(f"qr: {cols} columns (at most 16)")
    a32 = a.to(torch.float32).contiguous()
    q = torch.empty_like(a32)
    r = torch.empty(cols, cols, dtype=torch.float32, device=a.device)
    L = _lib.load()
    if rows * cols <= QR_REGISTER_ELEMS:
        _lib.check(L.stacr_qr(_ptr(a32), rows, cols, _ptr(q), _ptr(r), _stream(a.device)), "stacr_qr")
        return q, r
    wsb = ctypes.c_size_t()
    _lib.check(L.stacr_qr_tall_workspace_bytes(rows, cols, ctypes.byref(wsb)), "stacr_qr_tall")
    ws = torch.empty(wsb.value, dtype=torch.uint8, device=a.device)
    _lib.check(L.stacr_qr_tall(_ptr(a32), rows, cols, _ptr(q), _ptr(r), _ptr(ws), wsb.value, _stream(a.device)),
               "stacr_qr_tall")
    return q, r


def weight_grad(g2d: torch.Tensor, coeff: torch.Tensor, q: torch.Tensor, residual, bits: int, transposed: bool,
                out_dtype: torch.dtype, bias_dtype: torch.dtype | None = None, census: torch.Tensor | None = None):
    """dW (and dbias when bias_dtype is given) from the saved factors (stacr/layers.py:172-198).

    ``residual`` is None or (idx, data, scale); ``coeff`` and ``q`` are cast to G's dtype first, as
    the reference does.  dW is d_out x d_in, or d_in x d_out when ``transposed``.  ``census``: the
    entry census save_with_census returned with this residual (the same dW, one launch fewer).
    """
    require_gpu(g2d, "grad_output")
    g2d = g2d.contiguous()
    rows, d_out = g2d.shape
    d_in, rank = q.shape
    dt = dtype_code(g2d.dtype)
    coeff = coeff.to(g2d.dtype).contiguous()
    q = q.to(g2d.dtype).contiguous()
    device = g2d.device
    if residual is not None and residual[0].numel():
        idx, data, scale = residual
        nnz = idx.numel()
        ib = idx.element_size()
        vdt = dtype_code(data.dtype) if bits == 0 else 0
    else:
        idx = data = scale = None
        nnz, ib, vdt = 0, 4, 0
    dw = torch.empty((d_in, d_out) if transposed else (d_out, d_in), dtype=out_dtype, device=device)
    db = torch.empty(d_out, dtype=bias_dtype, device=device) if bias_dtype is not None else None
    L = _lib.load()
    ws_bytes = ctypes.c_size_t()
    _lib.check(L.stacr_weight_grad_workspace_bytes(rows, d_out, d_in, rank, nnz, ctypes.byref(ws_bytes)),
               "stacr_weight_grad")
    ws = torch.empty(max(1, ws_bytes.value), dtype=torch.uint8, device=device)
    if census is not None and nnz:
        _lib.check(L.stacr_weight_grad_census(_ptr(g2d), dt, rows, d_out, _ptr(coeff), _ptr(q), d_in, rank, _ptr(idx),
                                              ib, _ptr(data), _ptr(scale), int(bits), vdt, nnz,
                                              1 if transposed else 0, _ptr(dw), dtype_code(out_dtype), _ptr(db),
                                              dtype_code(bias_dtype) if db is not None else 0, _ptr(census),
                                              census.numel() * census.element_size(), _ptr(ws),
                                              ws_bytes.value, _stream(device)), "stacr_weight_grad_census")
        return dw, db
    _lib.check(L.stacr_weight_grad(_ptr(g2d), dt, rows, d_out, _ptr(coeff), _ptr(q), d_in, rank, _ptr(idx), ib,
                                   _ptr(data), _ptr(scale), int(bits), vdt, nnz, 1 if transposed else 0, _ptr(dw),
                                   dtype_code(out_dtype), _ptr(db), dtype_code(bias_dtype) if db is not None else 0,
                                   _ptr(ws), ws_bytes.value, _stream(device)), "stacr_weight_grad")
    return dw, db


def reconstruct(coeff: torch.Tensor, q: torch.Tensor, residual=None) -> torch.Tensor:
    """rnd(coeff Q^T) + the dense residual, in coeff's dtype (stacr/compressor.py:127-133,
    stacr/residual.py:13-20).

    ``residual`` is None or (flat indices, values); with a residual every element gets the
    addition (zeros away from the entries), as the reference adds the dense tensor.
    """
    require_gpu(coeff, "coefficients")
    coeff = coeff.contiguous()
    rows, rank = coeff.shape
    feats = q.shape[0]
    if q.shape[1] != rank:
        raise ValueError(f"basis has rank {q.shape[1]}, coefficients {rank}")
    q = q.to(coeff.dtype).contiguous()
    dt = dtype_code(coeff.dtype)
    out = torch.empty(rows, feats, dtype=coeff.dtype, device=coeff.device)
    idx = values = None
    nnz, ib = 0, 4
    if residual is not None:
        idx, values = residual
        nnz = idx.numel()
        if nnz:
            if idx.dtype not in (torch.int32, torch.int64):
                idx = idx.to(torch.int64)
            idx = idx.contiguous()
            ib = idx.element_size()
            values = values.to(coeff.dtype).contiguous()
            if values.numel() != nnz:
                raise ValueError("residual indices and values differ in length")
    L = _lib.load()
    _lib.check(L.stacr_reconstruct(_ptr(coeff), _ptr(q), dt, rows, feats, rank, _ptr(idx) if nnz else None, ib,
                                   _ptr(values) if nnz else None, nnz, 1 if residual is not None else 0, _ptr(out),
                                   _stream(coeff.device)), "stacr_reconstruct")
    return out


def index_stream_encode(idx: torch.Tensor):
    """Bit-packed delta stream of sorted flat indices (blocks of 256, one bit width per block).

    Returns (base int64[nb], word_off int32[nb + 1], words int32[256 nb], status int32[1]); the
    int32 tensors hold uint32 bit patterns, words[:word_off[nb]] is the stream, and a nonzero
    status means the input was not non-decreasing and non-negative with gaps below 2^32.
    """
    require_gpu(idx, "indices")
    if idx.dtype not in (torch.int32, torch.int64):
        raise TypeError(f"indices must be int32 or int64, got {idx.dtype}")
    idx = idx.contiguous().reshape(-1)
    nnz = idx.numel()
    L = _lib.load()
    nb, mw = ctypes.c_int64(), ctypes.c_int64()
    _lib.check(L.stacr_index_stream_sizes(nnz, ctypes.byref(nb), ctypes.byref(mw)), "stacr_index_stream_sizes")
    dev = idx.device
    base = torch.empty(nb.value, dtype=torch.int64, device=dev)
    word_off = torch.empty(nb.value + 1, dtype=torch.int32, device=dev)
    words = torch.empty(mw.value, dtype=torch.int32, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    _lib.check(L.stacr_index_stream_encode(_ptr(idx) if nnz else None, idx.element_size(), nnz,
                                           _ptr(base) if nnz else None, _ptr(word_off), _ptr(words) if nnz else None,
                                           _ptr(status), _stream(dev)), "stacr_index_stream_encode")
    return base, word_off, words, status


def index_stream_decode(base: torch.Tensor, word_off: torch.Tensor, words: torch.Tensor, nnz: int,
                        dtype: torch.dtype = torch.int32) -> torch.Tensor:
    """The sorted flat indices of a stream from index_stream_encode, as int32 or int64."""
    if dtype not in (torch.int32, torch.int64):
        raise TypeError(f"indices decode to int32 or int64, not {dtype}")
    dev = word_off.device
    require_gpu(word_off, "stream offsets")
    out = torch.empty(int(nnz), dtype=dtype, device=dev)
    if nnz == 0:
        return out
    if words.numel() == 0:  # every block of width 0 (a stream of no words); the library wants a buffer
        words = torch.zeros(1, dtype=torch.int32, device=dev)
    L = _lib.load()
    _lib.check(L.stacr_index_stream_decode(_ptr(base.contiguous()), _ptr(word_off.contiguous()),
                                           _ptr(words.contiguous()), int(nnz), _ptr(out), out.element_size(),
                                           _stream(dev)), "stacr_index_stream_decode")
    return out


def quantize_rows_int8(coeff: torch.Tensor):
    """(int8 codes rows x rank, fp32 scales[rows]): one scale per row, s = safe max |c| / 127."""
    require_gpu(coeff, "coefficients")
    if coeff.dim() != 2:
        raise ValueError(f"coefficients must be rows x rank, got shape {tuple(coeff.shape)}")
    coeff = coeff.contiguous()
    rows, rank = coeff.shape
    codes = torch.empty(rows, rank, dtype=torch.int8, device=coeff.device)
    scales = torch.empty(rows, dtype=torch.float32, device=coeff.device)
    if rows and rank:
        L = _lib.load()
        _lib.check(L.stacr_quantize_rows_int8(_ptr(coeff), dtype_code(coeff.dtype), rows, rank, _ptr(codes),
                                              _ptr(scales), _stream(coeff.device)), "stacr_quantize_rows_int8")
    return codes, scales


def dequantize_rows_int8(codes: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """codes * scale[row] in fp32, rounded once to ``dtype``."""
    require_gpu(codes, "codes")
    if codes.dtype != torch.int8 or scales.dtype != torch.float32:
        raise TypeError("codes must be int8 and scales float32")
    codes = codes.contiguous()
    rows, rank = codes.shape
    out = torch.empty(rows, rank, dtype=dtype, device=codes.device)
    if rows and rank:
        L = _lib.load()
        _lib.check(L.stacr_dequantize_rows_int8(_ptr(codes), _ptr(scales.contiguous()), rows, rank, _ptr(out),
                                                dtype_code(dtype), _stream(codes.device)), "stacr_dequantize_rows_int8")
    return out


# ------------------------------------------------------------------ C1 checkpoint-boundary codec
C1_STATS_BYTES = 48
C1_FLAGS = {"input_nan": 1, "coeff_nan": 2, "recon_nan": 4, "basis_nan": 8, "input_valid": 16, "coeff_valid": 32,
            "recon_valid": 64, "residual_valid": 128, "basis_valid": 256, "residual_nan": 512}
DTYPE_I8 = 3


def c1_observe(x2d: torch.Tensor, coeff: torch.Tensor, basis: torch.Tensor):
    """One pass over the boundary X (rows x hidden) with its fp32 coefficients and the basis:
    (stats uint8[48] on the device, fp32 scales[rank]); parse the stats with c1_parse_stats."""
    require_gpu(x2d, "boundary activation")
    if coeff.dtype != torch.float32:
        raise TypeError("C1 coefficients are fp32")
    x2d, coeff, basis = x2d.contiguous(), coeff.contiguous(), basis.contiguous()
    rows, hidden = x2d.shape
    rank = basis.shape[1]
    if coeff.shape != (rows, rank) or basis.shape[0] != hidden:
        raise ValueError("C1 shapes: x rows x hidden, coeff rows x rank, basis hidden x rank")
    L = _lib.load()
    nbytes = ctypes.c_size_t()
    _lib.check(L.stacr_c1_workspace_bytes(rows, hidden, rank, ctypes.byref(nbytes)), "stacr_c1_workspace_bytes")
    dev = x2d.device
    ws = torch.empty(max(1, nbytes.value), dtype=torch.uint8, device=dev)
    stats = torch.empty(C1_STATS_BYTES, dtype=torch.uint8, device=dev)
    scales = torch.empty(rank, dtype=torch.float32, device=dev)
    _lib.check(L.stacr_c1_observe(_ptr(x2d), dtype_code(x2d.dtype), rows, hidden, _ptr(coeff), _ptr(basis),
                                  dtype_code(basis.dtype), rank, _ptr(stats), _ptr(scales), _ptr(ws), nbytes.value,
                                  _stream(dev)), "stacr_c1_observe")
    return stats, scales


def c1_parse_stats(raw) -> dict:
    """The StacrC1Stats record (48 bytes, host copy) as a dict."""
    import struct

    b = bytes(raw.cpu().numpy().tobytes()) if isinstance(raw, torch.Tensor) else bytes(raw)
    err, denom, energy, xm, cm, rm, em, bm, flags, _ = struct.unpack("<ddffffffII", b[:C1_STATS_BYTES])
    return {"error": err, "denom": denom, "energy": energy, "input_max_abs": xm, "coeff_max_abs": cm,
            "reconstruction_max_abs": rm, "residual_max_abs": em, "basis_max_abs": bm, "flags": flags}


def c1_store(coeff: torch.Tensor, scales: torch.Tensor | None, quantize: bool, dtype: torch.dtype) -> torch.Tensor:
    """The record's coefficients: int8 codes with the per-component scales, or C in ``dtype``."""
    require_gpu(coeff, "coefficients")
    coeff = coeff.contiguous()
    rows, rank = coeff.shape
    out = torch.empty(rows, rank, dtype=torch.int8 if quantize else dtype, device=coeff.device)
    L = _lib.load()
    _lib.check(L.stacr_c1_store(_ptr(coeff), rows, rank, _ptr(scales) if quantize else None, 1 if quantize else 0,
                                _ptr(out), DTYPE_I8 if quantize else dtype_code(dtype), _stream(coeff.device)),
               "stacr_c1_store")
    return out


def c1_restore(coeff: torch.Tensor, scales: torch.Tensor | None, basis: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """sum_j c'_j q_j in fp32 rounded once to ``dtype`` (c' = code * scale for int8 coefficients)."""
    require_gpu(coeff, "coefficients")
    coeff, basis = coeff.contiguous(), basis.contiguous()
    rows, rank = coeff.shape
    hidden = basis.shape[0]
    out = torch.empty(rows, hidden, dtype=dtype, device=coeff.device)
    quant = coeff.dtype == torch.int8
    if quant and scales is None:
        raise ValueError("int8 coefficients need their scales")
    L = _lib.load()
    _lib.check(L.stacr_c1_restore(_ptr(coeff), DTYPE_I8 if quant else dtype_code(coeff.dtype),
                                  _ptr(scales.to(torch.float32).contiguous().reshape(-1)) if quant else None,
                                  _ptr(basis), dtype_code(basis.dtype), rows, hidden, rank, _ptr(out), dtype_code(dtype),
                                  _stream(coeff.device)), "stacr_c1_restore")
    return out
