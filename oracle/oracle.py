"""Python face of the CPU oracle (test infrastructure only).

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import this
module.  It is the checker and the timed CPU baseline, never part of the product path.

The integer/byte work (k rules, exact selection, quantization, nibble packing) and the fp64
weight gradient live in ``stacr_oracle.c`` (each function there cites the reference line it
restates).  This module adds the numpy pieces: dtype rounding, the fp64 projection
(stacr/layers.py:135-137), dequantization (stacr/quant.py:17-21,40-46), a composed save, the
adaptive engine's quantizers, index codecs and energies, and the fp64 Oja step.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle.so")

MODE_CHUNK, MODE_GLOBAL = 0, 1
MODES = {"chunk_topk": MODE_CHUNK, "topk": MODE_CHUNK, "global_topk": MODE_GLOBAL}

_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        i64, f64, i32 = ctypes.c_int64, ctypes.c_double, ctypes.c_int
        P = ctypes.c_void_p
        L.orc_py_round.argtypes, L.orc_py_round.restype = [f64], i64
        L.orc_chunk_k.argtypes, L.orc_chunk_k.restype = [i64, f64], i64
        L.orc_residual_plan.argtypes = [i64, i64, i32, f64, i64, P, P]
        L.orc_select.argtypes, L.orc_select.restype = [P, i64, i64, i32, f64, i64, P, P], i64
        L.orc_sorted_keys.argtypes = [P, i64, P]
        L.orc_quantize.argtypes = [P, i64, i32, P, P]
        L.orc_pack_int4.argtypes = [P, i64, P]
        L.orc_weight_grad.argtypes, L.orc_weight_grad.restype = [P, i64, i64, P, P, i64, i32, P, P, i64, P, P], i32
        L.orc_round_dtype.argtypes, L.orc_round_dtype.restype = [ctypes.c_float, i32], ctypes.c_float
        L.orc_residual_act.argtypes = [P, P, P, i64, i64, i32, i32, P]
        L.orc_lowrank.argtypes = [P, P, i64, i64, i32, i32, P]
        L.orc_select_explicit.argtypes, L.orc_select_explicit.restype = [P, i64, i64, i64, i64, i64, P, P], i64
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- k rules
def py_round(v: float) -> int:
    return int(lib().orc_py_round(float(v)))


def chunk_k(n: int, budget: float) -> int:
    return int(lib().orc_chunk_k(int(n), float(budget)))


def residual_plan(rows: int, feats: int, mode: str, budget: float, chunk_rows: int):
    """(k_total, sum of per-chunk k) following stacr/layers.py:16-41,44-54."""
    kt, ks = ctypes.c_int64(), ctypes.c_int64()
    lib().orc_residual_plan(int(rows), int(feats), MODES[mode], float(budget), int(chunk_rows),
                            ctypes.byref(kt), ctypes.byref(ks))
    return int(kt.value), int(ks.value)


# ---------------------------------------------------------------- dtype helpers
def round_to(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round fp32 values to bf16 / fp16 (nearest-even) and return them as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if dtype in ("f32", "float32"):
        return a.copy()
    if dtype in ("f16", "float16"):
        return a.astype(np.float16).astype(np.float32)
    if dtype in ("bf16", "bfloat16"):
        u = a.view(np.uint32).astype(np.uint64)
        nan = np.isnan(a)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
        out = r.view(np.float32).copy()
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def project_f64(x: np.ndarray, q: np.ndarray) -> np.ndarray:
    """C = X Q in fp64 (stacr/layers.py:137 before its final rounding)."""
    return np.asarray(x, np.float64) @ np.asarray(q, np.float64)


# ---------------------------------------------------------------- residual + selection
def select(resid: np.ndarray, mode: str, budget: float, chunk_rows: int):
    """Exact selection with the lowest-index tie rule; (idx int64 ascending, values fp32)."""
    resid = _c(resid, np.float32)
    rows, d = resid.shape
    if rows * d >= 2**32:
        raise ValueError("oracle selection supports fewer than 2^32 elements")
    kt, ks = residual_plan(rows, d, mode, budget, chunk_rows)
    idx = np.empty(max(ks, 1), np.int64)
    val = np.empty(max(ks, 1), np.float32)
    n = lib().orc_select(_ptr(resid), rows, d, MODES[mode], float(budget), int(chunk_rows),
                         _ptr(idx), _ptr(val))
    return idx[:n].copy(), val[:n].copy()


def sorted_keys(resid: np.ndarray) -> np.ndarray:
    flat = _c(resid, np.float32).reshape(-1)
    out = np.empty(flat.size, np.uint64)
    lib().orc_sorted_keys(_ptr(flat), flat.size, _ptr(out))
    return out


# ---------------------------------------------------------------- quantization
def quantize(vals: np.ndarray, bits: int):
    """stacr/quant.py:49-65 -> (q int8 before packing, scale fp32)."""
    vals = _c(vals, np.float32).reshape(-1)
    q = np.zeros(vals.size, np.int8)
    scale = np.zeros(1, np.float32)
    lib().orc_quantize(_ptr(vals), vals.size, int(bits), _ptr(q), _ptr(scale))
    return q, np.float32(scale[0])


def pack_int4(q: np.ndarray) -> np.ndarray:
    q = _c(q, np.int8).reshape(-1)
    out = np.zeros((q.size + 1) // 2, np.uint8)
    lib().orc_pack_int4(_ptr(q), q.size, _ptr(out))
    return out


def unpack_int4(packed: np.ndarray, length: int) -> np.ndarray:
    """stacr/quant.py:40-46."""
    p = np.asarray(packed, np.uint8)
    lo = (p & 0x0F).astype(np.int8)
    hi = ((p >> 4) & 0x0F).astype(np.int8)
    lo = np.where(lo > 7, lo - 16, lo).astype(np.int8)
    hi = np.where(hi > 7, hi - 16, hi).astype(np.int8)
    return np.stack([lo, hi], axis=1).reshape(-1)[:length]


def dequantize(data: np.ndarray, scale: float, bits: int, length: int) -> np.ndarray:
    """stacr/quant.py:17-21 with dtype fp32: data.to(f32) * scale.to(f32)."""
    if bits == 4:
        data = unpack_int4(data, length)
    if bits == 0:
        return np.asarray(data, np.float32).copy()
    return (np.asarray(data, np.float32) * np.float32(scale)).astype(np.float32)


# ---------------------------------------------------------------- weight gradient
def check_indices(idx: np.ndarray, total: int, ascending: bool = False) -> None:
    """Fail (AssertionError) when flat indices a kernel produced fall outside [0, total) or, with
    ``ascending``, are not strictly increasing, before anything indexes memory with them."""
    idx = np.asarray(idx, np.int64).reshape(-1)
    if idx.size == 0:
        return
    lo, hi = int(idx.min()), int(idx.max())
    if lo < 0 or hi >= total:
        raise AssertionError(f"flat index out of range: min {lo}, max {hi}, allowed [0, {total})")
    if ascending and idx.size > 1 and not bool(np.all(idx[1:] > idx[:-1])):
        bad = int(np.argmax(idx[1:] <= idx[:-1]))
        raise AssertionError(f"flat indices not strictly ascending at position {bad + 1}")


def weight_grad(g, c, q, idx, vals, d_in: int):
    """fp64 dW (d_out x d_in) and dbias following stacr/layers.py:172-198."""
    g, c, q = _c(g, np.float32), _c(c, np.float32), _c(q, np.float32)
    idx, vals = _c(idx, np.int64).reshape(-1), _c(vals, np.float32).reshape(-1)
    n, d_out = g.shape
    r = c.shape[1]
    check_indices(idx, n * d_in)
    if vals.size != idx.size:
        raise AssertionError(f"{idx.size} indices but {vals.size} values")
    dw = np.empty((d_out, d_in), np.float64)
    db = np.empty(d_out, np.float64)
    rc = lib().orc_weight_grad(_ptr(g), n, d_out, _ptr(c), _ptr(q), d_in, r, _ptr(idx), _ptr(vals),
                               idx.size, _ptr(dw), _ptr(db))
    if rc != 0:
        raise AssertionError("orc_weight_grad rejected an index outside [0, rows * d_in)")
    return dw, db


# ---------------------------------------------------------------- composed save (CPU baseline)
def save(x: np.ndarray, q: np.ndarray, dtype: str, mode: str, budget: float, chunk_rows: int,
         bits: int, coeff: np.ndarray | None = None):
    """The whole save step on the CPU, in the HIP path's arithmetic.

    ``coeff`` (already rounded to ``dtype``) may be supplied so that selection is compared on the
    identical residual; otherwise it is the fp64 projection rounded to ``dtype``.
    Returns (coeff, idx, q_or_values, scale).
    """
    xr = round_to(x, dtype)
    qr = round_to(q, dtype)
    if coeff is None:
        coeff = round_to(project_f64(xr, qr).astype(np.float32), dtype)
    resid = residual_act(xr, coeff, qr, dtype)
    idx, val = select(resid, mode, budget, chunk_rows)
    if bits == 0:
        return coeff, idx, val, np.float32(1.0)
    qv, scale = quantize(val, bits)
    return coeff, idx, (pack_int4(qv) if bits == 4 else qv), scale


# ================================================================ adaptive engine
# (stacr/adaptive.py, stacr/index_compression.py).  Test infrastructure, like the rest of this file.
DTYPE_CODE = {"f32": 0, "float32": 0, "bf16": 1, "bfloat16": 1, "f16": 2, "float16": 2}


def round_dtype_scalar(v: float, dtype: str) -> float:
    return float(lib().orc_round_dtype(float(v), DTYPE_CODE[dtype]))


def residual_act(x: np.ndarray, c: np.ndarray, q: np.ndarray, dtype: str) -> np.ndarray:
    """R = rnd(x - rnd(C Q^T)) in the activation dtype, both engines' arithmetic
    (stacr/layers.py:32,73, stacr/adaptive.py:1518-1519)."""
    x, c, q = _c(x, np.float32), _c(c, np.float32), _c(q, np.float32)
    rows, d = x.shape
    out = np.empty_like(x)
    lib().orc_residual_act(_ptr(x), _ptr(c), _ptr(q), rows, d, q.shape[1], DTYPE_CODE[dtype], _ptr(out))
    return out


def lowrank(c: np.ndarray, q: np.ndarray, dtype: str) -> np.ndarray:
    """L = rnd(C Q^T) in the activation dtype, the chain of residual_act (stacr/compressor.py:128)."""
    c, q = _c(c, np.float32), _c(q, np.float32)
    out = np.empty((c.shape[0], q.shape[0]), np.float32)
    lib().orc_lowrank(_ptr(c), _ptr(q), c.shape[0], q.shape[0], q.shape[1], DTYPE_CODE[dtype], _ptr(out))
    return out


def reconstruct(c: np.ndarray, q: np.ndarray, idx: np.ndarray | None, vals: np.ndarray | None,
                dtype: str) -> np.ndarray:
    """The saved-tensor hooks' dense unpack (stacr/compressor.py:127-133, stacr/residual.py:13-20):
    L = rnd(C Q^T) in the activation dtype (the fp32 chain of residual_act), then, with a residual
    (idx is not None), every element gets + dense: rnd(L + v) at the entries and L + 0 elsewhere
    (turning -0 into +0)."""
    low = lowrank(c, q, dtype)
    if idx is None:
        return low
    out = low + np.float32(0.0)
    flat = out.reshape(-1)
    idx = np.asarray(idx, np.int64)
    if idx.size:
        flat[idx] = round_to(low.reshape(-1)[idx] + np.asarray(vals, np.float32), dtype)
    return out


def adaptive_plan(rows: int, feats: int, budget: float, chunk_rows: int = 512):
    """(k, per-chunk k, chunk rows, index dtype) of the adaptive "topk" mode (stacr/adaptive.py:1357-1365,1524)."""
    total = rows * feats
    k = int(total * budget)
    idx_dtype = np.int16 if total < 32768 else (np.int32 if total <= 2**31 else np.int64)
    if k <= 0:
        return 0, 0, min(chunk_rows, rows), idx_dtype
    k = min(k, total)
    chunk = min(chunk_rows, rows)
    per_chunk_k = max(1, (k * chunk + rows - 1) // rows)
    return k, per_chunk_k, chunk, idx_dtype


def select_explicit(resid: np.ndarray, chunk_rows: int, k_chunk: int, k_total: int):
    resid = _c(resid, np.float32)
    rows, d = resid.shape
    n_chunks = (rows + chunk_rows - 1) // chunk_rows
    cap = max(1, n_chunks * k_chunk)
    idx = np.empty(cap, np.int64)
    val = np.empty(cap, np.float32)
    n = lib().orc_select_explicit(_ptr(resid), rows, d, int(chunk_rows), int(k_chunk), int(k_total), _ptr(idx),
                                  _ptr(val))
    return idx[:n].copy(), val[:n].copy()


def adaptive_save(x: np.ndarray, q: np.ndarray, dtype: str, budget: float, chunk_rows: int = 512,
                  coeff: np.ndarray | None = None):
    """coeff, idx (ascending, the reference's index dtype), values (fp32 copies of dtype values)."""
    xr, qr = round_to(x, dtype), round_to(q, dtype)
    if coeff is None:
        coeff = round_to(project_f64(xr, qr).astype(np.float32), dtype)
    rows, d = xr.shape
    k, pck, chunk, idx_dtype = adaptive_plan(rows, d, budget, chunk_rows)
    if k == 0:
        return coeff, None, None
    resid = residual_act(xr, coeff, qr, dtype)
    idx, val = select_explicit(resid, chunk, pck, k)
    return coeff, idx.astype(idx_dtype), val


def _np_dtype_round(a: np.ndarray, dtype: str) -> np.ndarray:
    return round_to(np.asarray(a, np.float32), dtype)


def adaptive_quantize(values: np.ndarray, dtype: str, bits: int):
    """quantize_int8 / quantize_int4 (stacr/adaptive.py:44-120) on dtype values held as fp32.

    Returns (q int8 in [-qmax, qmax], scale value (float), scale dtype name)."""
    v = np.asarray(values, np.float32).reshape(-1)
    qmax = 7.0 if bits == 4 else 127.0
    if v.size == 0:
        return np.zeros(0, np.int8), 1.0, dtype
    amax = np.float32(np.max(np.abs(v)))
    scale = _np_dtype_round(np.float32(amax) / np.float32(qmax), dtype).reshape(-1)[0]
    if scale == 0:
        if amax == 0:
            return np.zeros(v.size, np.int8), 1.0, dtype
        if dtype in ("bf16", "f16", "bfloat16", "float16"):
            s32 = np.float32(amax) / np.float32(qmax)
            q = np.clip(np.rint(v / s32), -qmax, qmax).astype(np.int8)
            return q, float(s32), "f32"
        s64 = np.float64(amax) / np.float64(qmax)
        q = np.clip(np.rint(v.astype(np.float64) / s64), -qmax, qmax).astype(np.int8)
        return q, float(s64), "f64"
    with np.errstate(invalid="ignore", over="ignore"):
        quot = _np_dtype_round(v / np.float32(scale), dtype)
        q = np.clip(np.rint(quot), -qmax, qmax).astype(np.int8)
    return q, float(scale), dtype


def adaptive_pack_int4(q: np.ndarray) -> np.ndarray:
    """(q + 8) nibbles, even entry low, odd length padded with 8 (stacr/adaptive.py:110-119)."""
    u = (np.asarray(q, np.int16) + 8).astype(np.uint8)
    if u.size % 2:
        u = np.concatenate([u, np.array([8], np.uint8)])
    return (u[0::2] | (u[1::2] << 4)).astype(np.uint8)


def adaptive_dequantize(q: np.ndarray, scale: float, scale_dtype: str) -> np.ndarray:
    """q.to(scale dtype) * scale, as fp32 (fp64 for an fp64 scale)."""
    qf = np.asarray(q, np.float32)
    if scale_dtype == "f64":
        return qf.astype(np.float64) * np.float64(scale)
    return _np_dtype_round(qf * np.float32(scale), scale_dtype)


def csr_encode(sorted_idx: np.ndarray, b_flat: int, n: int):
    """row_ptrs (int32) and column indices (int16 when n < 32768) of row-sorted flat indices."""
    flat = np.asarray(sorted_idx, np.int64)
    rows = flat // n
    counts = np.bincount(rows, minlength=b_flat)[:b_flat]
    ptr = np.zeros(b_flat + 1, np.int64)
    ptr[1:] = np.cumsum(counts)
    col_dtype = np.int16 if n < 32768 else (np.int32 if n <= 2**31 else np.int64)
    return ptr.astype(np.int32 if flat.size < 2**31 else np.int64), (flat % n).astype(col_dtype)


def csr_decode(ptr: np.ndarray, cols: np.ndarray, n: int) -> np.ndarray:
    counts = np.diff(np.asarray(ptr, np.int64))
    rows = np.repeat(np.arange(counts.size, dtype=np.int64), counts)
    return rows * n + np.asarray(cols, np.int64)


def delta_encode(sorted_idx: np.ndarray, b_flat: int, n: int):
    flat = np.asarray(sorted_idx, np.int64)
    base = flat[:1].astype(np.int32 if b_flat * n <= 2**31 else np.int64)
    if flat.size > 1:
        d = np.diff(flat)
        m = int(d.max())
        dd = np.int16 if m <= 32767 else (np.int32 if m < 2**31 else np.int64)
        return base, d.astype(dd)
    return base, np.zeros(0, np.int16)


def delta_decode(base: np.ndarray, deltas: np.ndarray, nnz: int) -> np.ndarray:
    out = np.zeros(nnz, np.int64)
    out[0] = int(np.asarray(base).reshape(-1)[0])
    out[1:] = np.asarray(deltas, np.int64)
    return np.cumsum(out)


def adaptive_energy(x: np.ndarray, c: np.ndarray, dtype: str):
    """(residual energy, |X|^2, |C|^2, mean c_j^2) as stacr/adaptive.py:1388-1393,1953-1958 compute them,
    with the sums in fp64 before the dtype rounding."""
    xr, cr = np.asarray(x, np.float32), np.asarray(c, np.float32)
    x2 = round_dtype_scalar(float(_np_dtype_round(xr * xr, dtype).astype(np.float64).sum()), dtype)
    c2 = round_dtype_scalar(float(_np_dtype_round(cr * cr, dtype).astype(np.float64).sum()), dtype)
    d0 = round_dtype_scalar(x2 - c2, dtype)
    diff = d0 if np.isnan(d0) else max(d0, 0.0)  # torch.clamp keeps NaN
    num = round_dtype_scalar(np.sqrt(np.float32(diff)), dtype)
    den = round_dtype_scalar(round_dtype_scalar(np.sqrt(np.float32(x2)), dtype) + np.float32(1e-8), dtype)
    with np.errstate(invalid="ignore", divide="ignore"):  # an overflowed 16-bit sum gives inf / inf
        e = round_dtype_scalar(np.float32(num) / np.float32(den), dtype)
    per_rank = (cr.astype(np.float64) ** 2).mean(axis=0)
    return e, x2, c2, per_rank



def oja_step(x: np.ndarray, q: np.ndarray, lr: float):
    """(update, stepped) of one Oja step in fp64 (stacr/layers.py:346-348, stacr/oja.py:73-79):
    Y = XQ, update = X^T Y / max(1, N) - Q (Y^T Y / max(1, N)), stepped = Q + lr * update."""
    xd, qd = np.asarray(x, np.float64), np.asarray(q, np.float64)
    n = max(1, xd.shape[0])
    y = xd @ qd
    update = xd.T @ y / n - qd @ (y.T @ y / n)
    return update, qd + float(lr) * update


def orthonormalize(m: np.ndarray) -> np.ndarray:
    """Reduced QR's Q (stacr/oja.py:8-11); column signs follow numpy's LAPACK call."""
    q, _ = np.linalg.qr(np.asarray(m, np.float64), mode="reduced")
    return q


# ================================================================ other projection-engine selectors
# (stacr/layers.py:55-99), on the dtype-native residual of residual_act.
def uniform_positions(total: int, k: int) -> np.ndarray:
    """floor(i * total / k), i = 0..k-1: the union of the reference's per-chunk ranges (:89-98)."""
    i = np.arange(k, dtype=np.uint64)
    return (i * np.uint64(total) // np.uint64(k)).astype(np.int64)


def select_uniform(resid: np.ndarray, k: int):
    flat = np.asarray(resid, np.float32).reshape(-1)
    idx = uniform_positions(flat.size, k)
    return idx, flat[idx]


def block_energies(resid: np.ndarray, block_size: int, dtype: str) -> np.ndarray:
    """rnd(sum_o rnd(r_o^2)) per block of block_size consecutive elements, the sum an fp32
    sequence of additions in element order (:84)."""
    sq = round_to(np.asarray(resid, np.float32) ** 2, dtype).reshape(-1, block_size)
    acc = np.zeros(sq.shape[0], np.float32)
    for o in range(block_size):
        acc = (acc + sq[:, o]).astype(np.float32)
    return round_to(acc, dtype)


def block_sparse_counts(rows: int, feats: int, budget: float, chunk_rows: int, block_size: int):
    """count per chunk = max(1, round(budget * blocks in the chunk)) (:83)."""
    out = []
    for start in range(0, rows, chunk_rows):
        blocks = min(chunk_rows, rows - start) * feats // block_size
        out.append(max(1, int(round(budget * blocks))))
    return out


def select_block_sparse(resid: np.ndarray, budget: float, chunk_rows: int, block_size: int, dtype: str):
    """Per chunk the top-count blocks by energy (ties: lowest block), all their elements, ascending."""
    resid = np.asarray(resid, np.float32)
    rows, feats = resid.shape
    flat = resid.reshape(-1)
    energy = block_energies(resid, block_size, dtype)
    keys = energy.view(np.uint32) & np.uint32(0x7FFFFFFF)  # NaN above +inf, as torch.topk orders it
    per_chunk_blocks = chunk_rows * feats // block_size
    chosen = []
    for c, count in enumerate(block_sparse_counts(rows, feats, budget, chunk_rows, block_size)):
        lo = c * per_chunk_blocks
        hi = min(lo + per_chunk_blocks, energy.size)
        b = np.arange(lo, hi)
        order = np.lexsort((b, -keys[lo:hi].astype(np.int64)))
        chosen.append(np.sort(b[order[:count]]))
    blocks = np.concatenate(chosen).astype(np.int64)
    idx = (blocks[:, None] * block_size + np.arange(block_size)).reshape(-1)
    return idx, flat[idx]


def select_threshold(resid: np.ndarray, threshold: float, dtype: str, cap: int):
    """First `cap` positions with |r| >= threshold rounded to dtype (torch promotes the fp32 0-dim
    quantile to the magnitude's dtype for the comparison, :65)."""
    flat = np.asarray(resid, np.float32).reshape(-1)
    t = np.float32(round_dtype_scalar(float(threshold), dtype))
    with np.errstate(invalid="ignore"):
        idx = np.nonzero(np.abs(flat) >= t)[0][:cap].astype(np.int64)
    return idx, flat[idx]


def adaptive_select_above(resid: np.ndarray, threshold: float, dtype: str):
    """Every position with |r| > threshold, ascending, with its value: the adaptive engine's
    `chunk_flat.abs() > threshold_val` + `nonzero` over its chunks (stacr/adaptive.py:1493-1517 streaming
    top-k, :1590-1606 "threshold", :1762-1778 "adaptive_threshold").  torch compares a tensor with a
    Python float or a 0-dim tensor in the tensor's dtype, so the threshold is rounded to dtype first."""
    flat = np.asarray(resid, np.float32).reshape(-1)
    t = np.float32(round_dtype_scalar(float(threshold), dtype))
    with np.errstate(invalid="ignore"):
        idx = np.nonzero(np.abs(flat) > t)[0].astype(np.int64)
    return idx, flat[idx]


# ================================================================ adaptive engine's block_sparse
# (stacr/adaptive.py:1788-1938), on the dtype-native residual of residual_act.
def adaptive_block_energies(resid: np.ndarray, block_size: int, dtype: str) -> np.ndarray:
    """Energy of every block of `block_size` columns of one row, the row's last block padded with
    zeros (:1847-1868): rnd(sum_o rnd(r_o^2)), an fp32 sum in column order; rows * ceil(d / bs) values."""
    resid = np.asarray(resid, np.float32)
    rows, d = resid.shape
    bpr = -(-d // block_size)
    padded = np.zeros((rows, bpr * block_size), np.float32)
    padded[:, :d] = resid
    sq = round_to(padded * padded, dtype).reshape(rows * bpr, block_size)
    acc = np.zeros(rows * bpr, np.float32)
    for o in range(block_size):
        acc = (acc + sq[:, o]).astype(np.float32)
    return round_to(acc, dtype)


def adaptive_block_plan(rows: int, feats: int, budget: float, chunk_rows: int, block_size: int):
    """(k_blocks, chunk rows, blocks kept per chunk) of the adaptive selector (:1791-1802, :1833)."""
    total = rows * feats
    k = min(int(total * budget), total)
    if k <= 0:
        return 0, 0, 0
    k_blocks = max(1, -(-k // block_size))
    chunk = min(chunk_rows, rows)
    return k_blocks, chunk, max(1, (k_blocks * chunk + rows - 1) // rows)


def adaptive_select_block_sparse(resid: np.ndarray, budget: float, chunk_rows: int, block_size: int, dtype: str):
    """(idx ascending, values) of the adaptive block_sparse selector: per chunk the top blocks by
    energy, then the top k_blocks of all candidates, ties to the lowest block (the reference's
    torch.topk leaves them open); every stored column of the kept blocks (padding dropped)."""
    resid = np.asarray(resid, np.float32)
    rows, d = resid.shape
    k_blocks, chunk, per = adaptive_block_plan(rows, d, budget, chunk_rows, block_size)
    if k_blocks == 0:
        return np.zeros(0, np.int64), np.zeros(0, np.float32)
    bpr = -(-d // block_size)
    keys = adaptive_block_energies(resid, block_size, dtype).view(np.uint32) & np.uint32(0x7FFFFFFF)
    keys = keys.astype(np.int64)
    cands = []
    for start in range(0, rows, chunk):
        lo, hi = start * bpr, min(start + chunk, rows) * bpr
        b = np.arange(lo, hi)
        order = np.lexsort((b, -keys[lo:hi]))
        cands.append(b[order[:min(per, hi - lo)]])
    cand = np.concatenate(cands)
    if cand.size > k_blocks:
        cand = cand[np.lexsort((cand, -keys[cand]))[:k_blocks]]
    cand = np.sort(cand)
    cols = (cand % bpr)[:, None] * block_size + np.arange(block_size)[None, :]
    flat = (cand // bpr)[:, None] * d + cols
    idx = flat[cols < d].astype(np.int64)
    return idx, resid.reshape(-1)[idx]


# ================================================================ compact save outputs
# The bit-packed index stream and row-quantized coefficients of the library's codecs.  The stream
# is a denser form of the delta codec (stacr/index_compression.py:231-269) and decodes by its rule
# (base plus cumulative deltas, :327-342); the row quantizer is the C1 codec's safe-max rule
# (stacr/protocols/checkpointing.py:374-393) with the maximum taken per row.
STREAM_BLOCK = 256


def index_stream_encode(idx: np.ndarray):
    """(base int64[nb], word_off uint32[nb + 1], words uint32[word_off[nb]], status) of the stream:
    block b's deltas d_0 = 0, d_j = idx[256 b + j] - idx[256 b + j - 1] in w_b = bit length of the
    block's largest delta, slot j at bits [j w_b, (j + 1) w_b) of the block's 8 w_b words (least
    significant bit first).  status: 1 a decreasing pair, 2 a gap >= 2^32, 4 a negative index (such
    deltas are stored as 0)."""
    v = np.asarray(idx, np.int64).reshape(-1)
    nnz = v.size
    nb = -(-nnz // STREAM_BLOCK)
    base = np.zeros(nb, np.int64)
    word_off = np.zeros(nb + 1, np.uint64)
    blocks = []
    status = 0
    for b in range(nb):
        blk = v[b * STREAM_BLOCK:(b + 1) * STREAM_BLOCK]
        base[b] = blk[0]
        d = np.zeros(STREAM_BLOCK, np.int64)
        d[1:blk.size] = np.diff(blk)
        if (blk < 0).any():
            status |= 4
        if (d < 0).any():
            status |= 1
        if (d > 0xFFFFFFFF).any():
            status |= 2
        d[(d < 0) | (d > 0xFFFFFFFF)] = 0
        w = int(d.max()).bit_length()
        bits = 0
        for j in range(STREAM_BLOCK):
            bits |= int(d[j]) << (j * w)
        words = np.array([(bits >> (32 * k)) & 0xFFFFFFFF for k in range(8 * w)], np.uint64)
        blocks.append(words.astype(np.uint32))
        word_off[b + 1] = word_off[b] + 8 * w
    words = np.concatenate(blocks) if blocks else np.zeros(0, np.uint32)
    return base, word_off.astype(np.uint32), words, status


def index_stream_decode(base: np.ndarray, word_off: np.ndarray, words: np.ndarray, nnz: int) -> np.ndarray:
    """base[b] + inclusive prefix sums of block b's deltas (int64)."""
    out = np.zeros(nnz, np.int64)
    words = np.asarray(words, np.uint64)
    for b in range(len(base)):
        lo, hi = int(word_off[b]), int(word_off[b + 1])
        w = (hi - lo) // 8
        bits = 0
        for k in range(hi - lo):
            bits |= int(words[lo + k]) << (32 * k)
        n = min(STREAM_BLOCK, nnz - b * STREAM_BLOCK)
        d = [(bits >> (j * w)) & ((1 << w) - 1) for j in range(n)]
        out[b * STREAM_BLOCK:b * STREAM_BLOCK + n] = int(base[b]) + np.cumsum(np.asarray(d, np.int64))
    return out


def quantize_rows_int8(c: np.ndarray):
    """(codes int8 rows x rank, scales fp32[rows]): m = the row's max |c| in fp32 (NaN if it holds
    one), s = (m finite and > 0 ? m : 1) / 127 in fp32, q = clamp(round half to even(c / s), -127,
    127) with fp32 division, a NaN quotient coded 0."""
    c = np.asarray(c, np.float32)
    with np.errstate(invalid="ignore"):
        m = np.abs(c).max(axis=1) if c.shape[1] else np.zeros(c.shape[0], np.float32)
        safe = np.where(np.isfinite(m) & (m > 0), m, np.float32(1.0)).astype(np.float32)
        s = (safe / np.float32(127.0)).astype(np.float32)
        qv = np.rint((c / s[:, None]).astype(np.float32))
        qv = np.where(np.isnan(qv), np.float32(0.0), np.clip(qv, -127, 127))
    return qv.astype(np.int8), s


def dequantize_rows_int8(codes: np.ndarray, scales: np.ndarray, dtype: str) -> np.ndarray:
    """codes * scale in fp32, rounded once to dtype."""
    return round_to(np.asarray(codes, np.float32) * np.asarray(scales, np.float32)[:, None], dtype)


# ================================================================ C1 checkpoint-boundary codec
# CheckpointBoundaryCodec.pack_tensor / unpack_record (stacr/protocols/checkpointing.py:374-400,
# 411-545) on given fp32 coefficients, in the library's arithmetic: the reconstruction is the
# fp32 chain of lowrank, squares are rounded to fp32 and summed in fp64.
def _safe_max(a: np.ndarray):
    """(largest |v| that is not NaN (inf included) or 0, any value not NaN, any NaN)."""
    a = np.abs(np.asarray(a, np.float32)).reshape(-1)
    ok = ~np.isnan(a)
    return (float(a[ok].max()) if ok.any() else 0.0), bool(ok.any()), bool((~ok).any())


def c1_scales(coeff: np.ndarray) -> np.ndarray:
    """s_j = (m_j finite and > 0 ? m_j : 1) / 127 in fp32, m_j = max over rows of |c_j| (NaN if one
    is NaN) (_quantize_coefficients, :383-392)."""
    c = np.abs(np.asarray(coeff, np.float32))
    m = np.where(np.isnan(c).any(axis=0), np.float32(np.nan), np.where(np.isnan(c), 0, c).max(axis=0, initial=0.0))
    safe = np.where(np.isfinite(m) & (m > 0), m, np.float32(1.0)).astype(np.float32)
    return (safe / np.float32(127.0)).astype(np.float32)


def c1_observe(x: np.ndarray, coeff: np.ndarray, basis: np.ndarray) -> dict:
    x = np.asarray(x, np.float32)
    c = np.asarray(coeff, np.float32)
    q = np.asarray(basis, np.float32)
    p = lowrank(c, q, "f32")
    with np.errstate(invalid="ignore", over="ignore"):
        e = (x - p).astype(np.float32)
        err = float((e * e).astype(np.float32).astype(np.float64).sum())
        den = float((x * x).astype(np.float32).astype(np.float64).sum())
        energy = float(np.float32(err) / max(np.float32(den), np.float32(1e-12)))
    out = {"error": err, "denom": den, "energy": energy, "flags": 0}
    for name, arr, bits in (("input", x, (1, 16)), ("coeff", c, (2, 32)), ("reconstruction", p, (4, 64)),
                            ("basis", q, (8, 256)), ("residual", e, (512, 128))):
        m, valid, nan = _safe_max(arr)
        out[f"{name}_max_abs"] = m
        out["flags"] |= (bits[0] if nan else 0) | (bits[1] if valid else 0)
    return out


def c1_store(coeff: np.ndarray, scales: np.ndarray | None, dtype: str):
    """int8 clamp(round half even(c / s_j), -127, 127) (fp32 division, NaN coded 0) when scales are
    given, else C rounded to dtype."""
    c = np.asarray(coeff, np.float32)
    if scales is None:
        return round_to(c, dtype)
    with np.errstate(invalid="ignore"):
        qv = np.rint((c / np.asarray(scales, np.float32)[None, :]).astype(np.float32))
        qv = np.where(np.isnan(qv), np.float32(0.0), np.clip(qv, -127, 127))
    return qv.astype(np.int8)


def c1_restore(coeff: np.ndarray, scales: np.ndarray | None, basis: np.ndarray, dtype: str) -> np.ndarray:
    """sum_j c'_j q_j (the fp32 chain) rounded to dtype; c' = code * s_j in fp32 for int8 codes."""
    c = np.asarray(coeff, np.float32)
    if scales is not None:
        c = (c * np.asarray(scales, np.float32)[None, :]).astype(np.float32)
    return lowrank(c, np.asarray(basis, np.float32), dtype)
