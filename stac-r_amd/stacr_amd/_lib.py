"""Loads libstacr_amd.so (the HIP kernels behind the C ABI in include/stacr_amd.h).

torch is imported first so that the library binds to the HIP runtime torch already loaded
(both carry the SONAME libamdhip64.so.7); streams and device pointers are then shared.
There is no fallback: if the library is missing, every compute entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libstacr_amd.so")

STACR_OK = 0
STACR_ERR_INVALID = 1
STACR_ERR_UNSUPPORTED = 2
STACR_ERR_WORKSPACE = 3
STACR_ERR_HIP = 4

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
MODE_CHUNK_TOPK, MODE_GLOBAL_TOPK = 0, 1
MAX_RANK = 32
SCALE_F64 = 3  # scale record dtype code: fp64 (an fp32 scale that underflowed)

# Every symbol declared in include/stacr_amd.h, with its ctypes signature.
_i64, _i32, _f64, _p, _sz = ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_void_p, ctypes.c_size_t
_P64, _PSZ, _PI32 = ctypes.POINTER(_i64), ctypes.POINTER(_sz), ctypes.POINTER(_i32)
SIGNATURES = {
    "stacr_abi_version": ([], _i32),
    "stacr_last_error": ([], ctypes.c_char_p),
    "stacr_residual_plan": ([_i64, _i64, _i32, _f64, _i64, _P64, _P64, _PI32], _i32),
    "stacr_save_workspace_bytes": ([_i64, _i64, _i32, _i32, _i32, _f64, _i64, _i32, _PSZ], _i32),
    "stacr_save": ([_p, _p, _i32, _i64, _i64, _i32, _i32, _f64, _i64, _i32, _p, _p, _i32, _p, _p, _p, _sz, _p],
                   _i32),
    "stacr_save_census_bytes": ([_i64, _i64, _PSZ], _i32),
    "stacr_save_census": ([_p, _p, _i32, _i64, _i64, _i32, _i32, _f64, _i64, _i32, _p, _p, _i32, _p, _p, _p, _sz, _p,
                           _sz, _p, _p], _i32),
    "stacr_select_residual": ([_p, _p, _p, _i32, _i64, _i64, _i32, _i32, _f64, _i64, _i32, _p, _i32, _p, _p, _p,
                               _sz, _p], _i32),
    "stacr_quantize_values": ([_p, _i32, _i64, _i32, _p, _p, _p, _sz, _p], _i32),
    "stacr_profile_begin": ([_i32, _f64], _i32),
    "stacr_profile_end": ([_i32, _p, _p, _p, _p], _i32),
    "stacr_weight_grad_workspace_bytes": ([_i64, _i64, _i64, _i32, _i64, _PSZ], _i32),
    "stacr_weight_grad": ([_p, _i32, _i64, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _p, _i32, _i32, _i64, _i32, _p,
                           _i32, _p, _i32, _p, _sz, _p], _i32),
    "stacr_weight_grad_census": ([_p, _i32, _i64, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _p, _i32, _i32, _i64, _i32,
                                  _p, _i32, _p, _i32, _p, _sz, _p, _sz, _p], _i32),
    "stacr_weight_grad_noalloc": ([_p, _i32, _i64, _i64, _p, _p, _i64, _i32, _p, _i32, _p, _p, _i32, _i32, _i64, _i32,
                                   _p, _i32, _p, _i32, _p], _i32),
    "stacr_adaptive_residual_plan": ([_i64, _i64, _f64, _i64, _P64, _P64, _PI32], _i32),
    "stacr_adaptive_save_workspace_bytes": ([_i64, _i64, _i32, _i32, _f64, _i64, _PSZ], _i32),
    "stacr_adaptive_save": ([_p, _p, _i32, _i64, _i64, _i32, _f64, _i64, _p, _p, _p, _i32, _p, _p, _p, _sz, _p],
                            _i32),
    "stacr_adaptive_save_y_workspace_bytes": ([_i64, _i64, _i32, _i32, _i32, _f64, _i64, _PSZ], _i32),
    "stacr_adaptive_save_y": ([_p, _p, _i32, _i64, _i64, _i32, _i32, _f64, _i64, _p, _p, _p, _i32, _p, _p, _p,
                               ctypes.POINTER(ctypes.c_int), _p, _sz, _p], _i32),
    "stacr_adaptive_quantize": ([_p, _i32, _i64, _i32, _p, _p, _p, _sz, _p], _i32),
    "stacr_adaptive_dequantize": ([_p, _i32, _p, _i64, _p, _i32, _p], _i32),
    "stacr_csr_encode": ([_p, _i32, _i64, _i64, _i64, _p, _i32, _p, _i32, _p], _i32),
    "stacr_csr_decode": ([_p, _i32, _p, _i32, _i64, _i64, _i64, _p, _i32, _p], _i32),
    "stacr_delta_max": ([_p, _i32, _i64, _p, _p], _i32),
    "stacr_delta_encode": ([_p, _i32, _i64, _p, _i32, _p, _i32, _p], _i32),
    "stacr_delta_decode_workspace_bytes": ([_i64, _PSZ], _i32),
    "stacr_delta_decode": ([_p, _i32, _p, _i32, _i64, _p, _i32, _p, _sz, _p], _i32),
    "stacr_select_uniform": ([_p, _p, _p, _i32, _i64, _i64, _i32, _i64, _p, _i32, _p, _p], _i32),
    "stacr_block_sparse_plan": ([_i64, _i64, _f64, _i64, _i64, _P64, _P64, _P64, _PSZ], _i32),
    "stacr_select_block_sparse": ([_p, _p, _p, _i32, _i64, _i64, _i32, _f64, _i64, _i64, _p, _i32, _p, _p, _sz,
                                   _p], _i32),
    "stacr_sample_magnitudes": ([_p, _p, _p, _i32, _i64, _i64, _i32, _p, _i64, _p, _p], _i32),
    "stacr_threshold_workspace_bytes": ([_i64, _i64, _PSZ], _i32),
    "stacr_select_threshold": ([_p, _p, _p, _i32, _i64, _i64, _i32, _p, _i64, _p, _i32, _p, _p, _p, _sz, _p],
                               _i32),
    "stacr_adaptive_block_sparse_plan": ([_i64, _i64, _f64, _i64, _i64, _P64, _P64, _PI32, _PSZ], _i32),
    "stacr_adaptive_select_block_sparse": ([_p, _p, _p, _i32, _i64, _i64, _i32, _f64, _i64, _i64, _p, _i32, _p, _p, _p,
                                            _sz, _p], _i32),
    "stacr_oja_workspace_bytes": ([_i64, _i64, _i32, _PSZ], _i32),
    "stacr_oja_step": ([_p, _i32, _i64, _i64, _p, _i32, ctypes.c_float, _p, _p, _p, _sz, _p], _i32),
    "stacr_oja_step_given_y": ([_p, _i32, _i64, _i64, _p, _i32, _p, ctypes.c_float, _p, _p, _p, _sz, _p], _i32),
    "stacr_qr": ([_p, _i64, _i32, _p, _p, _p], _i32),
    "stacr_qr_tall_workspace_bytes": ([_i64, _i32, _PSZ], _i32),
    "stacr_qr_tall": ([_p, _i64, _i32, _p, _p, _p, _sz, _p], _i32),
    "stacr_reconstruct": ([_p, _p, _i32, _i64, _i64, _i32, _p, _i32, _p, _i64, _i32, _p, _p], _i32),
    "stacr_index_stream_sizes": ([_i64, _p, _p], _i32),
    "stacr_index_stream_encode": ([_p, _i32, _i64, _p, _p, _p, _p, _p], _i32),
    "stacr_index_stream_decode": ([_p, _p, _p, _i64, _p, _i32, _p], _i32),
    "stacr_quantize_rows_int8": ([_p, _i32, _i64, _i32, _p, _p, _p], _i32),
    "stacr_dequantize_rows_int8": ([_p, _p, _i64, _i32, _p, _i32, _p], _i32),
    "stacr_c1_workspace_bytes": ([_i64, _i64, _i32, _p], _i32),
    "stacr_c1_observe": ([_p, _i32, _i64, _i64, _p, _p, _i32, _i32, _p, _p, _p, _sz, _p], _i32),
    "stacr_c1_store": ([_p, _i64, _i32, _p, _i32, _p, _i32, _p], _i32),
    "stacr_c1_restore": ([_p, _i32, _p, _p, _i32, _i64, _i64, _i32, _p, _i32, _p], _i32),
}

_lib = None


class StacrLibraryError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (python stac-r_amd/build.py)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise StacrLibraryError(
                f"{LIB_PATH} is missing: build the HIP library first (python stac-r_amd/build.py)"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes, fn.restype = args, res
        if lib.stacr_abi_version() != 1:
            raise StacrLibraryError("libstacr_amd.so ABI version mismatch")
        _lib = lib
    return _lib


class KernelTimer:
    """Context manager around stacr_profile_begin/end: per-kernel (total ms, launches)."""

    def __init__(self, max_launches: int = 4096, sleep_us: float = 20.0):
        self.max_launches, self.sleep_us = int(max_launches), float(sleep_us)
        self.results: dict[str, tuple[float, int]] = {}

    def __enter__(self):
        check(load().stacr_profile_begin(self.max_launches, self.sleep_us), "stacr_profile_begin")
        return self

    def __exit__(self, *exc):
        cap = 64
        names = ctypes.create_string_buffer(64 * cap)
        ms = (ctypes.c_double * cap)()
        cnt = (ctypes.c_int * cap)()
        n = ctypes.c_int()
        check(load().stacr_profile_end(cap, ctypes.cast(names, ctypes.c_void_p), ctypes.cast(ms, ctypes.c_void_p),
                                       ctypes.cast(cnt, ctypes.c_void_p), ctypes.cast(ctypes.byref(n), ctypes.c_void_p)),
              "stacr_profile_end")
        raw = names.raw
        for i in range(n.value):
            name = raw[64 * i: 64 * (i + 1)].split(b"\0", 1)[0].decode()
            self.results[name] = (ms[i], cnt[i])
        return False


def check(rc: int, what: str) -> None:
    if rc == STACR_OK:
        return
    msg = load().stacr_last_error().decode(errors="replace")
    if rc == STACR_ERR_INVALID:
        raise ValueError(f"{what}: {msg}")
    if rc == STACR_ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg}")
