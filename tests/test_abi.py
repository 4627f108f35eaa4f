"""The C ABI library: loads, exports every declared symbol, host-side rules and error paths.

No kernel is launched here (no GPU in the CPU suite); the compute parity tests are in
test_gpu_parity.py.
"""
import ctypes
import os
import re

import pytest

from oracle import oracle as orc

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "stacr_amd.h")


def _lib():
    from stacr_amd import _lib as L

    if not os.path.exists(L.LIB_PATH):
        pytest.skip("libstacr_amd.so not built")
    return L


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^(?:int|const char \*)\s*(stacr_\w+)\(", text, re.M)))


def test_header_declares_the_abi():
    names = declared_functions()
    assert {"stacr_save", "stacr_weight_grad", "stacr_residual_plan", "stacr_last_error"} <= set(names)


def test_library_exports_every_declared_symbol():
    L = _lib()
    lib = ctypes.CDLL(L.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(L.SIGNATURES), "ctypes signatures out of sync with the header"
    assert L.load().stacr_abi_version() == 1


@pytest.mark.parametrize(
    "rows,feats,mode,budget,chunk",
    [(4096, 768, "chunk_topk", 0.005, 512), (8192, 1024, "global_topk", 0.005, 512),
     (8192, 4096, "chunk_topk", 0.005, 512), (5, 16, "chunk_topk", 0.17, 1), (5, 16, "chunk_topk", 0.25, 2),
     (5, 16, "global_topk", 0.25, 2), (37, 24, "chunk_topk", 0.05, 8), (3, 4, "chunk_topk", 0.0625, 1),
     (1000, 3, "topk", 0.3, 7), (0, 16, "chunk_topk", 0.5, 4), (7, 9, "chunk_topk", 0.0, 4)],
)
def test_residual_plan_matches_oracle(rows, feats, mode, budget, chunk):
    from stacr_amd import kernels

    _lib()
    k_total, k_saved, ib = kernels.residual_plan(rows, feats, mode, budget, chunk)
    o_total, o_sum = orc.residual_plan(rows, feats, "chunk_topk" if mode == "topk" else mode, budget, chunk)
    assert k_total == o_total
    assert k_saved == (min(o_sum, o_total) if o_total else 0)
    assert ib == 4


def test_index_width_switches_at_2_31():
    from stacr_amd import kernels

    _lib()
    assert kernels.residual_plan(2**20, 2**11 - 1, "global_topk", 1e-6, 512)[2] == 4
    assert kernels.residual_plan(2**20, 2**11, "global_topk", 1e-6, 512)[2] == 8


def test_workspace_queries_and_error_paths():
    L = _lib().load()
    b = ctypes.c_size_t()
    assert L.stacr_save_workspace_bytes(8192, 1024, 8, 1, 1, 0.005, 512, 8, ctypes.byref(b)) == 0
    assert b.value > 0
    assert L.stacr_weight_grad_workspace_bytes(8192, 4096, 1024, 8, 41943, ctypes.byref(b)) == 0
    assert b.value >= (8192 + 1) * 4  # per-row residual offsets
    # rank outside the supported range -> UNSUPPORTED with a message
    assert L.stacr_save_workspace_bytes(64, 64, 33, 1, 0, 0.1, 16, 8, ctypes.byref(b)) == 2
    assert b"rank" in L.stacr_last_error()
    # bad dtype / bits / budget -> INVALID
    assert L.stacr_save_workspace_bytes(64, 64, 8, 7, 0, 0.1, 16, 8, ctypes.byref(b)) == 1
    assert L.stacr_save_workspace_bytes(64, 64, 8, 1, 0, 0.1, 16, 5, ctypes.byref(b)) == 1
    assert L.stacr_save_workspace_bytes(64, 64, 8, 1, 0, 1.5, 16, 8, ctypes.byref(b)) == 1
    assert L.stacr_save_workspace_bytes(64, 64, 8, 1, 0, 0.1, 0, 8, ctypes.byref(b)) == 1
    # more than 2^32 elements is outside the kernels' index range
    assert L.stacr_save_workspace_bytes(2**22, 2**10, 8, 1, 1, 0.1, 16, 8, ctypes.byref(b)) == 2
    # a null workspace is rejected before any launch
    rc = L.stacr_save(ctypes.c_void_p(16), ctypes.c_void_p(16), 1, 64, 64, 8, 0, 0.1, 16, 8, ctypes.c_void_p(16),
                      ctypes.c_void_p(16), 4, ctypes.c_void_p(16), ctypes.c_void_p(16), None, 0, None)
    assert rc == 1 and b"workspace" in L.stacr_last_error()
    rc = L.stacr_quantize_values(ctypes.c_void_p(16), 0, 10, 3, ctypes.c_void_p(16), ctypes.c_void_p(16),
                                 ctypes.c_void_p(16), 4, None)
    assert rc == 1


def test_python_errors_map_from_status_codes():
    from stacr_amd import _lib as L

    _lib()
    with pytest.raises(NotImplementedError):
        L.load().stacr_save_workspace_bytes(64, 64, 40, 1, 0, 0.1, 16, 8, ctypes.byref(ctypes.c_size_t()))
        L.check(2, "probe")
    with pytest.raises(ValueError):
        L.check(1, "probe")


def test_compact_output_and_c1_host_rules():
    """Host-side sizes and argument checks of the index stream and the C1 codec (no launches)."""
    L = _lib()
    lib = L.load()
    nb, mw = ctypes.c_int64(), ctypes.c_int64()
    assert lib.stacr_index_stream_sizes(41943, ctypes.byref(nb), ctypes.byref(mw)) == 0
    assert (nb.value, mw.value) == (164, 164 * 256)
    assert lib.stacr_index_stream_sizes(-1, ctypes.byref(nb), ctypes.byref(mw)) == 1
    assert lib.stacr_index_stream_sizes(1 << 31, ctypes.byref(nb), ctypes.byref(mw)) == 1
    assert lib.stacr_index_stream_encode(None, 3, 0, None, None, None, None, None) == 1  # idx_bytes 3
    ws = ctypes.c_size_t()
    assert lib.stacr_c1_workspace_bytes(8192, 1024, 96, ctypes.byref(ws)) == 0 and ws.value > 0
    for rank in (0, 129):
        assert lib.stacr_c1_workspace_bytes(8, 8, rank, ctypes.byref(ws)) == 1
    # int8 storage needs the int8 code and its scales; a float store cannot be int8
    assert lib.stacr_c1_store(None, 4, 8, None, 1, None, 1, None) == 1
    assert lib.stacr_c1_store(None, 4, 8, None, 0, None, 3, None) == 1
    assert lib.stacr_quantize_rows_int8(None, 7, 4, 8, None, None, None) == 1
