"""The allocation-free weight gradient (stacr_weight_grad_noalloc) against stacr_weight_grad.

Both run the same kernels; the only difference is where the plan lives (a static per-GPU device
array instead of a caller workspace).  Two calls in a row, the second on a smaller problem, each
checked against stacr_weight_grad on the same inputs, dbias bit-equal in both:
* the first (bf16 Conv1D 1024 -> 4096, d_out a multiple of 16) runs the matrix-core tiles kernels,
  whose sums have a fixed order, so dW is bit-equal too (a plan word left over from an earlier call
  in the shared scratch would show);
* the second (fp32, d_out = 1000, not a multiple of 16) runs the general kernels, which add the
  sparse term's pieces in LDS arrival order: dW within rel-L2 1e-6.
An oversized problem is refused on the host.
"""
import ctypes

import pytest
import torch

from gpu_cases import make_activation, make_basis, make_grad

pytestmark = pytest.mark.gpu


def _p(t):
    return ctypes.c_void_p(t.data_ptr() if t is not None and t.numel() else None)


def _noalloc(g, coeff, q, res, bits, transposed, out_dtype, bias_dtype):
    from stacr_amd import _lib, kernels

    rows, d_out = g.shape
    d_in, rank = q.shape
    idx, data, scale = res if res is not None else (None, None, None)
    nnz = idx.numel() if idx is not None else 0
    dw = torch.empty((d_in, d_out) if transposed else (d_out, d_in), dtype=out_dtype, device=g.device)
    db = torch.empty(d_out, dtype=bias_dtype, device=g.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(g.device).cuda_stream)
    rc = _lib.load().stacr_weight_grad_noalloc(
        _p(g), kernels.dtype_code(g.dtype), rows, d_out, _p(coeff), _p(q), d_in, rank, _p(idx),
        idx.element_size() if idx is not None else 4, _p(data), _p(scale), bits, 0, nnz, int(transposed), _p(dw),
        kernels.dtype_code(out_dtype), _p(db), kernels.dtype_code(bias_dtype), stream)
    _lib.check(rc, "stacr_weight_grad_noalloc")
    return dw, db


def _rel(a, b):
    a, b = a.double(), b.double()
    return ((a - b).norm() / b.norm()).item()


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def test_noalloc_matches_workspace_entry_point_twice(dev):
    from stacr_amd import kernels

    # first the north-star layer (bf16, Conv1D, global top-k), then a smaller fp32 problem
    for rows, d_in, d_out, dtype, transposed, mode in ((8192, 1024, 4096, torch.bfloat16, True, "global_topk"),
                                                        (2048, 768, 1000, torch.float32, False, "chunk_topk")):
        print("CASE noalloc", rows, d_in, d_out, dtype, flush=True)
        x = make_activation(rows, d_in, lognormal=True).to(dev, dtype)
        q = make_basis(d_in, 8).to(dev, dtype)
        g = make_grad(rows, d_out).to(dev, dtype)
        coeff, idx, data, scale = kernels.save(x, q, mode=mode, budget=0.005, chunk_rows=512, bits=8)
        want_dw, want_db = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, transposed, dtype, dtype)
        got_dw, got_db = _noalloc(g, coeff, q, (idx, data, scale), 8, transposed, dtype, dtype)
        torch.cuda.synchronize()
        assert torch.equal(got_db, want_db)
        if d_out % 16 == 0:  # tiles kernels: fixed-order sums
            assert torch.equal(got_dw, want_dw), f"rel-L2 {_rel(got_dw, want_dw):.3g}"
        else:  # general kernels: arrival-order fp32 sums of the sparse term
            assert _rel(got_dw, want_dw) <= 1e-6


def test_noalloc_refuses_problems_above_its_scratch(dev):
    from stacr_amd import _lib

    need = ctypes.c_size_t()
    shape = (65536, 4096, 16384, 16, 8_000_000)  # rows, d_out, d_in, rank, nnz
    _lib.check(_lib.load().stacr_weight_grad_workspace_bytes(*shape, ctypes.byref(need)), "workspace")
    assert need.value > (48 << 20)
    dummy = torch.empty(16, device=dev)
    stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    rows, d_out, d_in, rank, nnz = shape
    rc = _lib.load().stacr_weight_grad_noalloc(_p(dummy), 1, rows, d_out, _p(dummy), _p(dummy), d_in, rank,
                                               _p(dummy), 4, _p(dummy), _p(dummy), 8, 0, nnz, 0, _p(dummy), 1, None, 1,
                                               stream)
    assert rc == _lib.STACR_ERR_UNSUPPORTED
    assert "static scratch" in _lib.load().stacr_last_error().decode()
