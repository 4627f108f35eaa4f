"""The torch-CPU restatement that bench.py times as its CPU baseline agrees with the C oracle.

Selections are compared as sets (torch.topk(sorted=False) leaves order open) on fp32 residuals
with no tie at the cut; codes and scale bit-exact; dW by rel-L2 against the fp64 oracle.
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis, make_grad
from oracle import oracle as orc
from oracle import torch_path as tp


@pytest.mark.parametrize("mode,rows,d,chunk,budget", [
    ("global_topk", 1024, 96, 256, 0.01),
    ("chunk_topk", 1000, 64, 128, 0.02),
    ("chunk_topk", 37, 24, 8, 0.05),  # per-chunk minimum of one entry, then the budget trim
])
def test_selection_codes_and_weight_grad_match_oracle(mode, rows, d, chunk, budget):
    x = make_activation(rows, d)
    q = make_basis(d, 4)
    g = make_grad(rows, 40)
    coeff, idx, codes, scale = tp.save(x, q, mode, budget, chunk, 8)
    cf = coeff.numpy()
    resid = orc.residual_act(x.numpy(), cf, q.numpy(), "f32")
    keys = np.sort(np.abs(resid).reshape(-1))[::-1]
    k = orc.residual_plan(rows, d, mode, budget, chunk)[0]
    oidx, oval = orc.select(resid, mode, budget, chunk)
    assert keys[oidx.size - 1] > keys[oidx.size]  # no tie at the cut: the set is unique
    order = np.argsort(idx.numpy())
    assert np.array_equal(idx.numpy()[order].astype(np.int64), oidx)
    oq, oscale = orc.quantize(oval, 8)
    assert np.array_equal(codes.numpy()[order], oq) and np.float32(scale.item()) == oscale
    assert idx.numel() <= k
    dw = tp.weight_grad(g, coeff, q, idx, codes, scale, d, False, torch.float32)
    vals = orc.dequantize(oq, oscale, 8, oidx.size)
    odw, _ = orc.weight_grad(g.numpy(), cf, q.numpy(), oidx, vals, d)
    assert np.linalg.norm(dw.double().numpy() - odw) / np.linalg.norm(odw) < 1e-5


def test_transposed_and_no_residual():
    x, q, g = make_activation(64, 32), make_basis(32, 4), make_grad(64, 16)
    coeff, idx, codes, scale = tp.save(x, q, "chunk_topk", 0.0, 16, 8)
    assert idx is None
    dw = tp.weight_grad(g, coeff, q, None, None, None, 32, True, torch.float32)
    odw, _ = orc.weight_grad(g.numpy(), coeff.numpy(), q.numpy(), np.zeros(0, np.int64), np.zeros(0, np.float32), 32)
    assert dw.shape == (32, 16)
    assert np.allclose(dw.double().numpy(), odw.T, rtol=1e-5, atol=1e-5)
