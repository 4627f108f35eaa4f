"""GPU parity of the "uniform", "block_sparse" and "sampled" selectors against the oracle.

On the kernel's own coefficients the selected indices and values are bit-exact against the
oracle's restatement (tests/test_oracle_selectors.py pins it).  "sampled" draws its positions
with torch's seeded generator on the GPU and its threshold with torch.quantile; the test repeats
both library calls on the oracle's magnitudes and compares the capped compaction bit for bit.
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _factors(rows, d, r, dtype, dev):
    from stacr_amd import kernels

    x = make_activation(rows, d).to(DT[dtype]).to(dev)
    q = make_basis(d, r).to(DT[dtype]).to(dev)
    coeff, _, _, _ = kernels.save(x, q, mode="chunk_topk", budget=0.0, chunk_rows=512, bits=0)
    resid = orc.residual_act(x.float().cpu().numpy(), coeff.float().cpu().numpy(), q.float().cpu().numpy(), dtype)
    return x, q, coeff, resid


CASES = [
    ("cfg3_c_fc_shape", 8192, 1024, 8, "bf16", 0.005),
    ("small_f32", 300, 96, 5, "f32", 0.1),
    ("odd_f16", 7, 13, 3, "f16", 0.5),
    ("rank32", 130, 64, 32, "bf16", 0.05),
]


@pytest.mark.parametrize("name,rows,d,r,dtype,budget", CASES)
def test_uniform_matches_oracle(name, rows, d, r, dtype, budget):
    from stacr_amd import kernels

    dev = _dev()
    print(f"[uniform] {name}", flush=True)
    x, q, coeff, resid = _factors(rows, d, r, dtype, dev)
    k = int(round(budget * rows * d))
    idx, val = kernels.select_uniform(x, coeff, q, k)
    idx_ref, val_ref = orc.select_uniform(resid, k)
    assert idx.dtype == torch.int32
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    assert np.array_equal(val.float().cpu().numpy(), val_ref)


BLOCK_CASES = [
    ("cfg3_c_fc_shape", 8192, 1024, 8, "bf16", 0.005, 512, 16),
    ("small_f32", 300, 96, 5, "f32", 0.1, 7, 8),
    ("f16_bs4", 100, 48, 4, "f16", 0.3, 512, 4),
    ("all_blocks", 20, 32, 2, "bf16", 1.0, 3, 16),
    ("one_row_chunks", 5, 16, 4, "f32", 0.25, 1, 4),
]


@pytest.mark.parametrize("name,rows,d,r,dtype,budget,chunk,bs", BLOCK_CASES)
def test_block_sparse_matches_oracle(name, rows, d, r, dtype, budget, chunk, bs):
    from stacr_amd import kernels

    dev = _dev()
    print(f"[block_sparse] {name}", flush=True)
    x, q, coeff, resid = _factors(rows, d, r, dtype, dev)
    idx, val = kernels.select_block_sparse(x, coeff, q, budget, chunk, bs)
    idx_ref, val_ref = orc.select_block_sparse(resid, budget, chunk, bs, dtype)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    assert np.array_equal(val.float().cpu().numpy(), val_ref)


def test_block_sparse_falls_back_to_chunk_topk_when_blocks_do_not_tile_rows():
    from stacr_amd.layers import _select_residual

    dev = _dev()
    x, q, coeff, _ = _factors(64, 30, 4, "bf16", dev)
    i_b, v_b = _select_residual(x, coeff, q, 0.1, 16, "block_sparse", 16, 0.1)
    i_c, v_c = _select_residual(x, coeff, q, 0.1, 16, "chunk_topk", 16, 0.1)
    assert torch.equal(i_b, i_c) and torch.equal(v_b, v_c)


SAMPLED_CASES = [
    ("cfg3_c_fc_shape", 8192, 1024, 8, "bf16", 0.005, 0.1),
    ("small_f32", 300, 96, 5, "f32", 0.1, 0.1),
    ("f16_min_sample", 64, 64, 4, "f16", 0.05, 0.01),
]


@pytest.mark.parametrize("name,rows,d,r,dtype,budget,ratio", SAMPLED_CASES)
def test_sampled_matches_oracle(name, rows, d, r, dtype, budget, ratio):
    from stacr_amd import kernels

    dev = _dev()
    print(f"[sampled] {name}", flush=True)
    x, q, coeff, resid = _factors(rows, d, r, dtype, dev)
    total = rows * d
    k_total = int(round(budget * total))
    gen = torch.Generator(device=dev).manual_seed(0)
    n = max(1024, int(total * ratio))
    pos = torch.randint(total, (n,), device=dev, generator=gen)
    mags = kernels.sample_magnitudes(x, coeff, q, pos)
    flat = resid.reshape(-1)
    mag_ref = np.abs(flat[pos.cpu().numpy()])
    assert np.array_equal(mags.float().cpu().numpy(), mag_ref)
    thr = torch.quantile(torch.from_numpy(mag_ref).to(dev), 1.0 - budget)
    idx, val = kernels.select_sampled(x, coeff, q, budget, ratio, k_total)
    idx_ref, val_ref = orc.select_threshold(resid, float(thr.item()), dtype, k_total)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    assert np.array_equal(val.float().cpu().numpy(), val_ref)
    assert idx.numel() <= k_total


@pytest.mark.parametrize("thr,cap", [(0.0, 700), (0.0, 0), (1e30, 500), (float("nan"), 500), (0.7, 10 ** 6),
                                     (0.7, None), (1e30, None)])
def test_threshold_compaction_cap_and_empty(thr, cap):
    """Capped, empty and uncapped selections; cap None is the count-only call (cap 0 at the C ABI),
    then the selection sized by that count."""
    from stacr_amd import kernels

    dev = _dev()
    x, q, coeff, resid = _factors(40, 32, 4, "bf16", dev)
    cap = min(cap, 40 * 32) if cap is not None else None
    idx, val = kernels.select_threshold(x, coeff, q, torch.tensor(thr), cap)
    idx_ref, val_ref = orc.select_threshold(resid, thr, "bf16", 40 * 32 if cap is None else cap)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref)
    assert np.array_equal(val.float().cpu().numpy(), val_ref)
