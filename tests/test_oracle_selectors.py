"""Pins of the oracle's "uniform", "block_sparse" and "sampled" selectors (stacr/layers.py:55-99).

uniform: the reference's own per-chunk loop (ceil boundaries, floor positions), run here in
exact integers, must give the oracle's closed form for every chunk size.  block_sparse: energies
against torch's dtype-native square-and-sum on the CPU, selection against brute-force sorting,
counts against the reference's stored_bytes rule.  sampled: the threshold comparison against
torch's own `magnitude >= threshold` promotion on the CPU.
"""
import math

import numpy as np
import pytest
import torch

from oracle import oracle as orc

TDT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


@pytest.mark.parametrize("rows,feats,budget", [(5, 16, 0.25), (37, 11, 0.1), (512, 64, 0.005), (3, 3, 1.0)])
@pytest.mark.parametrize("chunk_rows", [1, 2, 7, 512])
def test_uniform_closed_form_equals_reference_chunk_loop(rows, feats, budget, chunk_rows):
    total = rows * feats
    k = int(round(budget * total))
    got = orc.uniform_positions(total, k)
    ref = []
    for start in range(0, rows, chunk_rows):  # stacr/layers.py:89-98 in exact integers
        stop = min(start + chunk_rows, rows)
        first = -((-start * feats * k) // total)
        last = -((-stop * feats * k) // total)
        ref.extend((i * total) // k for i in range(first, last))
        # the reference's float ceil agrees with the exact one at these sizes
        assert first == math.ceil(start * feats * k / total) and last == math.ceil(stop * feats * k / total)
    assert got.tolist() == ref
    assert got.size == k and np.all(np.diff(got) > 0) and got[-1] < total


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_block_energies_match_torch_square_sum(dtype):
    rng = np.random.default_rng(1)
    r = torch.from_numpy(rng.standard_normal((64, 96)).astype(np.float32)).to(TDT[dtype])
    ref = r.reshape(-1, 16).square().sum(1).float().numpy()
    got = orc.block_energies(r.float().numpy(), 16, dtype)
    if dtype == "f32":  # the sum order of torch's reduction is its own
        np.testing.assert_allclose(got, ref, rtol=1e-6)
    else:
        assert np.mean(got == ref) >= 0.99
        np.testing.assert_allclose(got, ref, rtol=2 ** -7)


@pytest.mark.parametrize("rows,feats,chunk_rows,bs,budget", [(5, 16, 2, 4, 0.25), (40, 32, 7, 8, 0.1),
                                                            (9, 12, 512, 3, 0.5), (6, 8, 1, 8, 1.0)])
def test_block_sparse_selection_matches_brute_force(rows, feats, chunk_rows, bs, budget):
    rng = np.random.default_rng(rows)
    resid = rng.standard_normal((rows, feats)).astype(np.float32)
    resid[rng.random((rows, feats)) < 0.2] = 0.5  # equal-energy blocks
    idx, val = orc.select_block_sparse(resid, budget, chunk_rows, bs, "f32")
    energy = orc.block_energies(resid, bs, "f32")
    per = chunk_rows * feats // bs
    expect = []
    for c, start in enumerate(range(0, rows, chunk_rows)):
        blocks = list(range(c * per, min((c + 1) * per, energy.size)))
        count = max(1, int(round(budget * len(blocks))))
        best = sorted(blocks, key=lambda b: (-float(energy[b]), b))[:count]
        expect.extend(e for b in sorted(best) for e in range(b * bs, (b + 1) * bs))
    assert idx.tolist() == expect
    assert np.array_equal(val, resid.reshape(-1)[idx])
    # reference tests/test_memory.py:43-65: 5 rows x 16, one-row chunks, blocks of 4, budget 0.17
    assert sum(orc.block_sparse_counts(5, 16, 0.17, 1, 4)) * 4 == 20


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
def test_threshold_comparison_follows_torch_promotion(dtype):
    rng = np.random.default_rng(2)
    r = torch.from_numpy(rng.standard_normal(5000).astype(np.float32)).to(TDT[dtype])
    mag = r.abs()
    for thr in (0.5, 1.0117, 1.004, 2.3333, 0.0):
        t = torch.tensor(thr, dtype=torch.float32)
        ref = (mag >= t).nonzero(as_tuple=True)[0][:300].numpy()
        idx, val = orc.select_threshold(r.float().numpy(), thr, dtype, 300)
        assert np.array_equal(idx, ref)
        assert np.array_equal(val, r.float().numpy()[ref])


def _brute_adaptive_blocks(resid, budget, chunk_rows, bs, dtype):
    """Plain-Python restatement: energies block by block, candidates chunk by chunk, global cut."""
    rows, d = resid.shape
    bpr = -(-d // bs)
    energies = []
    for r in range(rows):
        for b in range(bpr):
            acc = np.float32(0)
            for o in range(bs):
                c = b * bs + o
                v = np.float32(resid[r, c]) if c < d else np.float32(0)
                acc = np.float32(acc + orc.round_to(np.array([v * v], np.float32), dtype)[0])
            energies.append(float(orc.round_to(np.array([acc], np.float32), dtype)[0]))
    k = min(int(rows * d * budget), rows * d)
    k_blocks = max(1, -(-k // bs))
    chunk = min(chunk_rows, rows)
    per = max(1, (k_blocks * chunk + rows - 1) // rows)
    cand = []
    for start in range(0, rows, chunk):
        blocks = list(range(start * bpr, min(start + chunk, rows) * bpr))
        blocks.sort(key=lambda i: (-energies[i], i))
        cand += blocks[:per]
    cand.sort(key=lambda i: (-energies[i], i))
    kept = sorted(cand[:k_blocks])
    idx = [(b // bpr) * d + (b % bpr) * bs + o for b in kept for o in range(bs) if (b % bpr) * bs + o < d]
    return np.array(idx, np.int64)


@pytest.mark.parametrize("rows,d,chunk,bs,budget,dtype", [
    (12, 40, 5, 16, 0.1, "f32"),    # padded row ends, three chunks, global cut
    (9, 32, 4, 8, 0.3, "bf16"),     # no padding, partial last chunk
    (7, 10, 7, 4, 0.5, "f16"),      # one chunk, padding, many blocks kept
    (30, 17, 8, 16, 0.02, "f32"),   # blocks wider than the padding, per-chunk minimum of one
])
def test_adaptive_block_sparse_matches_brute_force(rows, d, chunk, bs, budget, dtype):
    rng = np.random.default_rng(rows * d)
    resid = orc.round_to(rng.standard_normal((rows, d)).astype(np.float32) * rng.uniform(0.1, 3, (1, d)), dtype)
    idx, vals = orc.adaptive_select_block_sparse(resid, budget, chunk, bs, dtype)
    assert np.array_equal(idx, _brute_adaptive_blocks(resid, budget, chunk, bs, dtype))
    assert np.array_equal(vals, resid.reshape(-1)[idx])


def test_adaptive_block_sparse_equals_projection_rule_when_counts_agree():
    """With one chunk and feats % bs == 0 both engines keep the same number of whole blocks."""
    rng = np.random.default_rng(3)
    resid = orc.round_to(rng.standard_normal((16, 64)).astype(np.float32), "bf16")
    a, _ = orc.adaptive_select_block_sparse(resid, 0.25, 16, 16, "bf16")   # k 256 -> 16 blocks
    b, _ = orc.select_block_sparse(resid, 0.25, 16, 16, "bf16")            # round(0.25 * 64) = 16
    assert np.array_equal(a, b)


def test_adaptive_block_energy_matches_torch_padded_sum():
    """The reference forms block scores with torch ops on the padded residual in its dtype
    (stacr/adaptive.py:1857-1868): F.pad, view, square, sum(dim=2).  16-bit scores are bit-equal
    (the final rounding hides the fp32 summation order); fp32 scores agree to a few ulps, the
    order torch's own reduction adds in being internal to it."""
    import torch
    from torch.nn import functional as F

    rng = np.random.default_rng(8)
    for dtype, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)):
        resid = orc.round_to(rng.standard_normal((6, 37)).astype(np.float32), dtype)
        t = F.pad(torch.from_numpy(resid).to(tdt), (0, 48 - 37)).view(6, 3, 16)
        want = (t * t).sum(dim=2).float().reshape(-1).numpy()
        got = orc.adaptive_block_energies(resid, 16, dtype)
        if dtype == "f32":
            assert np.allclose(got, want, rtol=16 * np.finfo(np.float32).eps, atol=0)
        else:
            assert np.array_equal(got, want)
