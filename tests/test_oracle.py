"""Pins the CPU oracle (oracle/) before anything is compared against it.

Each check is chosen so that a plausible mistake in the oracle (a dropped trim, a wrong k rounding,
a transposed index, a sign slip in the nibble packing) fails at least one of them:
known answers from the reference's own tests, closed forms, and brute force with an independent
algorithm (numpy lexsort instead of the oracle's quickselect).
"""
import numpy as np
import pytest

from oracle import oracle as orc


# ------------------------------------------------------------------ selection known answers
def test_global_topk_vs_chunk_known_answer():
    """Reference tests/test_integration.py:106-114."""
    x = np.array([[100.0, 90.0, 80.0, 70.0], [4.0, 3.0, 2.0, 1.0]], np.float32)
    idx, val = orc.select(x, "global_topk", 0.5, 1)
    assert set(idx.tolist()) == {0, 1, 2, 3}
    assert set(val.tolist()) == {100.0, 90.0, 80.0, 70.0}
    idx, _ = orc.select(x, "chunk_topk", 0.5, 1)
    assert set(idx.tolist()) == {0, 1, 4, 5}


def test_single_row_topk_known_answer():
    """Reference tests/test_residual.py:6-11: budget .5 of [1,-3,2,.5] keeps two, max 3."""
    r = np.array([[1.0, -3.0, 2.0, 0.5]], np.float32)
    idx, val = orc.select(r, "chunk_topk", 0.5, 512)
    assert idx.tolist() == [1, 2]
    assert np.abs(val).max() == 3.0
    assert val.tolist() == [-3.0, 2.0]


def test_trim_count_matches_reference_capacity_rule():
    """Reference stored_bytes rule (stacr/layers.py:417-449; tests/test_memory.py:366-388):
    5x16 rows of one row per chunk at budget .17 -> chunks keep 3 each (15) -> trimmed to 14."""
    rng = np.random.default_rng(0)
    r = rng.standard_normal((5, 16)).astype(np.float32)
    assert orc.residual_plan(5, 16, "chunk_topk", 0.17, 1) == (14, 15)
    idx, _ = orc.select(r, "chunk_topk", 0.17, 1)
    assert idx.size == 14
    # the trim drops the globally smallest of the 15 chunk survivors
    keep = []
    for row in range(5):
        order = np.lexsort((np.arange(16), -np.abs(r[row])))[:3]
        keep += [row * 16 + int(i) for i in order]
    keep = np.array(keep)
    mags = np.abs(r.reshape(-1)[keep])
    drop = keep[np.lexsort((keep, mags))[0]]
    assert sorted(set(keep.tolist()) - {int(drop)}) == idx.tolist()


@pytest.mark.parametrize(
    "rows,feats,mode,budget,chunk,expected",
    [
        (4096, 768, "chunk_topk", 0.005, 512, (15729, 15728)),  # config 1
        (8192, 1024, "global_topk", 0.005, 512, (41943, 41943)),  # config 3 c_fc
        (8192, 4096, "global_topk", 0.005, 512, (167772, 167772)),  # config 3 c_proj
        (8192, 1024, "chunk_topk", 0.005, 512, (41943, 41936)),  # config 5, d_in 1024
        (8192, 4096, "chunk_topk", 0.005, 512, (167772, 167776)),  # config 5, d_in 4096: trim 4
        (5, 16, "chunk_topk", 0.005, 512, (0, 0)),  # round(0.4) == 0 -> no residual
        (2, 4, "chunk_topk", 0.0625, 1, (0, 0)),  # round(0.5) == 0: half to even
        (2, 4, "chunk_topk", 0.1875, 1, (2, 2)),  # round(1.5) == 2
    ],
)
def test_k_rules(rows, feats, mode, budget, chunk, expected):
    assert orc.residual_plan(rows, feats, mode, budget, chunk) == expected


def _brute_select(resid, mode, budget, chunk_rows):
    """Independent restatement by full lexsort (no quickselect, no composite keys)."""
    rows, d = resid.shape
    total = rows * d
    k_total = int(round(budget * total))
    if k_total <= 0:
        return np.zeros(0, np.int64)
    flat = resid.reshape(-1)
    mag = np.abs(flat)
    if mode == "global_topk":
        order = np.lexsort((np.arange(total), -mag))
        return np.sort(order[:k_total])
    sel = []
    for start in range(0, rows, chunk_rows):
        stop = min(start + chunk_rows, rows)
        ids = np.arange(start * d, stop * d)
        k = max(1, min(ids.size, int(round(budget * ids.size))))
        order = np.lexsort((ids, -mag[ids]))
        sel.append(ids[order[:k]])
    sel = np.concatenate(sel)
    if sel.size > k_total:
        order = np.lexsort((sel, -mag[sel]))
        sel = sel[order[:k_total]]
    return np.sort(sel)


@pytest.mark.parametrize("mode", ["chunk_topk", "global_topk"])
@pytest.mark.parametrize(
    "rows,d,budget,chunk", [(37, 24, 0.05, 8), (64, 33, 0.01, 16), (9, 5, 0.3, 2), (100, 7, 0.17, 3)]
)
def test_selection_matches_brute_force(mode, rows, d, budget, chunk):
    rng = np.random.default_rng(rows * 1000 + d)
    r = rng.standard_normal((rows, d)).astype(np.float32)
    r[rng.random(r.shape) < 0.05] *= 20.0
    idx, val = orc.select(r, mode, budget, chunk)
    ref = _brute_select(r, mode, budget, chunk)
    assert idx.tolist() == ref.tolist()
    assert np.array_equal(val, r.reshape(-1)[ref])


def test_ties_take_lowest_flat_index():
    r = np.ones((4, 8), np.float32)
    r[:, ::2] *= -1.0  # equal magnitudes, mixed signs
    idx, _ = orc.select(r, "global_topk", 0.25, 512)
    assert idx.tolist() == list(range(8))
    idx, _ = orc.select(r, "chunk_topk", 0.25, 2)
    assert idx.tolist() == [0, 1, 2, 3, 16, 17, 18, 19]
    z = np.zeros((3, 4), np.float32)
    idx, val = orc.select(z, "global_topk", 0.5, 512)
    assert idx.tolist() == list(range(6)) and not val.any()


# ------------------------------------------------------------------ quantization closed forms
def test_quantize_tiny_values_keep_positive_fp32_scale():
    """Reference tests/test_integration.py:147-152."""
    v = np.array([0.0, 1e-6, -1e-6], np.float32)
    q, scale = orc.quantize(v, 8)
    assert scale.dtype == np.float32 and scale > 0
    assert np.allclose(orc.dequantize(q, scale, 8, 3), v, atol=1e-8)
    q, scale = orc.quantize(np.zeros(4, np.float32), 8)
    assert scale == np.float32(np.finfo(np.float32).tiny) and not q.any()


def test_quantize_exact_scale_round_half_even_and_clamp():
    s = 2.0**-7
    v = np.array([127, 0.5, 1.5, 2.5, -3.5, -127, 64.25], np.float32) * np.float32(s)
    q, scale = orc.quantize(v, 8)
    assert scale == np.float32(s)
    assert q.tolist() == [127, 0, 2, 2, -4, -127, 64]
    q, scale = orc.quantize(np.array([7, -7, 0.5, 1.5, 2.5], np.float32) * 0.125, 4)
    assert scale == np.float32(0.125)
    assert q.tolist() == [7, -7, 0, 2, 2]
    assert orc.pack_int4(q).tolist() == [0x97, 0x20, 0x02]


def test_quantize_bits0_is_passthrough():
    v = np.array([1.5, -2.0], np.float32)
    _, scale = orc.quantize(v, 0)
    assert scale == 1.0


def test_int4_nibbles_round_trip_and_layout():
    q = np.arange(-8, 8, dtype=np.int8)
    packed = orc.pack_int4(q)
    assert packed[0] == ((-8 & 0xF) | ((-7 & 0xF) << 4))
    assert np.array_equal(orc.unpack_int4(packed, q.size), q)
    odd = np.array([3, -1, 5], np.int8)
    p = orc.pack_int4(odd)
    assert p.tolist() == [0xF3, 0x05]
    assert np.array_equal(orc.unpack_int4(p, 3), odd)


# ------------------------------------------------------------------ residual arithmetic
def test_residual_close_to_fp64_and_exact_in_span():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 40)).astype(np.float32)
    q = np.linalg.qr(rng.standard_normal((40, 8)))[0].astype(np.float32)
    c = (x.astype(np.float64) @ q).astype(np.float32)
    r = orc.residual_act(x, c, q, "f32")
    r64 = x.astype(np.float64) - c.astype(np.float64) @ q.astype(np.float64).T
    assert np.abs(r - r64).max() <= 1e-5
    # X exactly in the span of a unit-vector basis with exact coefficients -> zero residual
    q = np.zeros((40, 4), np.float32)
    q[[3, 9, 17, 31], [0, 1, 2, 3]] = 1.0
    c = rng.integers(-5, 5, (16, 4)).astype(np.float32)
    x = c @ q.T
    assert not orc.residual_act(x, c, q, "f32").any()


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rank", [1, 5, 8, 16])
def test_residual_matches_torch_dtype_native_ops(dtype, rank):
    """The reference forms the residual with torch ops in the activation dtype
    (stacr/layers.py:32,73); torch's CPU kernels give the same bits as the restatement."""
    import torch

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    rng = np.random.default_rng(rank)
    q = torch.from_numpy(np.linalg.qr(rng.standard_normal((384, rank)))[0].astype(np.float32)).to(tdt)
    x = torch.from_numpy((rng.standard_normal((256, 384)) * 2).astype(np.float32)).to(tdt)
    c = x.mm(q)
    ref = (x - c.mm(q.t())).float().numpy()
    got = orc.residual_act(x.float().numpy(), c.float().numpy(), q.float().numpy(), dtype)
    assert np.array_equal(got, ref)
    # one rounding of the exact difference disagrees on many entries: the pin sees both roundings
    one = orc.round_to((x.double() - c.double().mm(q.double().t())).float().numpy(), dtype)
    assert np.mean(one != ref) > 0.02


@pytest.mark.parametrize("dtype", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("rank", [1, 5, 8, 16])
def test_reconstruct_matches_torch_dtype_native_ops(dtype, rank):
    """The saved-tensor hooks' unpack (stacr/compressor.py:127-133, stacr/residual.py:13-20) with
    torch's CPU ops: coeff.mm(basis.t()) in the dtype, plus the dense residual (zeros elsewhere)."""
    import torch

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}[dtype]
    rng = np.random.default_rng(10 + rank)
    q = torch.from_numpy(np.linalg.qr(rng.standard_normal((384, rank)))[0].astype(np.float32)).to(tdt)
    x = torch.from_numpy((rng.standard_normal((96, 384)) * 2).astype(np.float32)).to(tdt)
    c = x.mm(q)
    low = c.mm(q.t())
    assert np.array_equal(orc.lowrank(c.float().numpy(), q.float().numpy(), dtype), low.float().numpy())
    idx = np.sort(rng.choice(96 * 384, 500, replace=False))
    vals = torch.from_numpy(rng.standard_normal(500).astype(np.float32)).to(tdt)
    dense = torch.zeros(96 * 384, dtype=tdt)
    dense[torch.from_numpy(idx)] = vals
    ref = (low + dense.reshape(96, 384)).float().numpy()
    got = orc.reconstruct(c.float().numpy(), q.float().numpy(), idx, vals.float().numpy(), dtype)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))  # bits, signed zeros included
    assert np.array_equal(orc.reconstruct(c.float().numpy(), q.float().numpy(), None, None, dtype), low.float().numpy())


def test_reconstruct_closed_forms_and_signed_zeros():
    """Unit basis vectors and exact coefficients give X back exactly; an empty residual still turns
    -0 into +0 (the reference adds a zero tensor), while no residual leaves -0; C = 0 gives the
    dense residual."""
    rng = np.random.default_rng(4)
    q = np.zeros((40, 4), np.float32)
    q[[3, 9, 17, 31], [0, 1, 2, 3]] = 1.0
    c = rng.integers(-5, 5, (16, 4)).astype(np.float32)
    assert np.array_equal(orc.reconstruct(c, q, None, None, "bf16"), c @ q.T)
    # a tiny negative product rounds to -0 in fp16 (the chain itself never yields -0 from +0)
    ct, qt = np.array([[-1e-8]], np.float32), np.array([[1.0]], np.float32)
    low = orc.lowrank(ct, qt, "f16")
    assert low[0, 0] == 0 and np.signbit(low[0, 0])
    assert np.signbit(orc.reconstruct(ct, qt, None, None, "f16")[0, 0])
    assert not np.signbit(orc.reconstruct(ct, qt, np.zeros(0, np.int64), np.zeros(0, np.float32), "f16")[0, 0])
    # at an entry: rnd(L + v), with L = -0 and v = -0 staying -0
    assert np.signbit(orc.reconstruct(ct, qt, np.array([0]), np.array([-0.0], np.float32), "f16")[0, 0])
    idx = np.array([0, 7, 79], np.int64)
    vals = np.array([1.5, -2.0, 3.25], np.float32)
    out = orc.reconstruct(np.zeros((2, 4), np.float32), q, idx, vals, "f32")
    want = np.zeros(80, np.float32)
    want[idx] = vals
    assert np.array_equal(out.reshape(-1), want)


# ------------------------------------------------------------------ weight gradient closed forms
def test_weight_grad_full_budget_equals_dense():
    rng = np.random.default_rng(5)
    n, d_in, d_out, r = 12, 10, 7, 3
    x = rng.standard_normal((n, d_in)).astype(np.float32)
    g = rng.standard_normal((n, d_out)).astype(np.float32)
    q = np.linalg.qr(rng.standard_normal((d_in, r)))[0].astype(np.float32)
    c = (x.astype(np.float64) @ q).astype(np.float32)
    resid = orc.residual_act(x, c, q, "f32")
    idx, val = orc.select(resid, "global_topk", 1.0, 512)
    assert idx.size == n * d_in
    dw, db = orc.weight_grad(g, c, q, idx, val, d_in)
    dense = g.astype(np.float64).T @ x.astype(np.float64)
    assert np.abs(dw - dense).max() <= 1e-5 * np.abs(dense).max()
    assert np.allclose(db, g.astype(np.float64).sum(0))


def test_weight_grad_single_entry_and_identity_basis():
    rng = np.random.default_rng(6)
    n, d_in, d_out = 5, 6, 4
    g = rng.standard_normal((n, d_out)).astype(np.float32)
    c = np.zeros((n, 2), np.float32)
    q = np.zeros((d_in, 2), np.float32)
    dw, _ = orc.weight_grad(g, c, q, np.array([2 * d_in + 3]), np.array([1.5], np.float32), d_in)
    expect = np.zeros((d_out, d_in))
    expect[:, 3] = 1.5 * g[2].astype(np.float64)
    assert np.array_equal(dw, expect)
    # rank-d identity basis: C = X exactly, so dW = G^T X with no residual
    x = rng.standard_normal((n, d_in)).astype(np.float32)
    dw, _ = orc.weight_grad(g, x, np.eye(d_in, dtype=np.float32), np.zeros(0, np.int64),
                            np.zeros(0, np.float32), d_in)
    assert np.allclose(dw, g.astype(np.float64).T @ x.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_weight_grad_rejects_out_of_range_indices():
    """Indices a kernel emitted are checked before the oracle indexes G with them: a bad one fails
    the calling test (AssertionError) instead of crashing the test process."""
    rng = np.random.default_rng(5)
    g = rng.standard_normal((8, 3)).astype(np.float32)
    c = rng.standard_normal((8, 2)).astype(np.float32)
    q = rng.standard_normal((4, 2)).astype(np.float32)
    vals = np.ones(2, np.float32)
    for bad in ([0, 32], [-1, 3], [5, 1 << 40]):
        with pytest.raises(AssertionError, match="out of range"):
            orc.weight_grad(g, c, q, np.array(bad, np.int64), vals, 4)
    with pytest.raises(AssertionError, match="ascending"):
        orc.check_indices(np.array([3, 3, 7]), 32, ascending=True)
    orc.check_indices(np.array([0, 3, 31]), 32, ascending=True)
    # the C entry point itself refuses (returns non-zero) without the Python pre-check
    idx = np.array([0, 32], np.int64)
    dw = np.empty((3, 4)); db = np.empty(3)
    rc = orc.lib().orc_weight_grad(orc._ptr(g), 8, 3, orc._ptr(c), orc._ptr(q), 4, 2, orc._ptr(idx),
                                   orc._ptr(vals), 2, orc._ptr(dw), orc._ptr(db))
    assert rc != 0
