"""Pins of the oracle's adaptive-engine restatements (stacr/adaptive.py, stacr/index_compression.py).

Each check compares the restatement with something independent of it: torch's own dtype-native
arithmetic (the reference runs on it), brute force, closed forms, and the reference's known
answers (tests/test_adaptive.py:186-195,211-218,231-239).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def _bits_f32(n, seed):
    rng = np.random.default_rng(seed)
    u = rng.integers(0, 2**32, size=n, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x3F800000, 0x3F808000, 0x3F818000, 0x387FC000, 0x33800000, 0x33000000,
                        0x477FE000, 0x477FF000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x00000001, 0x1F800000],
                       np.uint32)
    return np.concatenate([u, special]).view(np.float32)


def test_dtype_rounding_matches_torch_casts():
    v = _bits_f32(20000, 1)
    bf = np.array([orc.round_dtype_scalar(float(f), "bf16") for f in v], np.float32)
    hf = np.array([orc.round_dtype_scalar(float(f), "f16") for f in v], np.float32)
    t = torch.from_numpy(v.copy())
    ref_bf = t.to(torch.bfloat16).float().numpy()
    ref_hf = t.to(torch.float16).float().numpy()
    for got, ref in ((bf, ref_bf), (hf, ref_hf)):
        nan = np.isnan(ref)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_residual_act_close_to_fp64_and_exact_in_span(dtype):
    rng = np.random.default_rng(2)
    rows, d, r = 48, 40, 5
    q, _ = np.linalg.qr(rng.standard_normal((d, r)))
    q = orc.round_to(q.astype(np.float32), dtype)
    c = orc.round_to(rng.standard_normal((rows, r)).astype(np.float32), dtype)
    x = orc.round_to(rng.standard_normal((rows, d)).astype(np.float32), dtype)
    got = orc.residual_act(x, c, q, dtype)
    p64 = c.astype(np.float64) @ q.astype(np.float64).T
    ref = orc.round_to((x.astype(np.float64) - orc.round_to(p64.astype(np.float32), dtype)).astype(np.float32), dtype)
    ulp = {"f32": 2.0**-22, "bf16": 2.0**-7, "f16": 2.0**-9}[dtype]
    assert np.all(np.abs(got - ref) <= ulp * (np.abs(x) + np.abs(p64) + 1e-30) * 2)
    # identity basis columns: the projection of c onto them is c itself, so x == c there gives 0
    qi = np.eye(d, r, dtype=np.float32)
    xi = np.zeros((rows, d), np.float32)
    xi[:, :r] = c
    assert np.all(orc.residual_act(xi, c, qi, dtype) == 0)


@pytest.mark.parametrize("rows,d,chunk,kc,kt", [(37, 11, 8, 9, 30), (64, 16, 16, 40, 100), (10, 7, 3, 50, 20),
                                                (5, 4, 512, 3, 3)])
def test_select_explicit_matches_brute_force(rows, d, chunk, kc, kt):
    rng = np.random.default_rng(rows + d)
    resid = rng.standard_normal((rows, d)).astype(np.float32)
    resid[rng.random((rows, d)) < 0.1] = 0.5  # ties
    idx, val = orc.select_explicit(resid, chunk, kc, kt)
    flat = resid.reshape(-1)
    cand = []
    for s in range(0, rows, chunk):
        lo, hi = s * d, min(s + chunk, rows) * d
        seg = np.arange(lo, hi)
        order = np.lexsort((seg, -np.abs(flat[seg])))
        cand.extend(seg[order[:min(kc, hi - lo)]])
    cand = np.array(cand)
    if cand.size > kt:
        order = np.lexsort((cand, -np.abs(flat[cand])))
        cand = cand[order[:kt]]
    assert np.array_equal(idx, np.sort(cand))
    assert np.array_equal(val, flat[idx])


def test_adaptive_k_rules_match_config_counts():
    # configuration 4 (16 x 2048 tokens): 335,544 entries for d_in 2048 (5,243 per chunk),
    # 1,342,177 for d_in 8192 (20,972 per chunk)
    assert orc.adaptive_plan(32768, 2048, 0.005)[:2] == (335544, 5243)
    assert orc.adaptive_plan(32768, 8192, 0.005)[:2] == (1342177, 20972)
    assert orc.adaptive_plan(10, 10, 0.005)[0] == 0          # floor(0.5) = 0: no residual
    assert orc.adaptive_plan(100, 300, 0.5)[3] == np.int16   # 30000 < 32768
    assert orc.adaptive_plan(128, 256, 0.5)[3] == np.int32   # 32768


def _torch_quantize(t: torch.Tensor, bits: int):
    """torch's dtype-native arithmetic on the reference's expression (stacr/adaptive.py:58-76,97-108)."""
    qmax = 7.0 if bits == 4 else 127.0
    abs_max = t.abs().max()
    scale = abs_max / qmax
    if scale == 0:
        if abs_max == 0:
            return torch.zeros_like(t, dtype=torch.int8), torch.ones(1, dtype=t.dtype)
        return _torch_quantize(t.float() if t.element_size() < 4 else t.double(), bits)
    return torch.clamp(torch.round(t / scale), -qmax, qmax).to(torch.int8), scale.unsqueeze(0)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("case", ["normal", "wide", "zero", "tiny"])
def test_adaptive_quantize_matches_dtype_native_arithmetic(dtype, bits, case):
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    rng = np.random.default_rng(3)
    if case == "normal":
        v = rng.standard_normal(997).astype(np.float32)
    elif case == "wide":
        v = (rng.standard_normal(997) * np.exp(rng.standard_normal(997) * 3)).astype(np.float32)
    elif case == "zero":
        v = np.zeros(33, np.float32)
    else:
        v = np.full(5, {"f32": 1e-44, "bf16": 1e-40, "f16": 6e-8}[dtype], np.float32)
    t = torch.from_numpy(v).to(tdt)
    vr = t.float().numpy()
    q, scale, sdt = orc.adaptive_quantize(vr, dtype, bits)
    tq, tscale = _torch_quantize(t, bits)
    assert np.array_equal(q, tq.numpy())
    assert scale == float(tscale.double())
    expect_dt = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16", torch.float64: "f64"}
    assert sdt == expect_dt[tscale.dtype]


@pytest.mark.parametrize("bits", [4, 8])
def test_adaptive_quantize_reference_known_answers(bits):
    # tests/test_adaptive.py:186-195: round trip within scale / 2
    x = np.array([-2.0, -0.5, 0.0, 0.5, 2.0], np.float32)
    q, scale, sdt = orc.adaptive_quantize(x, "f32", bits)
    rec = orc.adaptive_dequantize(q, scale, sdt)
    assert np.all(np.abs(rec - x) <= scale / 2 + 1e-6)
    # tests/test_adaptive.py:231-239: zero and 6e-8 fp16 survive within 1 %
    for value in (0.0, 6e-8):
        v = torch.full((5,), value, dtype=torch.float16).float().numpy()
        q, scale, sdt = orc.adaptive_quantize(v, "f16", bits)
        rec = orc.adaptive_dequantize(q, scale, sdt)
        np.testing.assert_allclose(rec.astype(np.float64), v.astype(np.float64), rtol=0.01, atol=0)


def test_int4_nibbles_and_all_zero_bytes():
    assert orc.adaptive_pack_int4(np.array([-7, 7, 0], np.int8)).tolist() == [0x01 | (0x0F << 4), 0x88]
    q, _, _ = orc.adaptive_quantize(np.zeros(6, np.float32), "f32", 4)
    assert orc.adaptive_pack_int4(q).tolist() == [0x88] * 3


def test_codecs_match_library_routines_and_round_trip():
    rng = np.random.default_rng(4)
    b_flat, n = 300, 700
    idx = np.sort(rng.choice(b_flat * n, size=5000, replace=False)).astype(np.int64)
    ptr, cols = orc.csr_encode(idx, b_flat, n)
    t = torch.from_numpy(idx)
    counts = torch.bincount(torch.div(t, n, rounding_mode="floor"), minlength=b_flat)
    assert np.array_equal(ptr[1:], torch.cumsum(counts, 0).numpy()) and ptr[0] == 0
    assert cols.dtype == np.int16 and np.array_equal(cols, (idx % n).astype(np.int16))
    assert np.array_equal(orc.csr_decode(ptr, cols, n), idx)
    base, deltas = orc.delta_encode(idx, b_flat, n)
    assert deltas.dtype == np.int16 and base.dtype == np.int32
    assert np.array_equal(orc.delta_decode(base, deltas, idx.size), idx)
    # delta width follows the largest gap
    wide = np.array([0, 40000, 40001], np.int64)
    assert orc.delta_encode(wide, 10, 10**5)[1].dtype == np.int32


def test_codecs_reference_known_answer_above_int32():
    # tests/test_adaptive.py:211-218 (indices above the int32 range, B_flat=4, N=2^30)
    idx = np.sort(np.array([2**31 + 15, 2**32 - 1, 2**31 + 2], np.int64))
    ptr, cols = orc.csr_encode(idx, 4, 2**30)
    assert np.array_equal(orc.csr_decode(ptr, cols, 2**30), idx)
    base, deltas = orc.delta_encode(idx, 4, 2**30)
    assert base.dtype == np.int64
    assert np.array_equal(orc.delta_decode(base, deltas, idx.size), idx)


def test_energy_closed_forms():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((64, 12)).astype(np.float32)
    e, x2, c2, per_rank = orc.adaptive_energy(x, np.zeros((64, 3), np.float32), "f32")
    assert abs(e - 1.0) < 1e-6 and c2 == 0.0 and np.all(per_rank == 0)
    # C carrying all of X's energy: residual energy 0
    e, _, _, _ = orc.adaptive_energy(x, x, "f32")
    assert e == 0.0


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_select_above_matches_torch_comparison(dtype):
    """The threshold modes' selection against torch's own `abs() > threshold` + `nonzero` (the
    reference's ops) on dtype-native values: thresholds equal to present magnitudes (strict, so
    excluded), ones that round up or down to a present magnitude in the dtype, 0-dim tensors as
    the sampled quantiles are, zero, and NaN residuals."""
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    rng = np.random.default_rng(5)
    r = torch.from_numpy(rng.standard_normal(4096).astype(np.float32)).to(tdt)
    r[::97] = 0.0
    r[5] = float("nan")
    r[11] = 0.1  # 0.1 rounded to the dtype: a threshold of 0.1 excludes it (strict after rounding)
    resid = r.float().numpy()
    present = float(r[40].abs())
    thresholds = [0.1, present, np.nextafter(np.float32(present), np.float32(0)), 0.0, -0.0, -1.0, 1.0, 2.5, 1e-30,
                  torch.tensor(present, dtype=tdt), torch.tensor(0.75, dtype=torch.float32)]
    for t in thresholds:
        expected = (r.abs() > t).nonzero().reshape(-1).numpy()
        tv = float(t) if torch.is_tensor(t) else t
        if torch.is_tensor(t) and t.dtype != tdt:
            continue  # (the engine rounds 0-dim quantiles to the activation dtype before comparing)
        idx, vals = orc.adaptive_select_above(resid, tv, dtype)
        assert np.array_equal(idx, expected), (dtype, t)
        assert np.array_equal(vals, resid[expected])
    assert 11 not in orc.adaptive_select_above(resid, 0.1, dtype)[0]
