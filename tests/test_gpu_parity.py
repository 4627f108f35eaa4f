"""Parity of the HIP save / weight-gradient path against the CPU oracle (needs an MI355X).

Bars:
  * coefficients: rel-L2 against the fp64 projection of the same (dtype-rounded) operands,
    <= 1e-5 in fp32 and <= 2e-2 in bf16/fp16;
  * selected indices, int8 / packed int4 bytes, bits-0 values and the fp32 scale: bit-exact
    against the oracle run on the kernel's own coefficients (identical residual arithmetic);
  * dW / dbias: rel-L2 against the fp64 oracle, <= 1e-5 (fp32) and <= 2e-2 (bf16/fp16).
  * bf16 coefficients, dW and dbias are also held to what one rounding of an fp32-accumulated
    result allows: elementwise |got - exact| <= half an ulp of the larger magnitude plus a small
    accumulation term, and rel-L2 <= 4e-3 (a result rounded once to bf16 sits near 1.5e-3).
All calls go through the C ABI (stacr_amd.kernels / the drop-in layer).
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis, make_grad
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def announce(*parts):
    print("CASE", *parts, flush=True)


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 numbers at |v| (8 significant bits; the normal-range spacing below 2^-126)."""
    e = np.floor(np.log2(np.maximum(np.abs(np.asarray(v, np.float64)), 2.0**-126)))
    return np.exp2(e - 7)


def assert_rounded_once_bf16(got, exact, accum_abs=None, what="result"):
    """got (bf16 values) against the exact fp64 result: each element within half an ulp of the larger
    magnitude plus `accum_abs` (a bound on the fp32 accumulation error, elementwise or scalar;
    default 1e-4 of the result's rms), and rel-L2 <= 4e-3."""
    got = np.asarray(got, np.float64)
    exact = np.asarray(exact, np.float64)
    if accum_abs is None:
        accum_abs = 1e-4 * float(np.sqrt(np.mean(exact * exact)))
    bound = 0.5 * bf16_ulp(np.maximum(np.abs(got), np.abs(exact))) + accum_abs
    err = np.abs(got - exact)
    worst = int(np.argmax(err - bound))
    assert np.all(err <= bound), (f"{what}: element {np.unravel_index(worst, err.shape)} off by "
                                  f"{err.flat[worst]:.4g} > bound {np.broadcast_to(bound, err.shape).flat[worst]:.4g}")
    assert rel_l2(got, exact) <= 4e-3, f"{what}: rel-L2 {rel_l2(got, exact):.3g} above 4e-3"


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def run_and_check_save(dev, rows, d, rank, dtype, mode, budget, chunk, bits, lognormal=False, seed=1234):
    from stacr_amd import kernels

    announce("save", rows, d, rank, dtype, mode, budget, chunk, bits)
    x = make_activation(rows, d, lognormal=lognormal, seed=seed)
    q = make_basis(d, rank)
    xd, qd = x.to(dev, DT[dtype]), q.to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(xd, qd, mode=mode, budget=budget, chunk_rows=chunk, bits=bits)
    torch.cuda.synchronize()
    xf, qf, cf = _np(xd), _np(qd), _np(coeff)
    assert coeff.shape == (rows, rank) and coeff.dtype == DT[dtype]
    exact = orc.project_f64(xf, qf)
    assert rel_l2(cf, exact) <= TOL[dtype]
    if dtype == "bf16":
        # fp32 accumulation over d terms: |error| <= d * 2^-24 * sum |x||q| (elementwise)
        accum = d * 2.0**-24 * (np.abs(xf).astype(np.float64) @ np.abs(qf).astype(np.float64))
        assert_rounded_once_bf16(cf, exact, accum, "coefficients")
    omode = "chunk_topk" if mode == "topk" else mode
    if budget <= 0:
        assert idx is None and data is None and scale is None
        return
    _, oidx, odata, oscale = orc.save(xf, qf, dtype, omode, budget, chunk, bits, coeff=cf)
    if oidx.size == 0:
        assert idx is None
        return
    assert idx.dtype == torch.int32
    orc.check_indices(idx.cpu().numpy(), rows * d, ascending=True)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), oidx)
    if bits == 0:
        assert data.dtype == DT[dtype]
        assert np.array_equal(_np(data), odata)
        assert scale.item() == 1.0
    else:
        assert np.array_equal(data.cpu().numpy().view(np.int8 if bits == 8 else np.uint8), odata)
        assert np.float32(scale.item()) == oscale
    return idx, data, scale, coeff, xd, qd


SAVE_CASES = [
    # name: rows, d, rank, dtype, mode, budget, chunk_rows, bits, lognormal
    ("cfg1_fp32_chunk", 4096, 768, 8, "f32", "chunk_topk", 0.005, 512, 8, False),
    ("cfg3_cfc_bf16_global", 8192, 1024, 8, "bf16", "global_topk", 0.005, 512, 8, True),
    ("cfg3_cproj_bf16_global", 8192, 4096, 8, "bf16", "global_topk", 0.005, 512, 8, True),
    ("cfg2_turbo_bf16_no_residual", 8192, 1280, 8, "bf16", "chunk_topk", 0.0, 512, 8, False),
    ("cfg5_cproj_bf16_chunk", 8192, 4096, 8, "bf16", "chunk_topk", 0.005, 512, 8, True),
    ("cfg4_shape_bf16_chunk", 1024, 8192, 16, "bf16", "chunk_topk", 0.005, 512, 8, False),
    ("chunk_trim_bf16", 1536, 4096, 8, "bf16", "chunk_topk", 0.005, 512, 8, False),
    ("chunk_trim_small", 37, 24, 4, "f32", "chunk_topk", 0.05, 8, 8, False),
    ("f16_scalar_path_int4", 300, 20, 3, "f16", "chunk_topk", 0.1, 64, 4, False),
    ("bf16_bits0_global", 1000, 96, 5, "bf16", "global_topk", 0.02, 512, 0, False),
    ("ref_tiny_bits0", 5, 16, 4, "f32", "chunk_topk", 0.25, 2, 0, False),
    ("ref_tiny_bits4", 5, 16, 4, "f32", "chunk_topk", 0.25, 2, 4, False),
    ("ref_tiny_global", 5, 16, 4, "f32", "global_topk", 0.25, 2, 8, False),
    ("fp32_odd_width", 64, 30, 2, "f32", "topk", 0.1, 16, 8, False),
    ("fp32_wide_rows", 64, 8192, 16, "f32", "global_topk", 0.01, 512, 8, False),
    ("bf16_rank32", 512, 256, 32, "bf16", "chunk_topk", 0.01, 128, 8, False),
    ("fp32_rank1", 256, 64, 1, "f32", "global_topk", 0.05, 512, 8, False),
    ("partial_last_chunk", 1000, 128, 8, "bf16", "chunk_topk", 0.01, 300, 8, False),
    ("no_residual_budget", 64, 64, 4, "f32", "chunk_topk", 0.0, 16, 8, False),
    # batched path: 16-bit types skip the last radix pass; 128+ workgroups per chunk use
    # histogram copies, fewer do not
    ("f16_batched_global_copies", 2048, 1024, 8, "f16", "global_topk", 0.005, 512, 8, True),
    ("f16_batched_chunk", 1024, 512, 4, "f16", "chunk_topk", 0.01, 256, 8, False),
    ("bf16_batched_global_one_copy", 512, 1024, 8, "bf16", "global_topk", 0.01, 512, 8, False),
    ("f32_batched_global_copies", 4096, 512, 8, "f32", "global_topk", 0.01, 512, 8, True),
    # bf16 batched path ends the selection in the emission pass: chunks with a partial last
    # workgroup and a trim to k_total, and a chunked run without quantization
    ("bf16_batched_chunk_trim", 1000, 1024, 8, "bf16", "chunk_topk", 0.005, 100, 8, True),
    ("bf16_batched_chunk_bits0", 2048, 1024, 4, "bf16", "chunk_topk", 0.01, 512, 0, False),
    # a budget whose per-workgroup quota exceeds the candidate list: the stored-residual passes
    ("bf16_batched_large_budget", 1024, 1024, 8, "bf16", "global_topk", 0.05, 512, 8, True),
    # 16-bit rows of 2048 < d <= 4096: the projection pass takes two vectors a thread and stores
    # the residual; the later passes read it as twice the rows of half the width (cfg3 c_proj,
    # cfg5 c_proj and chunk_trim_bf16 above also run here)
    ("f16_wide_global_copies", 2048, 4096, 8, "f16", "global_topk", 0.005, 512, 8, True),
    ("bf16_wide_2560_partial_vectors", 1024, 2560, 8, "bf16", "global_topk", 0.01, 512, 8, True),
    ("bf16_wide_chunk_partial_int4", 1000, 3072, 5, "bf16", "chunk_topk", 0.01, 300, 4, False),
    ("f16_wide_rank4_bits0", 512, 4096, 4, "f16", "global_topk", 0.01, 512, 0, False),
    ("bf16_wide_rank1_odd_chunk", 777, 2064, 1, "bf16", "chunk_topk", 0.02, 37, 8, False),
    ("bf16_wide_no_residual", 256, 4096, 8, "bf16", "chunk_topk", 0.0, 128, 8, False),
    # rank 16 (cfg4) and rows up to 8192 features: the projection pass with 256 / 512 threads a
    # row, the later passes on the residual as rows of <= 2048 features (2, 3 or 4 per row)
    ("bf16_rank16_d2048_chunk", 2048, 2048, 16, "bf16", "chunk_topk", 0.005, 512, 8, True),
    ("f16_rank16_d3072_global", 1024, 3072, 16, "f16", "global_topk", 0.01, 512, 8, False),
    ("bf16_rank12_d6144_chunk_int4", 600, 6144, 12, "bf16", "chunk_topk", 0.005, 200, 4, False),
    ("bf16_rank3_d8192_global", 512, 8192, 3, "bf16", "global_topk", 0.005, 512, 8, True),
    ("bf16_rank16_d1024_bits0", 1000, 1024, 16, "bf16", "global_topk", 0.01, 512, 0, False),
    ("f16_rank16_d8192_per_row", 256, 8192, 16, "f16", "chunk_topk", 0.005, 128, 8, False),
    ("bf16_rank16_d8192_no_residual", 256, 8192, 16, "bf16", "chunk_topk", 0.0, 128, 8, False),
]


@pytest.mark.parametrize("case", SAVE_CASES, ids=[c[0] for c in SAVE_CASES])
def test_save_matches_oracle(dev, case):
    run_and_check_save(dev, *case[1:])


def _crafted_activation(kind, rows, d):
    """Inputs on which some bf16 batched workgroups cannot use their candidate lists: 'outlier_rows'
    scales rows 32..47 (one workgroup's rows at d = 1024) by 1000, so that workgroup alone holds
    more than its quota above the chunk's level-0 bin; 'tie_block' sets rows 0..15 to +-1 under a
    zero basis, so one bin holds 16384 equal keys (more than the list holds, and ties at the
    threshold); 'outlier_scattered' scales every 40th row by 300."""
    x = make_activation(rows, d, lognormal=True)
    if kind == "outlier_rows":
        x[32:48] *= 1000.0
    elif kind == "outlier_scattered":
        x[::40] *= 300.0
    elif kind == "tie_block":
        g = torch.Generator().manual_seed(7)
        x = 0.01 * torch.randn(rows, d, generator=g)
        x[:16] = torch.where(torch.rand(16, d, generator=g) < 0.5, -1.0, 1.0)
    return x


@pytest.mark.parametrize("kind,rows,d,mode,budget,chunk,bits", [
    ("outlier_rows", 2048, 1024, "global_topk", 0.005, 512, 8),
    ("outlier_rows", 2048, 1024, "chunk_topk", 0.005, 256, 8),
    ("tie_block", 512, 1024, "global_topk", 0.005, 512, 0),
    ("tie_block", 1024, 1024, "chunk_topk", 0.01, 128, 8),
    ("outlier_scattered", 4096, 1024, "global_topk", 0.005, 512, 8),
    # wide rows (the level-1 pass writes the lists from the stored residual; overflowing lists
    # fall back to the stored residual)
    ("tie_block", 512, 4096, "global_topk", 0.005, 512, 0),
    ("outlier_rows", 1024, 4096, "chunk_topk", 0.005, 256, 8),
    ("outlier_scattered", 2048, 4096, "global_topk", 0.005, 512, 8),
])
def test_save_candidate_fallback_matches_oracle(dev, kind, rows, d, mode, budget, chunk, bits):
    """bf16 saves keep per-workgroup candidate lists (kept by the projection pass, or by the level-1
    pass from a stored residual); a workgroup whose list cannot hold every element at or above its
    chunk's level-0 bin recomputes its residuals from X (reads them from the stored residual).
    Selection and quantization stay bit-exact against the oracle either way."""
    from stacr_amd import kernels

    rank = 8
    announce("save candidate fallback", kind, rows, d, mode, budget, chunk, bits)
    x = _crafted_activation(kind, rows, d)
    q = torch.zeros(d, rank) if kind == "tie_block" else make_basis(d, rank)
    xd, qd = x.to(dev, torch.bfloat16), q.to(dev, torch.bfloat16)
    coeff, idx, data, scale = kernels.save(xd, qd, mode=mode, budget=budget, chunk_rows=chunk, bits=bits)
    torch.cuda.synchronize()
    xf, qf, cf = _np(xd), _np(qd), _np(coeff)
    _, oidx, odata, oscale = orc.save(xf, qf, "bf16", mode, budget, chunk, bits, coeff=cf)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), oidx)
    if bits == 0:
        assert np.array_equal(_np(data), odata)
    else:
        assert np.array_equal(data.cpu().numpy().view(np.int8), odata)
        assert np.float32(scale.item()) == oscale
    if kind == "tie_block":  # the ties at the threshold (chunk 0) go to its lowest flat indices
        first = oidx[oidx < min(chunk, rows) * d] if mode == "chunk_topk" else oidx
        assert first.size > 0 and first.max() < 16 * d


@pytest.mark.parametrize("d,dtype,rank", [(4096, "bf16", 8), (2560, "f16", 8), (1024, "bf16", 8), (8192, "bf16", 16),
                                          (2048, "f16", 16)])
def test_save_from_given_coefficients_matches_full_save(dev, d, dtype, rank):
    """With the coefficients given (stacr_select_residual), the selection and quantization are the
    full save's, bit for bit, on the batched and wide-row paths."""
    from stacr_amd import kernels

    announce("save from coeff", d, dtype, rank)
    rows = 1024
    xd = make_activation(rows, d, lognormal=True).to(dev, DT[dtype])
    qd = make_basis(d, rank).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(xd, qd, mode="global_topk", budget=0.005, chunk_rows=512, bits=8)
    c2, i2, d2, s2 = kernels.save(xd, qd, mode="global_topk", budget=0.005, chunk_rows=512, bits=8, coeff=coeff)
    torch.cuda.synchronize()
    assert torch.equal(i2, idx) and torch.equal(d2, data) and torch.equal(s2, scale)


def test_save_is_deterministic(dev):
    from stacr_amd import kernels

    announce("determinism")
    x = make_activation(4096, 1024).to(dev, torch.bfloat16)
    q = make_basis(1024, 8).to(dev, torch.bfloat16)
    a = kernels.save(x, q, mode="global_topk", budget=0.005, chunk_rows=512, bits=8)
    b = kernels.save(x, q, mode="global_topk", budget=0.005, chunk_rows=512, bits=8)
    for u, v in zip(a, b):
        assert torch.equal(u, v)


# ------------------------------------------------------------------ reference known answers on the GPU
def test_global_topk_vs_chunk_known_answer(dev):
    """Reference tests/test_integration.py:106-114 through _select_residual."""
    from stacr_amd.layers import _select_residual

    announce("kat global vs chunk")
    x = torch.tensor([[100.0, 90.0, 80.0, 70.0], [4.0, 3.0, 2.0, 1.0]], device=dev)
    q, c = torch.zeros(4, 1, device=dev), torch.zeros(2, 1, device=dev)
    i, v = _select_residual(x, c, q, 0.5, 1, "global_topk", 2, 0.1)
    assert set(i.tolist()) == {0, 1, 2, 3}
    assert set(v.tolist()) == {100.0, 90.0, 80.0, 70.0}
    local, _ = _select_residual(x, c, q, 0.5, 1, "chunk_topk", 2, 0.1)
    assert set(local.tolist()) == {0, 1, 4, 5}


def test_ties_take_lowest_flat_index(dev):
    from stacr_amd.layers import _select_residual

    announce("ties")
    x = torch.ones(4, 8, device=dev)
    x[:, ::2] *= -1.0
    q, c = torch.zeros(8, 1, device=dev), torch.zeros(4, 1, device=dev)
    i, _ = _select_residual(x, c, q, 0.25, 512, "global_topk")
    assert i.tolist() == list(range(8))
    i, _ = _select_residual(x, c, q, 0.25, 2, "chunk_topk")
    assert i.tolist() == [0, 1, 2, 3, 16, 17, 18, 19]


def test_exact_span_gives_zero_residual_lowest_indices(dev):
    """X exactly in the span of a unit-vector basis: every residual is 0, all keys tie."""
    from stacr_amd import kernels

    announce("zero residual")
    d, rank, rows = 64, 4, 32
    q = torch.zeros(d, rank)
    q[[3, 9, 17, 31], [0, 1, 2, 3]] = 1.0
    c = torch.randint(-5, 5, (rows, rank)).float()
    x = (c @ q.t()).to(dev)
    coeff, idx, data, scale = kernels.save(x, q.to(dev), mode="global_topk", budget=0.05, chunk_rows=512, bits=8)
    k = orc.residual_plan(rows, d, "global_topk", 0.05, 512)[0]
    assert torch.equal(coeff.cpu(), c)
    assert idx.tolist() == list(range(k))
    assert not data.any() and scale.item() == np.float32(np.finfo(np.float32).tiny)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
def test_quantize_values_known_answers(dev, dtype):
    import stacr_amd

    announce("quantize", dtype)
    v = torch.tensor([0.0, 1e-6, -1e-6], dtype=DT[dtype], device=dev)
    p = stacr_amd.quantize_values(v, 8)
    assert p.scale.dtype == torch.float32 and p.scale.item() > 0
    assert torch.allclose(p.dequantize(torch.float32), v.float(), atol=1e-8)
    s = 2.0**-7
    v = torch.tensor([127, 0.5, 1.5, 2.5, -3.5, -127, 64.25], device=dev) * s
    p = stacr_amd.quantize_values(v, 8)
    assert p.scale.item() == s and p.data.tolist() == [127, 0, 2, 2, -4, -127, 64]
    p = stacr_amd.quantize_values(torch.tensor([7, -7, 0.5, 1.5, 2.5], device=dev) * 0.125, 4)
    assert p.scale.item() == 0.125 and p.data.tolist() == [0x97, 0x20, 0x02]
    rnd = torch.randn(1001, generator=torch.Generator().manual_seed(3)).to(dev, DT[dtype])
    for bits in (4, 8):
        p = stacr_amd.quantize_values(rnd, bits)
        oq, oscale = orc.quantize(_np(rnd), bits)
        got = p.data.cpu().numpy()
        want = oq if bits == 8 else orc.pack_int4(oq)
        assert np.array_equal(got.view(np.int8) if bits == 8 else got, want)
        assert np.float32(p.scale.item()) == oscale


# ------------------------------------------------------------------ weight gradient
GRAD_CASES = [
    # name: rows, d_in, d_out, rank, dtype, transposed, bits, mode, budget, lognormal
    ("cfg1_fp32", 4096, 768, 3072, 8, "f32", False, 8, "chunk_topk", 0.005, False),
    # the north-star layer pair at its own size (cfg3), and cfg2's Turbo layer
    ("cfg3_cfc_bf16_conv1d_full", 8192, 1024, 4096, 8, "bf16", True, 8, "global_topk", 0.005, True),
    ("cfg3_cproj_bf16_conv1d_full", 8192, 4096, 1024, 8, "bf16", True, 8, "global_topk", 0.005, True),
    ("cfg2_turbo_bf16_full", 8192, 1280, 5120, 8, "bf16", False, 8, "chunk_topk", 0.0, False),
    # no residual, the rows of each output slab split over two workgroups: 2900 rows are 6 blocks
    # (3 + 3, the last one partial) over 25 slabs (no XCD remap), 2100 rows 5 blocks (2 + 3)
    ("turbo_split_ragged_bf16_conv1d", 2900, 300, 400, 5, "bf16", True, 8, "chunk_topk", 0.0, False),
    ("turbo_split_ragged_f16", 2100, 130, 160, 7, "f16", False, 8, "chunk_topk", 0.0, False),
    ("cfg3_cfc_bf16_conv1d", 2048, 1024, 4096, 8, "bf16", True, 8, "global_topk", 0.005, False),
    ("fp32_bits0", 512, 256, 384, 4, "f32", False, 0, "chunk_topk", 0.02, False),
    ("fp32_bits4_conv1d_rank5", 1100, 300, 160, 5, "f32", True, 4, "chunk_topk", 0.02, True),
    ("f16_bits4_rank3", 300, 40, 70, 3, "f16", False, 4, "chunk_topk", 0.1, False),
    ("fp32_lowrank_only", 256, 128, 96, 8, "f32", True, 8, "chunk_topk", 0.0, False),
    ("bf16_rank16", 1024, 2048, 512, 16, "bf16", False, 8, "chunk_topk", 0.005, False),
    # the wide kernel (32-output slabs, every entry through matrix-core chunks): cfg4's two layer
    # shapes at 4096 rows with stored values and int8 codes, and fp16 with nibbles over parts of 750
    ("cfg4_up_wide_bf16_values", 4096, 2048, 8192, 16, "bf16", False, 0, "chunk_topk", 0.005, False),
    ("cfg4_down_wide_bf16_conv1d", 4096, 8192, 2048, 16, "bf16", True, 8, "chunk_topk", 0.005, False),
    ("wide_f16_bits4_parts750_rank5", 2048, 1500, 8192, 5, "f16", False, 4, "chunk_topk", 0.01, True),
]


@pytest.mark.parametrize("case", GRAD_CASES, ids=[c[0] for c in GRAD_CASES])
def test_weight_grad_matches_oracle(dev, case):
    from stacr_amd import kernels

    _, rows, d_in, d_out, rank, dtype, transposed, bits, mode, budget, lognormal = case
    announce("grad", *case)
    x = make_activation(rows, d_in, lognormal=lognormal).to(dev, DT[dtype])
    q = make_basis(d_in, rank).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(x, q, mode=mode, budget=budget, chunk_rows=512, bits=bits)
    residual = None if idx is None else (idx, data, scale)
    dw, db = kernels.weight_grad(g, coeff, q, residual, bits, transposed, DT[dtype], DT[dtype])
    torch.cuda.synchronize()
    if idx is None:
        oidx, ovals = np.zeros(0, np.int64), np.zeros(0, np.float32)
    else:
        oidx = idx.cpu().numpy().astype(np.int64)
        orc.check_indices(oidx, rows * d_in, ascending=True)
        if bits == 0:
            ovals = _np(data)
        else:
            raw = data.cpu().numpy()
            ovals = orc.dequantize(raw.view(np.int8) if bits == 8 else raw, np.float32(scale.item()), bits, oidx.size)
    odw, odb = orc.weight_grad(_np(g), _np(coeff), _np(q), oidx, ovals, d_in)
    got = _np(dw)
    assert got.shape == ((d_in, d_out) if transposed else (d_out, d_in))
    got = got.T if transposed else got
    assert rel_l2(got, odw) <= TOL[dtype]
    assert rel_l2(_np(db), odb) <= TOL[dtype]
    if dtype == "bf16":
        assert_rounded_once_bf16(got, odw, what="dW")
        assert_rounded_once_bf16(_np(db), odb, what="dbias")


@pytest.mark.parametrize("dtype,budget,rank", [("bf16", 0.03, 8), ("f32", 0.03, 8), ("f16", 0.004, 16),
                                               ("bf16", 0.2, 4)])
def test_weight_grad_heavy_features_and_many_rounds(dev, dtype, budget, rank):
    """A few input features carry most of the residual (every entry of their columns is kept), and
    a 512-row block holds more entries than one bucketing round: owners, helper pieces and the
    extra rounds all contribute."""
    from stacr_amd import kernels

    announce("grad heavy", dtype, budget, rank)
    rows, d_in, d_out = 2048, 1024, 272
    x = make_activation(rows, d_in)
    x[:, 7] *= 60.0
    x[:, 300] *= 25.0
    x[:, 1000:1004] *= 10.0
    x = x.to(dev, DT[dtype])
    q = make_basis(d_in, rank).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(x, q, mode="chunk_topk", budget=budget, chunk_rows=512, bits=8)
    dw, db = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, False, DT[dtype], DT[dtype])
    oidx = idx.cpu().numpy().astype(np.int64)
    ovals = orc.dequantize(data.cpu().numpy().view(np.int8), np.float32(scale.item()), 8, oidx.size)
    assert np.count_nonzero(oidx % d_in == 7) > 0.8 * rows  # the heavy column is (almost) fully kept
    odw, odb = orc.weight_grad(_np(g), _np(coeff), _np(q), oidx, ovals, d_in)
    assert rel_l2(_np(dw), odw) <= TOL[dtype]
    assert rel_l2(_np(db), odb) <= TOL[dtype]


@pytest.mark.parametrize("budget,bits", [(0.03, 8), (0.2, 0)])
def test_weight_grad_wide_kernel_heavy_features(dev, budget, bits):
    """The wide kernel (d_out 8192: 256 workgroups of 32 outputs) with a few features carrying
    most entries (tiles of many chunks) and, at budget 0.2, more records a block than it stages in
    LDS (the rest read from memory)."""
    from stacr_amd import kernels

    announce("grad wide heavy", budget, bits)
    rows, d_in, d_out, rank = 2048, 1024, 8192, 8
    x = make_activation(rows, d_in)
    x[:, 7] *= 60.0
    x[:, 300] *= 25.0
    x[:, 1000:1004] *= 10.0
    x = x.to(dev, torch.bfloat16)
    q = make_basis(d_in, rank).to(dev, torch.bfloat16)
    g = make_grad(rows, d_out).to(dev, torch.bfloat16)
    coeff, idx, data, scale = kernels.save(x, q, mode="chunk_topk", budget=budget, chunk_rows=512, bits=bits)
    assert idx.numel() // 4 > 3584 or budget < 0.1  # records a block past the staged ones
    dw, db = kernels.weight_grad(g, coeff, q, (idx, data, scale), bits, False, torch.bfloat16, torch.bfloat16)
    oidx = idx.cpu().numpy().astype(np.int64)
    ovals = (_np(data) if bits == 0 else
             orc.dequantize(data.cpu().numpy().view(np.int8), np.float32(scale.item()), 8, oidx.size))
    assert np.count_nonzero(oidx % d_in == 7) > 0.8 * rows
    odw, odb = orc.weight_grad(_np(g), _np(coeff), _np(q), oidx, ovals, d_in)
    assert rel_l2(_np(dw), odw) <= TOL["bf16"]
    assert_rounded_once_bf16(_np(dw), odw, what="dW")
    assert rel_l2(_np(db), odb) <= TOL["bf16"]


@pytest.mark.parametrize("where", ["head", "tail", "middle"])
def test_weight_grad_rows_of_unequal_density(dev, where):
    """Global selection over rows of very unequal magnitude: the 512-row blocks' entry ranges lie
    far from where a proportional share of the entries would put them (before, after and around
    it), and one block holds most of the entries (several bucketing rounds)."""
    from stacr_amd import kernels

    announce("grad unequal rows", where)
    rows, d_in, d_out, rank = 4096, 1024, 272, 8
    x = make_activation(rows, d_in)
    hot = {"head": slice(0, 256), "tail": slice(3840, 4096), "middle": slice(1900, 2200)}[where]
    x[hot] *= 30.0
    x = x.to(dev, torch.bfloat16)
    q = make_basis(d_in, rank).to(dev, torch.bfloat16)
    g = make_grad(rows, d_out).to(dev, torch.bfloat16)
    coeff, idx, data, scale = kernels.save(x, q, mode="global_topk", budget=0.01, chunk_rows=512, bits=8)
    oidx = idx.cpu().numpy().astype(np.int64)
    t = oidx // d_in
    assert np.count_nonzero((t >= hot.start) & (t < hot.stop)) > 0.9 * oidx.size  # skewed as intended
    dw, db = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, False, torch.bfloat16, torch.bfloat16)
    ovals = orc.dequantize(data.cpu().numpy().view(np.int8), np.float32(scale.item()), 8, oidx.size)
    odw, odb = orc.weight_grad(_np(g), _np(coeff), _np(q), oidx, ovals, d_in)
    assert rel_l2(_np(dw), odw) <= TOL["bf16"]
    assert rel_l2(_np(db), odb) <= TOL["bf16"]


def test_weight_grad_int64_indices(dev):
    """The backward accepts int64 flat indices (used when rows*d >= 2^31-1)."""
    from stacr_amd import kernels

    announce("int64 indices")
    rows, d_in, d_out, rank = 256, 64, 48, 4
    x = make_activation(rows, d_in).to(dev)
    q = make_basis(d_in, rank).to(dev)
    g = make_grad(rows, d_out).to(dev)
    coeff, idx, data, scale = kernels.save(x, q, mode="chunk_topk", budget=0.05, chunk_rows=64, bits=8)
    a, _ = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, False, torch.float32)
    b, _ = kernels.weight_grad(g, coeff, q, (idx.long(), data, scale), 8, False, torch.float32)
    # entries of a feature are summed in bucket order, which may differ between runs (last bits)
    assert rel_l2(_np(a), _np(b)) <= 1e-6


@pytest.mark.parametrize("rows,d_in,d_out,rank,bias,dtype,lognormal", [
    (4096, 2048, 512, 16, False, "bf16", False),   # two parts, rank 16 without bias, many records a feature
    (2000, 3000, 272, 15, True, "f16", False),     # three parts of 1000, rank 15 + bias, partial last block
    (3072, 1024, 1024, 8, True, "bf16", True),     # one part, skewed columns
    (2000, 3000, 272, 15, True, "f32", False),     # fp32: Q rows of a part in two LDS chunks, partial block
    (3072, 1024, 1024, 8, True, "f32", True),      # fp32: one part, skewed columns
    (4096, 2048, 512, 16, False, "f32", False),    # fp32: two parts, rank 16, records past the staged ones
])
def test_weight_grad_matrix_core_shapes(dev, rows, d_in, d_out, rank, bias, dtype, lognormal):
    """The matrix-core path (16-bit G, or fp32 G with residual codes; rank + bias <= 16) against the
    oracle at shapes where a part's Q rows span two LDS stages, features have more light records a
    block than the two the streaming kernel loads with the operands, and parts do not cover whole
    1024-feature spans."""
    from stacr_amd import kernels

    announce("grad tiles shape", rows, d_in, d_out, rank, bias, dtype)
    x = make_activation(rows, d_in, lognormal=lognormal).to(dev, DT[dtype])
    q = make_basis(d_in, rank).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(x, q, mode="chunk_topk", budget=0.01, chunk_rows=512, bits=8)
    dw, db = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, False, DT[dtype], DT[dtype] if bias else None)
    torch.cuda.synchronize()
    oidx = idx.cpu().numpy().astype(np.int64)
    ovals = orc.dequantize(data.cpu().numpy().view(np.int8), np.float32(scale.item()), 8, oidx.size)
    odw, odb = orc.weight_grad(_np(g), _np(coeff), _np(q), oidx, ovals, d_in)
    assert rel_l2(_np(dw), odw) <= TOL[dtype]
    if dtype == "bf16":
        assert_rounded_once_bf16(_np(dw), odw, what="dW")
    if bias:
        assert rel_l2(_np(db), odb) <= TOL[dtype]
    else:
        assert db is None


@pytest.mark.parametrize("dtype,transposed,d_out", [("bf16", True, 1024), ("f16", False, 1024), ("f32", False, 1024),
                                                   ("bf16", True, 8192), ("f16", False, 8192)])
def test_weight_grad_matrix_core_path_is_deterministic(dev, dtype, transposed, d_out):
    """The matrix-core path at rank 8 (16-bit G; fp32 G with int8 codes): every sum of the weight
    gradient has a fixed order (light entries by one owner thread in ascending row order, per-wave
    tiles reduced in wave order), so repeated calls agree bit for bit, with int32 and int64 indices
    alike."""
    from stacr_amd import kernels

    announce("grad determinism", dtype, transposed, d_out)
    rows, d_in, rank = 4096, 1024, 8  # (d_out 8192: the wide kernel)
    x = make_activation(rows, d_in, lognormal=True).to(dev, DT[dtype])
    q = make_basis(d_in, rank).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(x, q, mode="global_topk", budget=0.005, chunk_rows=512, bits=8)
    first = kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, transposed, DT[dtype], DT[dtype])
    for ix in (idx, idx.long(), idx):
        again = kernels.weight_grad(g, coeff, q, (ix, data, scale), 8, transposed, DT[dtype], DT[dtype])
        assert torch.equal(again[0], first[0])
        assert torch.equal(again[1], first[1])


# problems the matrix-core tiles do not take: (G dtype, rank, bias, bits, d_out)
GENERAL_SET_CASES = [
    ("f32", 8, True, 0, 1024),    # fp32 G with unquantized values
    ("bf16", 16, True, 8, 1024),  # rank 16 and the bias column: 17 coefficient columns
    ("bf16", 32, False, 8, 512),  # rank 32
    ("f16", 8, True, 4, 1000),    # d_out not a multiple of 16
]


@pytest.mark.parametrize("dtype,rank,bias,bits,d_out", GENERAL_SET_CASES)
def test_weight_grad_general_set_is_deterministic(dev, dtype, rank, bias, bits, d_out):
    """The general kernel set (the problems above): each feature's entries are placed in its bucket
    in ascending row order (a per-feature row bitmap, not arrival order), so repeated calls agree
    bit for bit; heavy features (log-normal scales, budget 0.03) make the buckets long and split
    them over several pieces."""
    from stacr_amd import _lib, kernels

    announce("general-set determinism", dtype, rank, bias, bits, d_out)
    rows, d_in = 4096, 1024
    x = make_activation(rows, d_in, lognormal=True).to(dev, DT[dtype])
    q = make_basis(d_in, rank).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale = kernels.save(x, q, mode="global_topk", budget=0.03, chunk_rows=512, bits=bits)
    bdt = DT[dtype] if bias else None
    with _lib.KernelTimer(max_launches=16) as timer:
        first = kernels.weight_grad(g, coeff, q, (idx, data, scale), bits, False, DT[dtype], bdt)
        torch.cuda.synchronize()
    names = set(timer.results)
    assert names & {"k_dw_fused", "k_dw_fused_mfma"} and not names & {"k_tile_grad", "k_tile_wide"}, names
    for _ in range(3):
        again = kernels.weight_grad(g, coeff, q, (idx, data, scale), bits, False, DT[dtype], bdt)
        assert torch.equal(again[0], first[0])
        if bias:
            assert torch.equal(again[1], first[1])


# ------------------------------------------------------------------ the drop-in layer on the GPU
def _lowrank(rows, feats, rank, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(rows, rank, generator=g) @ torch.randn(rank, feats, generator=g) / rank**0.5


def test_layer_input_gradient_and_forward_are_native(dev):
    from stacr_amd import STACRLinear

    announce("layer native grads")
    torch.manual_seed(0)
    w = torch.nn.Parameter((torch.randn(64, 256) * 0.05).to(dev))
    b = torch.nn.Parameter(torch.randn(64, device=dev))
    layer = STACRLinear(w, b, rank=8, residual_budget=0.005)
    x = _lowrank(128, 256, 12).to(dev).requires_grad_(True)
    y = layer(x)
    g = torch.randn_like(y)
    y.backward(g)
    x2 = x.detach().clone().requires_grad_(True)
    w2, b2 = w.detach().clone().requires_grad_(True), b.detach().clone().requires_grad_(True)
    y2 = torch.nn.functional.linear(x2, w2, b2)
    y2.backward(g)
    assert torch.equal(y, y2)
    assert torch.equal(x.grad, x2.grad)
    assert torch.equal(b.grad, b2.grad)


def test_layer_weight_gradient_matches_factor_identity(dev):
    """Reference tests/test_layers.py:49-69 (brute-force top-k, bits 0)."""
    from stacr_amd import STACRLinear

    announce("layer factor identity")
    torch.manual_seed(0)
    rows, feats, out_f = 128, 256, 64
    w = torch.nn.Parameter((torch.randn(out_f, feats) * 0.05).to(dev))
    layer = STACRLinear(w, None, rank=8, residual_budget=0.01, residual_bits=0)
    x = _lowrank(rows, feats, 12)
    y = layer(x.to(dev))
    g = torch.randn_like(y)
    y.backward(g)
    q = layer.basis.float().cpu()
    coeff = x @ q
    recon = coeff @ q.t()
    resid = x - recon
    k = max(1, int(round(0.01 * resid.numel())))
    _, top = torch.topk(resid.reshape(-1).abs(), k)
    sparse = torch.zeros_like(resid).reshape(-1)
    sparse[top] = resid.reshape(-1)[top]
    expected = g.cpu().t() @ (recon + sparse.reshape_as(resid))
    assert torch.allclose(w.grad.cpu(), expected, atol=1e-3)


@pytest.mark.parametrize("mode", ["chunk_topk", "global_topk", "uniform", "block_sparse", "sampled", "none"])
@pytest.mark.parametrize("bits", [0, 4, 8])
def test_all_selectors_contract_from_the_saved_factors(dev, mode, bits):
    """Reference tests/test_integration.py:120-143: dW equals G^T (C Q^T + R_s) rebuilt from the
    saved tensors."""
    from stacr_amd import STACRLinear
    from stacr_amd.quant import QuantizedValues

    announce("selectors contract", mode, bits)
    torch.manual_seed(4)
    layer = STACRLinear.from_linear(torch.nn.Linear(16, 7).to(dev), rank=4, residual_budget=0.25, residual_bits=bits,
                                    residual_mode=mode, chunk_rows=2, residual_block_size=4)
    out = layer(torch.randn(5, 16, device=dev))
    coeff, _, q, *sparse = out.grad_fn.saved_tensors
    recon = coeff @ q.T
    if sparse:
        indices, data, scale = sparse
        vals = QuantizedValues(data, scale, bits, indices.numel()).dequantize(recon.dtype)
        recon.reshape(-1)[indices.long()] += vals
    g = torch.randn_like(out)
    out.backward(g)
    assert torch.allclose(layer.weight.grad, g.T @ recon, atol=2e-5, rtol=1e-5)


def test_turbo_drops_the_residual_channel(dev):
    from stacr_amd import STACRLinear

    announce("turbo")
    w = torch.nn.Parameter((torch.randn(64, 256) * 0.05).to(dev))
    layer = STACRLinear(w, None, rank=8, residual_budget=0.01, turbo_after_step=2)
    x = _lowrank(64, 256, 8).to(dev)
    layer.set_step(0)
    out = layer(x)
    assert len(out.grad_fn.saved_tensors) == 6 and out.grad_fn.has_residual
    layer.set_step(5)
    out = layer(x)
    assert len(out.grad_fn.saved_tensors) == 3 and not out.grad_fn.has_residual
    out.square().sum().backward()
    assert torch.isfinite(w.grad).all() and w.grad.abs().sum() > 0


def test_backward_never_stores_the_dense_activation(dev):
    from stacr_amd import STACRLinear

    announce("no dense save")
    rows, feats = 256, 512
    w = torch.nn.Parameter((torch.randn(128, feats) * 0.05).to(dev))
    layer = STACRLinear(w, None, rank=8, residual_budget=0.005)
    out = layer(_lowrank(rows, feats, 16).to(dev))
    for t in out.grad_fn.saved_tensors:
        assert t.numel() < rows * feats


def test_outstanding_forwards_keep_their_basis_versions(dev):
    from stacr_amd import STACRLinear

    announce("basis versions")
    layer = STACRLinear.from_linear(torch.nn.Linear(16, 7).to(dev), rank=4, residual_budget=0)
    x = torch.randn(5, 16, device=dev, requires_grad=True)
    a = layer(x)
    saved = a.grad_fn.saved_tensors[2].clone()
    first = layer.basis
    layer.set_step(1)
    b = layer(x * 3)
    assert layer.basis is not first
    assert torch.equal(saved, first)
    (a.square().sum() + b.square().sum()).backward()
    assert torch.isfinite(layer.weight.grad).all() and torch.isfinite(x.grad).all()


@pytest.mark.parametrize("use_reentrant", [False, True])
def test_checkpoint_replay_matches_direct_gradient(dev, use_reentrant):
    import copy

    from torch.utils.checkpoint import checkpoint

    from stacr_amd import STACRLinear

    announce("checkpoint replay", use_reentrant)
    direct = STACRLinear.from_linear(torch.nn.Linear(16, 7).to(dev), rank=4, residual_budget=0.2)
    replay = copy.deepcopy(direct)
    x = torch.randn(5, 16, device=dev, requires_grad=True)
    y = x.detach().clone().requires_grad_(True)
    direct(x).square().sum().backward()
    checkpoint(replay, y, use_reentrant=use_reentrant).square().sum().backward()
    assert torch.allclose(replay.weight.grad, direct.weight.grad)
    assert torch.allclose(y.grad, x.grad)
    assert torch.equal(replay.basis, direct.basis)


def test_state_dict_resumes_basis_and_step(dev):
    from stacr_amd import STACRLinear

    announce("state dict resume")
    torch.manual_seed(1)
    lin = torch.nn.Linear(16, 7).to(dev)
    original = STACRLinear.from_linear(lin, rank=4, residual_budget=0)
    original.set_step(9)
    original(torch.randn(5, 16, device=dev)).sum().backward()
    restored = STACRLinear.from_linear(torch.nn.Linear(16, 7).to(dev), rank=4, residual_budget=0)
    restored.load_state_dict(original.state_dict())
    assert restored.step == 9 and bool(restored.basis_ready)
    assert torch.equal(restored.basis, original.basis)
    x = torch.randn(5, 16, device=dev)
    for layer in (original, restored):
        layer.zero_grad()
        layer.set_step(10)
        layer(x).sum().backward()
    assert torch.equal(restored.basis, original.basis)


@pytest.mark.parametrize("transposed", [False, True])
def test_autocast_forward_input_and_bias_gradient_match_native(dev, transposed):
    """Reference tests/test_integration.py:83-103 under bf16 autocast on the GPU."""
    from stacr_amd import STACRLinear

    announce("autocast", transposed)
    torch.manual_seed(14)
    w = torch.nn.Parameter(torch.randn((16, 7) if transposed else (7, 16), device=dev))
    b = torch.nn.Parameter(torch.randn(7, device=dev))
    layer = STACRLinear(w, b, rank=4, transposed=transposed)
    x = torch.randn(3, 2, 16, device=dev, requires_grad=True)
    xr = x.detach().clone().requires_grad_(True)
    wr, br = w.detach().clone().requires_grad_(True), b.detach().clone().requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        actual = layer(x)
        expected = (torch.addmm(br, xr.reshape(-1, 16), wr).reshape(3, 2, 7) if transposed
                    else torch.nn.functional.linear(xr, wr, br))
    assert torch.equal(actual, expected)
    g = torch.randn_like(actual)
    actual.backward(g)
    expected.backward(g)
    assert torch.equal(x.grad, xr.grad)
    assert torch.equal(b.grad, br.grad)
    assert w.grad.dtype == w.dtype and w.grad.shape == w.shape


def test_stored_bytes_equals_saved_inventory_under_autocast(dev):
    """Reference tests/test_memory.py:43-65 (all four fixed-count selectors)."""
    from stacr_amd import STACRLinear

    for mode in ("chunk_topk", "block_sparse", "global_topk", "uniform"):
        announce("inventory", mode)
        layer = STACRLinear.from_linear(torch.nn.Linear(16, 7).to(dev), rank=4, residual_mode=mode, chunk_rows=1,
                                        residual_block_size=4, residual_budget=0.17)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            output = layer(torch.randn(5, 16, device=dev))
        coeff, weight, basis, indices, values, scale = output.grad_fn.saved_tensors
        inventory = sum(t.numel() * t.element_size() for t in (coeff, basis, indices, values, scale))
        estimate = layer.stored_bytes(5, value_bytes=2)
        assert estimate["residual_count"] == indices.numel()
        assert estimate["total"] == inventory + layer.basis.numel() * layer.basis.element_size()


@pytest.mark.parametrize("full", [False, True], ids=["turbo_default", "full_explicit"])
def test_turbo_step_50_freezes_basis_and_drops_residual(dev, full):
    """Reference tests/test_surgery.py:79-141 on the GPU."""
    from stacr_amd import apply_stacr, set_step

    announce("turbo step 50", full)
    torch.manual_seed(19)
    model = torch.nn.Sequential(torch.nn.Linear(12, 7, bias=False)).to(dev)
    weight = model[0].weight
    options = {"turbo_after_step": None} if full else {}
    layers = apply_stacr(model, surface="all", min_features=1, rank=3, residual_budget=0.25, update_interval=1,
                         oja_lr=0.2, **options)
    layer = layers[0]
    set_step(layers, 48)
    model(torch.randn(32, 12, device=dev)).sum().backward()
    initialized = layer.basis.detach().clone()
    set_step(layers, 49)
    model.zero_grad(set_to_none=True)
    before = model(torch.randn(32, 12, device=dev))
    assert before.grad_fn.has_residual
    assert not torch.equal(layer.basis, initialized)
    before.sum().backward()
    step49 = layer.basis.detach().clone()
    set_step(layers, 50)
    model.zero_grad(set_to_none=True)
    x = torch.randn(32, 12, device=dev, requires_grad=True)
    upstream = torch.randn(32, 7, device=dev)
    out = model(x)
    assert out.grad_fn.has_residual is full
    if not full:
        torch.testing.assert_close(layer.basis, step49, rtol=0, atol=0)
    torch.testing.assert_close(out, x @ weight.t())
    out.backward(upstream)
    torch.testing.assert_close(x.grad, upstream @ weight)
    if not full:
        low = (x.detach() @ step49) @ step49.t()
        torch.testing.assert_close(weight.grad, upstream.t() @ low)


@pytest.mark.parametrize("rows,d_in,d_out,mode,budget,chunk,dtype,expect", [
    (8192, 1024, 4096, "global_topk", 0.005, 512, "bf16", True),    # the north-star layer
    (8192, 4096, 1024, "global_topk", 0.005, 512, "bf16", True),    # cfg 3 c_proj: rows split into two segments
    (2048, 1024, 512, "global_topk", 0.02, 512, "bf16", True),      # quota past the list: lists from the stored residual
    (2048, 1024, 512, "chunk_topk", 0.01, 256, "bf16", True),
    (64, 1024, 256, "chunk_topk", 0.0001, 1, "bf16", False),         # one entry a row, trimmed to 7: no census
    (1000, 1024, 256, "chunk_topk", 0.005, 100, "bf16", True),       # chunks of 100 rows, 4-row workgroups
    (2048, 1024, 512, "global_topk", 0.005, 512, "f16", False),      # fp16 keeps the stored residual
    (4096, 1024, 8192, "global_topk", 0.005, 512, "bf16", True),     # the wide weight-gradient kernel
])
def test_entry_census_matches_count_and_gives_the_same_weight_gradient(dev, rows, d_in, d_out, mode, budget, chunk,
                                                                       dtype, expect):
    """stacr_save_census: the per-feature entry counts (8 copies summed) and every 512-row block's
    first entry equal a count of the saved indices; stacr_weight_grad_census gives the same dW bit
    for bit as stacr_weight_grad; saves that cannot write a census say so."""
    from stacr_amd import kernels

    announce("entry census", rows, d_in, d_out, mode, budget, chunk, dtype)
    x = make_activation(rows, d_in, lognormal=True).to(dev, DT[dtype])
    q = make_basis(d_in, 8).to(dev, DT[dtype])
    g = make_grad(rows, d_out).to(dev, DT[dtype])
    coeff, idx, data, scale, census = kernels.save_with_census(x, q, mode=mode, budget=budget, chunk_rows=chunk,
                                                               bits=8)
    c2, i2, d2, s2 = kernels.save(x, q, mode=mode, budget=budget, chunk_rows=chunk, bits=8)
    torch.cuda.synchronize()
    assert torch.equal(idx, i2) and torch.equal(data, d2) and torch.equal(scale, s2) and torch.equal(coeff, c2)
    assert (census is not None) == expect
    if census is None:
        return
    flat = idx.cpu().numpy().astype(np.int64)
    cen = census.cpu().numpy().view(np.uint32).astype(np.int64)
    counts = cen[:8 * d_in].reshape(8, d_in).sum(axis=0)
    assert np.array_equal(counts, np.bincount(flat % d_in, minlength=d_in))
    nb = -(-rows // 512)
    bstart = cen[8 * d_in:8 * d_in + nb + 1]
    assert np.array_equal(bstart, np.searchsorted(flat // d_in, np.arange(nb + 1) * 512))
    res = (idx, data, scale)
    dw1, _ = kernels.weight_grad(g, coeff, q, res, 8, True, DT[dtype])
    dw2, _ = kernels.weight_grad(g, coeff, q, res, 8, True, DT[dtype], census=census)
    torch.cuda.synchronize()
    assert torch.equal(dw1, dw2)


def test_weight_grad_census_refuses_a_census_too_small_for_the_problem(dev):
    """stacr_weight_grad_census reads counts for every input feature and a start for every 512-row
    block: a census buffer sized for another (smaller) problem is refused on the host, before any
    launch, instead of being read past its end."""
    from stacr_amd import kernels

    rows, d_in, d_out = 2048, 1024, 512
    x = make_activation(rows, d_in, lognormal=True).to(dev, torch.bfloat16)
    q = make_basis(d_in, 8).to(dev, torch.bfloat16)
    g = make_grad(rows, d_out).to(dev, torch.bfloat16)
    coeff, idx, data, scale, census = kernels.save_with_census(x, q, mode="global_topk", budget=0.005, chunk_rows=512,
                                                               bits=8)
    assert census is not None
    small = census[: 8 * 512].clone()  # a census of a 512-feature layer
    with pytest.raises(ValueError, match="census has"):
        kernels.weight_grad(g, coeff, q, (idx, data, scale), 8, True, torch.bfloat16, census=small)
