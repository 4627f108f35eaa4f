"""GPU parity of the adaptive-engine kernels against the oracle (stacr/adaptive.py,
stacr/index_compression.py).  Through the C ABI via stacr_amd.adaptive.

Bars: quantized codes, scales (value and dtype), encoded index streams, selected indices and
values bit-exact; coefficients rel-L2 <= 1e-5 (fp32) / 2e-2 (16-bit) against the fp64 projection;
dW rel-L2 <= 1e-5 (fp32) / 2e-2 (16-bit) against the fp64 factor formula.
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis, make_grad
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
SDT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16", torch.float64: "f64"}


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU")
    return torch.device("cuda:0")


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30)


# ---------------------------------------------------------------- quantizers
@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("case,n", [("normal", 4097), ("normal", 7), ("zero", 33), ("tiny", 5), ("one", 1)])
def test_adaptive_quantizer_matches_oracle(dtype, bits, case, n):
    from stacr_amd import adaptive as ad

    dev = _dev()
    rng = np.random.default_rng(n)
    if case == "normal":
        v = (rng.standard_normal(n) * np.exp(rng.standard_normal(n))).astype(np.float32)
    elif case == "zero":
        v = np.zeros(n, np.float32)
    elif case == "tiny":
        v = np.full(n, {"f32": 1e-44, "bf16": 1e-40, "f16": 6e-8}[dtype], np.float32)
    else:
        v = np.array([-0.75], np.float32)
    t = torch.from_numpy(v).to(DT[dtype]).to(dev)
    vr = t.float().cpu().numpy()
    q_ref, scale_ref, sdt_ref = orc.adaptive_quantize(vr, dtype, bits)
    if bits == 8:
        q, scale = ad.quantize_int8(t)
        assert np.array_equal(q.cpu().numpy(), q_ref)
        back = ad.dequantize_int8(q, scale)
    else:
        packed, scale, length = ad.quantize_int4(t)
        assert length == n
        assert np.array_equal(packed.cpu().numpy(), orc.adaptive_pack_int4(q_ref))
        back = ad.dequantize_int4(packed, scale, length)
    assert SDT[scale.dtype] == sdt_ref and scale.shape == (1,)
    assert float(scale.double().item()) == scale_ref
    ref_back = orc.adaptive_dequantize(q_ref, scale_ref, sdt_ref)
    assert back.dtype == scale.dtype
    assert np.array_equal(back.double().cpu().numpy(), np.asarray(ref_back, np.float64))


# ---------------------------------------------------------------- index codecs
@pytest.mark.parametrize("b_flat,n,nnz", [(300, 700, 5000), (8192, 1024, 41943), (4, 50000, 7), (3, 3, 1)])
def test_index_codecs_match_oracle_and_round_trip(b_flat, n, nnz):
    from stacr_amd import adaptive as ad

    dev = _dev()
    rng = np.random.default_rng(nnz)
    idx = np.sort(rng.choice(b_flat * n, size=nnz, replace=False)).astype(np.int64)
    idx_t = torch.from_numpy(idx.astype(np.int32 if b_flat * n < 2**31 else np.int64)).to(dev)
    c = ad.compress_indices(idx_t, b_flat, n, "csr", preserve_order=False)
    ptr_ref, cols_ref = orc.csr_encode(idx, b_flat, n)
    assert c.row_ptrs.dtype == torch.int32 and np.array_equal(c.row_ptrs.cpu().numpy(), ptr_ref)
    assert str(c.col_indices.dtype).endswith(str(cols_ref.dtype)) and np.array_equal(c.col_indices.cpu().numpy(), cols_ref)
    assert np.array_equal(ad.decompress_indices(c).cpu().numpy(), idx)
    dlt = ad.compress_indices(idx_t, b_flat, n, "delta", preserve_order=False)
    base_ref, d_ref = orc.delta_encode(idx, b_flat, n)
    assert np.array_equal(dlt.delta_base.cpu().numpy(), base_ref)
    assert str(dlt.col_indices.dtype).endswith(str(d_ref.dtype)) and np.array_equal(dlt.col_indices.cpu().numpy(), d_ref)
    assert np.array_equal(ad.decompress_indices(dlt).cpu().numpy(), idx)


@pytest.mark.parametrize("mode", ["csr", "delta"])
def test_index_codecs_reference_known_answer_above_int32(mode):
    # tests/test_adaptive.py:211-218: unsorted int64 indices, order restored on decode
    from stacr_amd import adaptive as ad

    dev = _dev()
    indices = torch.tensor([2**31 + 15, 2**32 - 1, 2**31 + 2], dtype=torch.int64, device=dev)
    packed = ad.compress_indices(indices, B_flat=4, N=2**30, mode=mode)
    assert torch.equal(ad.decompress_indices(packed), indices)
    assert ad._choose_index_dtype(2**32) == torch.int64


# ---------------------------------------------------------------- adaptive save
ADAPTIVE_CASES = [
    ("cfg4_shape_bf16", 2048, 1024, 16, "bf16", 0.005),
    ("small_f32", 300, 96, 8, "f32", 0.02),
    ("f16_int16_idx", 100, 300, 4, "f16", 0.01),
    ("odd_rank", 777, 264, 5, "bf16", 0.004),
    ("budget_floor_zero", 10, 10, 4, "f32", 0.005),
]


@pytest.mark.parametrize("name,rows,d,r,dtype,budget", ADAPTIVE_CASES)
def test_adaptive_save_matches_oracle(name, rows, d, r, dtype, budget):
    from stacr_amd import adaptive as ad

    dev = _dev()
    x = make_activation(rows, d).to(DT[dtype])
    q = make_basis(d, r).to(DT[dtype])
    coeff, idx, values, energy = ad.save(x.to(dev), q.to(dev), budget, 512)
    xf, qf = x.float().numpy(), q.float().numpy()
    cf = coeff.float().cpu().numpy()
    proj = orc.project_f64(xf, qf)
    assert _rel(cf, proj) <= (1e-5 if dtype == "f32" else 2e-2)
    _, idx_ref, val_ref = orc.adaptive_save(xf, qf, dtype, budget, 512, coeff=cf)
    if idx_ref is None:
        assert idx is None
    else:
        assert idx.dtype == {np.int16: torch.int16, np.int32: torch.int32, np.int64: torch.int64}[idx_ref.dtype.type]
        assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref.astype(np.int64))
        assert np.array_equal(values.float().cpu().numpy(), val_ref)
    e_ref, x2, c2, per_rank = orc.adaptive_energy(xf, cf, dtype)
    e = energy.cpu().numpy()
    tol = 1e-5 if dtype == "f32" else 2 ** -7

    def close(a, b, rtol):  # equal non-finite values (a 16-bit sum can overflow) or within rtol
        if not (np.isfinite(a) and np.isfinite(b)):
            return (np.isnan(a) and np.isnan(b)) or a == b
        return abs(a - b) <= rtol * max(abs(b), 1e-3)

    assert close(e[1], x2, tol) and close(e[2], c2, tol)
    assert close(e[0], e_ref, 4 * tol)
    np.testing.assert_allclose(e[3:3 + r], per_rank, rtol=1e-5, atol=1e-7)


SAVE_Y_CASES = [
    # rows, feats, q_cols, rank: the save uses the first `rank` of q_cols basis columns
    ("d2048_active5_of16", 4096, 2048, 16, 5),   # below the allocated rank: the wide pass for Y
    ("d8192_rank16", 2048, 8192, 16, 16),
    ("d3000_active7_of12", 1000, 3000, 12, 7),
    ("d1024_rank16_cfg4_like", 2048, 1024, 16, 16),
]


@pytest.mark.parametrize("name,rows,d,qc,r", SAVE_Y_CASES)
def test_adaptive_save_y_matches_oracle(name, rows, d, qc, r):
    """stacr_adaptive_save_y: Y = X B over all q_cols columns (fp32, within 1e-5 rel-L2 of the fp64
    product), the coefficients bf16(Y[:, :rank]) bit for bit, the selection on them bit-exact against
    the oracle, the energies from the same projection pass within the dtype's rounding."""
    from stacr_amd import adaptive as ad

    dev = _dev()
    print(f"CASE save_y {name}", flush=True)
    x = make_activation(rows, d).to(torch.bfloat16)
    q = make_basis(d, qc).to(torch.bfloat16)
    coeff, idx, values, energy, y = ad.save_y(x.to(dev), q.to(dev), r, 0.005, 512)
    assert y is not None and y.shape == (rows, qc)
    xf, qf = x.float().numpy(), q.float().numpy()
    exact = xf.astype(np.float64) @ qf.astype(np.float64)
    yf = y.cpu().numpy().astype(np.float64)
    assert np.linalg.norm(yf - exact) <= 1e-5 * np.linalg.norm(exact)
    assert torch.equal(coeff.cpu(), y[:, :r].cpu().to(torch.bfloat16))
    cf = coeff.float().cpu().numpy()
    _, idx_ref, val_ref = orc.adaptive_save(xf, qf[:, :r], "bf16", 0.005, 512, coeff=cf)
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), idx_ref.astype(np.int64))
    assert np.array_equal(values.float().cpu().numpy(), val_ref)
    e_ref, x2, c2, per_rank = orc.adaptive_energy(xf, cf, "bf16")
    e = energy.cpu().numpy()
    tol = 2 ** -7
    assert abs(e[1] - x2) <= tol * abs(x2) and abs(e[2] - c2) <= tol * abs(c2)
    assert abs(e[0] - e_ref) <= 4 * tol * max(abs(e_ref), 1e-3)
    np.testing.assert_allclose(e[3:3 + r], per_rank, rtol=1e-5, atol=1e-7)


# ---------------------------------------------------------------- the adaptive Function
FUNC_CONFIGS = [
    dict(residual_mode="topk", residual_budget=0.005, quantize_coefficients=True, quantize_residuals=True,
         residual_quantize_bits=4, index_compression="none"),
    dict(residual_mode="topk", residual_budget=0.005, quantize_coefficients=True, quantize_residuals=True,
         residual_quantize_bits=8, index_compression="csr"),
    dict(residual_mode="topk", residual_budget=0.01, quantize_coefficients=False, quantize_residuals=False,
         index_compression="delta"),
    dict(residual_mode="none", quantize_coefficients=True),
]


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("cfg_i", range(len(FUNC_CONFIGS)))
def test_adaptive_function_matches_factor_formula(dtype, cfg_i):
    from stacr_amd import adaptive as ad

    dev = _dev()
    cfg = FUNC_CONFIGS[cfg_i]
    rows, d_in, d_out, r = 1024, 256, 384, 8
    x = make_activation(rows, d_in).to(DT[dtype]).to(dev).requires_grad_(True)
    basis = make_basis(d_in, r).to(dev)
    lin = torch.nn.Linear(d_in, d_out).to(dev).to(DT[dtype])
    state = {"_schedule_step": 0}
    full = ad.STACRConfig(rank=r, **cfg).to_dict()  # the reference's (…, config, step_counter, layer_state)
    y = ad.STACRFunction.apply(x, lin.weight, lin.bias, basis, full, torch.zeros(1, dtype=torch.long), state)
    with torch.no_grad():  # the forward is the native dense op (mm, then the bias add)
        ref = torch.nn.functional.linear(x, lin.weight, lin.bias)
        assert torch.allclose(y.float(), ref.float(), rtol=1e-2 if dtype == "bf16" else 1e-5, atol=1e-2 if dtype == "bf16" else 1e-5)
    assert "last_residual_energy" in state
    g = make_grad(rows, d_out).to(DT[dtype]).to(dev)
    saved = y.grad_fn.saved_tensors
    y.backward(g)
    # rebuild the factors from the saved tensors with the oracle, then the fp64 factor formula
    c = saved[0].cpu()
    i = 2
    if cfg.get("quantize_coefficients"):
        s = saved[i]
        i += 1
        c = orc.adaptive_dequantize(c.numpy(), float(s.double().item()), SDT[s.dtype])
    else:
        c = c.float().numpy()
    i += 1  # bias
    idx = vals = None
    if cfg.get("residual_mode") == "topk" and len(saved) > i:
        v = saved[i].cpu()
        i += 1
        comp = cfg.get("index_compression", "none")
        if comp == "csr":
            idx = orc.csr_decode(saved[i].cpu().numpy(), saved[i + 1].cpu().numpy(), d_in)
            i += 2
        elif comp == "delta":
            idx = orc.delta_decode(saved[i + 1].cpu().numpy(), saved[i].cpu().numpy(), v.numel())
            i += 2
        else:
            idx = saved[i].cpu().numpy().astype(np.int64)
            i += 1
        if cfg.get("quantize_residuals"):
            s = saved[i]
            bits = cfg.get("residual_quantize_bits", 8)
            if bits == 8:
                qv = v.numpy()
            else:  # nibbles hold q + 8, even entry low
                p = v.numpy()
                qv = np.stack([p & 0xF, p >> 4], axis=1).reshape(-1)[:idx.size].astype(np.int16) - 8
            vals = orc.adaptive_dequantize(qv, float(s.double().item()), SDT[s.dtype])
        else:
            vals = v.float().numpy()
        vals = np.asarray(orc.round_to(np.asarray(vals, np.float32), dtype))
    gf = g.float().cpu().numpy()
    qf = basis.to(DT[dtype]).float().cpu().numpy()
    dw_ref, db_ref = orc.weight_grad(gf, np.asarray(c, np.float32), qf,
                                     idx if idx is not None else np.zeros(0, np.int64),
                                     vals if vals is not None else np.zeros(0, np.float32), d_in)
    dw = lin.weight.grad.double().cpu().numpy()
    assert _rel(dw, dw_ref) <= (1e-5 if dtype == "f32" else 2e-2)
    assert torch.allclose(x.grad.float(), (g @ lin.weight).float(), rtol=1e-2, atol=1e-2)
