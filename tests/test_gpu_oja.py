"""GPU parity of the Oja step (stacr_oja_step) against the oracle's fp64 step.

Bars (fp32 arithmetic): |update - update64| <= 1e-5 (|X^T Y / N| + |Q Y^T Y / N|) in Frobenius norm
(the two terms cancel when Q already spans X, so the bound is taken on the terms, not the
difference); stepped basis rel-L2 <= 1e-5; refreshed layer basis projector rel-L2 <= 1e-5
against the fp64 QR of the fp64 step.  Results must repeat bit for bit.
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


OJA_CASES = [
    ("cfg3_c_fc_shape", 8192, 1024, 16, "bf16", "random"),
    ("cfg3_aligned_basis", 8192, 1024, 16, "bf16", "aligned"),
    ("small_f32", 300, 96, 8, "f32", "random"),
    ("odd_f16", 1000, 130, 5, "f16", "random"),
    ("rank32_few_rows", 3, 40, 32, "f32", "random"),
    ("rank1_many_rows", 70000, 64, 1, "bf16", "random"),
    ("empty_batch", 0, 64, 4, "bf16", "random"),
    # bf16 X (features a multiple of 8, rank <= 16): the matrix-core passes
    ("mf_cfg3_c_fc_rank8", 8192, 1024, 8, "bf16", "random"),
    ("mf_aligned_rank8", 8192, 1024, 8, "bf16", "aligned"),
    ("mf_d2048_rank1", 300, 2048, 1, "bf16", "random"),
    ("mf_fewer_rows_than_a_tile", 3, 1024, 8, "bf16", "random"),
    ("mf_partial_feature_group", 1000, 264, 5, "bf16", "random"),
    ("mf_two_feature_groups_rank12", 3000, 4096, 12, "bf16", "random"),
    # fp16 X, d in {512, 1024, 2048}, rank <= 8: the one-pass VALU kernel
    ("onepass_d512_f16_ragged_rows", 1001, 512, 5, "f16", "random"),
    ("onepass_d1024_f16", 2048, 1024, 8, "f16", "random"),
    # config 4's refresh shapes: 16 x 2048 tokens, rank 16, d_in 2048 and 8192
    ("cfg4_up_rank16", 32768, 2048, 16, "bf16", "random"),
    ("cfg4_down_rank16", 32768, 8192, 16, "bf16", "random"),
]


@pytest.mark.parametrize("name,rows,d,r,dtype,kind", OJA_CASES)
def test_oja_step_matches_fp64_oracle(name, rows, d, r, dtype, kind):
    from stacr_amd import kernels

    dev = _dev()
    print(f"[oja] {name} rows={rows} d={d} r={r} {dtype}", flush=True)
    x = make_activation(max(rows, 1), d)[:rows].to(DT[dtype])
    if kind == "aligned":  # top right singular vectors, as the layer's first refresh leaves them
        _, _, vh = torch.linalg.svd(x.float()[:2048], full_matrices=False)
        q = vh[:r].t().contiguous()
    else:
        q = make_basis(d, r)
    lr = 0.05
    upd, stepped = kernels.oja_step(x.to(dev), q.to(dev), lr)
    upd2, stepped2 = kernels.oja_step(x.to(dev), q.to(dev), lr)
    assert torch.equal(upd, upd2) and torch.equal(stepped, stepped2)
    xf, qf = x.float().numpy(), q.float().numpy()
    u64, m64 = orc.oja_step(xf, qf, lr)
    xd, qd = xf.astype(np.float64), qf.astype(np.float64)
    n = max(1, rows)
    y = xd @ qd
    scale = np.linalg.norm(xd.T @ y / n) + np.linalg.norm(qd @ (y.T @ y / n))
    err = np.linalg.norm(upd.double().cpu().numpy() - u64)
    assert err <= 1e-5 * max(scale, 1e-30), (err, scale)
    m = stepped.double().cpu().numpy()
    assert np.linalg.norm(m - m64) <= 1e-5 * np.linalg.norm(m64)


GIVEN_Y_CASES = [
    ("cfg3_c_fc_rank8", 8192, 1024, 8),
    ("cfg4_up_rank16", 32768, 2048, 16),
    ("cfg4_down_rank16", 32768, 8192, 16),
    ("ragged_rows_odd_features", 1000, 264, 5),
    ("one_row", 4, 72, 16),
]


@pytest.mark.parametrize("name,rows,d,r", GIVEN_Y_CASES)
def test_oja_step_given_y_matches_fp64_oracle_and_the_full_step(name, rows, d, r):
    """stacr_oja_step_given_y (X read once, Y supplied): on the Y the full step's own projection
    would use, the update and stepped basis meet the fp64 oracle's bound, and equal the full
    step's (which computes Y itself) within fp32 rounding of Y; repeat calls are bit-identical."""
    from stacr_amd import kernels

    dev = _dev()
    print(f"[oja given Y] {name} rows={rows} d={d} r={r}", flush=True)
    x = make_activation(rows, d).to(torch.bfloat16)
    q = make_basis(d, r)
    lr = 0.05
    xd, qd = x.to(dev), q.to(dev)
    y = (x.double() @ q.double()).float().to(dev)  # fp32 rounding of the exact projection
    upd, stepped = kernels.oja_step_given_y(xd, qd, y, lr)
    upd2, stepped2 = kernels.oja_step_given_y(xd, qd, y, lr)
    assert torch.equal(upd, upd2) and torch.equal(stepped, stepped2)
    xf, qf = x.float().numpy(), q.float().numpy()
    u64, m64 = orc.oja_step(xf, qf, lr)
    x64, q64 = xf.astype(np.float64), qf.astype(np.float64)
    y64 = x64 @ q64
    scale = np.linalg.norm(x64.T @ y64 / rows) + np.linalg.norm(q64 @ (y64.T @ y64 / rows))
    err = np.linalg.norm(upd.double().cpu().numpy() - u64)
    assert err <= 1e-5 * scale, (err, scale)
    assert np.linalg.norm(stepped.double().cpu().numpy() - m64) <= 1e-5 * np.linalg.norm(m64)
    full_u, _ = kernels.oja_step(xd, qd, lr)
    assert torch.linalg.norm(full_u.double() - upd.double()).item() <= 1e-5 * scale


def test_oja_step_given_y_refuses_shapes_it_does_not_take():
    from stacr_amd import kernels

    dev = _dev()
    x = make_activation(64, 100).to(dev, torch.bfloat16)  # 100 features: not a multiple of 8
    q = make_basis(100, 4).to(dev)
    with pytest.raises(NotImplementedError):
        kernels.oja_step_given_y(x, q, torch.zeros(64, 4, device=dev), 0.1)
    x16 = make_activation(64, 128).to(dev, torch.float16)  # fp16 X
    with pytest.raises(NotImplementedError):
        kernels.oja_step_given_y(x16, make_basis(128, 4).to(dev), torch.zeros(64, 4, device=dev), 0.1)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_layer_refresh_runs_the_hip_step(dtype):
    """STACRLinear's second refresh (stacr/layers.py:346-353) through stacr_oja_step."""
    from stacr_amd import STACRLinear

    dev = _dev()
    torch.manual_seed(3)
    lin = torch.nn.Linear(256, 64).to(dev).to(DT[dtype])
    layer = STACRLinear.from_linear(lin, rank=8, update_interval=1, oja_lr=0.1).train()
    x0 = make_activation(512, 256, seed=11).to(DT[dtype]).to(dev)
    x1 = make_activation(512, 256, seed=12).to(DT[dtype]).to(dev)
    layer.set_step(0)
    layer(x0).float().sum().backward()
    q0 = layer.basis.detach().float().cpu().numpy()
    layer.set_step(1)
    layer(x1).float().sum().backward()
    q1 = layer.basis.detach().float().cpu().numpy()
    _, m64 = orc.oja_step(x1.float().cpu().numpy(), q0, 0.1)
    ref = orc.orthonormalize(m64)
    p_ref, p = ref @ ref.T, q1.astype(np.float64) @ q1.astype(np.float64).T
    tol = 1e-5 if dtype == "f32" else 2e-2  # a bf16 basis is rounded after the QR
    assert np.linalg.norm(p - p_ref) <= tol * np.linalg.norm(p_ref)


def test_oja_basis_update_uses_the_hip_step():
    from stacr_amd.oja import OjaBasis

    dev = _dev()
    ob = OjaBasis(features=96, rank=6, device=dev)
    x = make_activation(400, 96, seed=21).to(dev)
    ob.update(x)  # first call: SVD initialisation
    q0 = ob.basis.double().cpu().numpy()
    ob.update(x, lr=0.2)
    _, m64 = orc.oja_step(x.cpu().numpy(), q0.astype(np.float32), 0.2)
    ref = orc.orthonormalize(m64)
    q1 = ob.basis.double().cpu().numpy()
    assert np.linalg.norm(q1 @ q1.T - ref @ ref.T) <= 1e-5 * np.linalg.norm(ref @ ref.T)
