"""The saved-tensor compressor on the GPU (stacr/compressor.py, stacr/residual.py).

Bars: the dense reconstruction (stacr_reconstruct) bit-exact against the oracle (the same fp32
chain, rounded once, plus the dense residual, signed zeros included); pack's residual indices and
values bit-exact against the oracle's global top-k on the kernel's own coefficients (the
reference's rule k = max(1, min(n, round(budget n))), ties to the lowest index); coefficients
within rel-L2 2e-2 (16-bit) / 1e-5 (fp32) of the fp64 projection; the input gradient through
the hooks bit-equal to the uncompressed one (the weight is never compressed).
"""
import numpy as np
import pytest
import torch

from gpu_cases import make_activation, make_basis
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}
TOL = {"f32": 1e-5, "bf16": 2e-2, "f16": 2e-2}


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def announce(*parts):
    print("CASE", *parts, flush=True)


def _np(t):
    return t.detach().float().cpu().numpy()


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.mark.parametrize("rows,feats,rank,dtype,nnz", [
    (300, 1024, 8, "bf16", 1500),
    (77, 130, 5, "f16", 40),       # feats not a multiple of 4, rows not of 32
    (64, 512, 16, "f32", 300),
    (33, 96, 32, "bf16", 0),       # a residual without entries
    (1, 7, 1, "f16", 3),
    (4096, 2048, 8, "bf16", 41943),
])
def test_reconstruct_matches_oracle(dev, rows, feats, rank, dtype, nnz):
    from stacr_amd import kernels

    announce("reconstruct", rows, feats, rank, dtype, nnz)
    rng = np.random.default_rng(rows + feats)
    c = torch.from_numpy(rng.standard_normal((rows, rank)).astype(np.float32)).to(dev, DT[dtype])
    q = torch.from_numpy(np.linalg.qr(rng.standard_normal((feats, rank)))[0].astype(np.float32)).to(dev, DT[dtype])
    idx = np.sort(rng.choice(rows * feats, nnz, replace=False)).astype(np.int64)
    vals = torch.from_numpy(rng.standard_normal(nnz).astype(np.float32)).to(dev, DT[dtype])
    for ix in (torch.from_numpy(idx).to(dev), torch.from_numpy(idx.astype(np.int32)).to(dev)):
        out = kernels.reconstruct(c, q, (ix, vals))
        torch.cuda.synchronize()
        assert out.shape == (rows, feats) and out.dtype == DT[dtype]
        want = orc.reconstruct(_np(c), _np(q), idx, _np(vals), dtype)
        assert np.array_equal(_bits(_np(out)), _bits(want))
    none = kernels.reconstruct(c, q, None)
    assert np.array_equal(_bits(_np(none)), _bits(orc.reconstruct(_np(c), _np(q), None, None, dtype)))


def test_reconstruct_signed_zeros(dev):
    """A tiny negative product rounds to -0 in fp16: kept without a residual, +0 with one (the
    reference adds a zero tensor), and -0 + -0 at an entry stays -0."""
    from stacr_amd import kernels

    announce("reconstruct signed zeros")
    c = torch.tensor([[-1e-4], [1.0]], dtype=torch.float16, device=dev)  # (-1e-4)(1e-4) = -1e-8 -> -0
    q = torch.tensor([[1e-4], [1.0]], dtype=torch.float16, device=dev)
    bare = _np(kernels.reconstruct(c, q, None))
    assert np.signbit(bare[0, 0]) and bare[0, 0] == 0
    empty = (torch.empty(0, dtype=torch.int64, device=dev), torch.empty(0, dtype=torch.float16, device=dev))
    assert not np.signbit(_np(kernels.reconstruct(c, q, empty))[0, 0])
    one = (torch.tensor([0], device=dev), torch.tensor([-0.0], dtype=torch.float16, device=dev))
    assert np.signbit(_np(kernels.reconstruct(c, q, one))[0, 0])


def test_saved_tensor_context_runs_backward(dev):
    """Reference tests/test_hooks.py:6-19 on the GPU, plus: the input gradient uses the (never
    compressed) weight, so it equals the uncompressed one bit for bit; the weight gradient uses the
    reconstructed input.  (A sum loss saves no activation of its own.)"""
    from stacr_amd import STACRCompressor, STACRConfig, stacr_saved_tensors

    announce("saved-tensor context")
    torch.manual_seed(0)
    model = torch.nn.Linear(64, 32).to(dev)
    x = torch.randn(8, 64, device=dev, requires_grad=True)
    compressor = STACRCompressor(STACRConfig(rank=4, residual_budget=0.01, min_features=1, min_numel=1))
    seen = []
    pack = compressor.pack
    compressor.pack = lambda t: seen.append(pack(t)) or seen[-1]
    with stacr_saved_tensors(compressor):
        loss = model(x).pow(2).mean()
    loss.backward()
    assert model.weight.grad is not None and x.grad is not None
    # the leaf input (requires grad: treated as a parameter) passed through; pow's saved output did not
    assert [tuple(p.shape) for p in seen if not torch.is_tensor(p)] == [(8, 32)]
    model.zero_grad(set_to_none=True)
    x.grad = None
    seen.clear()
    h = x * 1.0  # an activation (not a leaf): compressed
    with stacr_saved_tensors(compressor):
        loss = model(h).sum()
    loss.backward()
    packed = [p for p in seen if not torch.is_tensor(p)]
    assert len(packed) == 1 and packed[0].shape == (8, 64)  # the input; the weight passed through
    x2 = x.detach().clone().requires_grad_(True)
    model2 = torch.nn.Linear(64, 32).to(dev)
    model2.load_state_dict(model.state_dict())
    model2(x2 * 1.0).sum().backward()
    assert torch.equal(x.grad, x2.grad)
    recon = compressor.unpack(packed[0])
    assert torch.allclose(model.weight.grad, torch.ones(8, 32, device=dev).t().mm(recon), rtol=1e-5, atol=1e-6)
    assert torch.equal(model.bias.grad, model2.bias.grad)


@pytest.mark.parametrize("shape,dtype,budget,lognormal", [
    ((4, 256, 512), "bf16", 0.01, True),
    ((1000, 384), "f16", 0.005, False),
    ((64, 512), "f32", 0.02, True),
    ((16, 128), "bf16", 1e-5, False),   # round(budget n) = 0: the reference still keeps one entry
])
def test_pack_unpack_against_oracle(dev, shape, dtype, budget, lognormal):
    from stacr_amd.compressor import PackedActivation, STACRCompressor, STACRConfig

    announce("pack/unpack", shape, dtype, budget)
    d = shape[-1]
    rows = int(np.prod(shape[:-1]))
    x = make_activation(rows, d, lognormal=lognormal).reshape(shape).to(dev, DT[dtype])
    comp = STACRCompressor(STACRConfig(rank=8, residual_budget=budget, min_features=1, min_numel=1))
    packed = comp.pack(x)
    torch.cuda.synchronize()
    assert isinstance(packed, PackedActivation) and packed.shape == shape and packed.dtype == DT[dtype]
    basis = packed.basis
    assert basis.dtype == DT[dtype] and basis.shape == (d, 8)
    xf, qf, cf = _np(x).reshape(rows, d), _np(basis), _np(packed.coeff)
    exact = orc.project_f64(xf, qf)
    assert np.linalg.norm(cf - exact) / np.linalg.norm(exact) <= TOL[dtype]
    n = rows * d
    k = max(1, min(n, int(round(budget * n))))
    resid = orc.residual_act(xf, cf, qf, dtype).reshape(-1)
    order = np.lexsort((np.arange(n), -np.abs(resid.astype(np.float64))))
    want = np.sort(order[:k])
    idx = packed.residual.indices.cpu().numpy()
    assert packed.residual.indices.dtype == torch.int64 and packed.residual.shape == shape
    assert np.array_equal(idx, want)
    assert np.array_equal(_bits(_np(packed.residual.values)), _bits(resid[want]))
    out = comp.unpack(packed)
    assert out.shape == shape and out.dtype == DT[dtype]
    ref = orc.reconstruct(cf, qf, want, resid[want], dtype).reshape(shape)
    assert np.array_equal(_bits(_np(out)), _bits(ref))
    # the reconstruction recovers X at the kept entries to within the dtype's rounding
    err = np.abs(_np(out).reshape(-1)[want] - xf.reshape(-1)[want])
    assert err.max() <= 2e-2 * (np.abs(xf).max() + 1)


def test_turbo_and_zero_budget_modes(dev):
    """Turbo (residual mode "none" after turbo_after_step) saves no residual; a zero budget saves
    an empty one (stacr/compressor.py:100-106,118-119, stacr/residual.py:26-30)."""
    from stacr_amd.compressor import STACRCompressor, STACRConfig

    announce("turbo / zero budget")
    x = make_activation(256, 256).to(dev, torch.bfloat16)
    turbo = STACRCompressor(STACRConfig(rank=4, min_features=1, min_numel=1, turbo_after_step=2))
    turbo.set_step(2)
    p = turbo.pack(x)
    assert p.residual is None
    assert np.array_equal(_bits(_np(turbo.unpack(p))), _bits(orc.reconstruct(_np(p.coeff), _np(p.basis), None, None, "bf16")))
    zero = STACRCompressor(STACRConfig(rank=4, residual_budget=0.0, min_features=1, min_numel=1))
    p = zero.pack(x)
    assert p.residual is not None and p.residual.indices.numel() == 0 and p.residual.indices.dtype == torch.int64
    empty = np.zeros(0, np.int64)
    assert np.array_equal(_bits(_np(zero.unpack(p))), _bits(orc.reconstruct(_np(p.coeff), _np(p.basis), empty, empty, "bf16")))


def test_select_topk_residual_rule(dev):
    """stacr/residual.py:23-33: k = max(1, min(n, round(budget n))) over the whole tensor, values
    taken from the tensor; ties to the lowest flat index, ascending."""
    from stacr_amd.compressor import select_topk_residual

    announce("select_topk_residual")
    r = torch.tensor([[0.5, -3.0, 2.0], [3.0, -0.25, 1.0]], device=dev)
    s = select_topk_residual(r, 0.34)  # round(2.04) = 2: |3.0| twice, lowest index first
    assert s.indices.tolist() == [1, 3] and s.values.tolist() == [-3.0, 3.0] and s.shape == (2, 3)
    s = select_topk_residual(r, 0.01)  # round(0.06) = 0 -> 1
    assert s.indices.tolist() == [1]
    assert select_topk_residual(r, 0.0).indices.numel() == 0
    s = select_topk_residual(r, 1.0)
    assert s.indices.tolist() == list(range(6))
    big = make_activation(512, 640).to(dev, torch.float16)
    s = select_topk_residual(big, 0.003)
    flat = _np(big).reshape(-1)
    k = int(round(0.003 * flat.size))
    want = np.sort(np.lexsort((np.arange(flat.size), -np.abs(flat.astype(np.float64))))[:k])
    assert np.array_equal(s.indices.cpu().numpy(), want)
