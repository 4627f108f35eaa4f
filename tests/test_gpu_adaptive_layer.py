"""The adaptive engine's drop-in layer on the GPU: the reference's adaptive layer tests
(tests/test_adaptive.py) and BASELINE config 4's 50-step loop, checked against the oracle.

Bars: forward output and grad_input bit-equal to the native ops; dW against the fp64 oracle on
the saved factors (rel-L2 <= 1e-5 for fp32 weights; bf16 weights: within one rounding of the
exact result, rel-L2 <= 4e-3); the save's selected indices, values and int8 coefficient codes
bit-exact against the oracle on the kernel's own coefficients.
"""
import copy

import numpy as np
import pytest
import torch
from torch import nn

from gpu_cases import make_activation, make_basis, make_grad
from oracle import oracle as orc
from test_gpu_parity import _np, announce, assert_rounded_once_bf16, rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


def _cfg(**kw):
    from stacr_amd.adaptive import STACRConfig

    return STACRConfig(**kw)


def _layer(dev, d_in, d_out, cfg, seed=21, dtype=torch.float32):
    from stacr_amd.adaptive import STACRLinear

    torch.manual_seed(seed)
    layer = STACRLinear(d_in, d_out, cfg).to(dev)
    layer.linear.to(dtype)
    return layer


@pytest.mark.parametrize("mode", ["none", "topk", "block_sparse", "sparse_only", "threshold", "adaptive_threshold"])
def test_modes_preserve_forward_and_input_gradient(dev, mode):
    """Reference tests/test_adaptive.py:21-36."""
    announce("adaptive modes", mode)
    layer = _layer(dev, 16, 7, _cfg(rank=4, residual_mode=mode, residual_budget=0.2))
    x = torch.randn(8, 16, device=dev, requires_grad=True)
    reference = x.detach().clone().requires_grad_(True)
    expected = reference.mm(layer.linear.weight.t()) + layer.linear.bias
    actual = layer(x)
    assert torch.equal(actual, expected)
    grad = torch.randn_like(actual)
    actual.backward(grad)
    expected.backward(grad)
    assert torch.equal(x.grad, reference.grad)
    assert torch.isfinite(layer.linear.weight.grad).all()


THRESHOLD_CASES = [("threshold", "f32"), ("threshold", "bf16"), ("adaptive_threshold", "bf16"),
                   ("adaptive_threshold", "f32"), ("streaming_topk", "bf16"), ("streaming_topk", "f16")]


@pytest.mark.parametrize("mode,dtype", THRESHOLD_CASES)
def test_threshold_selections_match_oracle(dev, mode, dtype):
    """residual_mode "threshold" (every |r| above residual_threshold), "adaptive_threshold" and
    streaming top-k (a quantile of sampled |r|, then every |r| above it), stacr/adaptive.py:1416-1517,
    1574-1622, 1628-1786: the saved indices and values bit-exact against the oracle on the kernel's
    coefficients, with the sample positions redrawn by the same torch.randint calls under the same
    seed and the quantile taken by torch as the reference takes it; then dW from the saved factors
    against the fp64 oracle."""
    from stacr_amd import adaptive as ad

    announce("adaptive threshold selection", mode, dtype)
    rows, d_in, d_out, r, budget = 2000, 384, 256, 8, 0.01
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    x = make_activation(rows, d_in, lognormal=True).to(dev, tdt)
    basis = make_basis(d_in, r).to(dev)
    lin = nn.Linear(d_in, d_out).to(dev).to(tdt)
    kw = dict(rank=r, residual_budget=budget, quantize_coefficients=False, quantize_residuals=False, warmup_steps=0,
              use_fused_kernel=False)
    if mode == "streaming_topk":
        kw.update(residual_mode="topk", streaming_topk=True, streaming_topk_sample_ratio=0.05)
    else:
        kw.update(residual_mode=mode, residual_threshold=6.0)
    cfg = ad.STACRConfig(**kw).to_dict()
    torch.manual_seed(77)
    y = ad.STACRFunction.apply(x, lin.weight, lin.bias, basis, cfg, torch.zeros(1, dtype=torch.long),
                               {"_schedule_step": 0})
    saved = y.grad_fn.saved_tensors
    coeff, values, idx = saved[0], saved[3], saved[4]  # (coefficients, weight, bias, values, indices)
    used_basis = y.grad_fn.basis
    resid = orc.residual_act(_np(x), _np(coeff), _np(used_basis), dtype)
    total = rows * d_in
    if mode == "threshold":
        thr = 6.0
    else:
        # the reference's sampling: per 512-row chunk, torch.randint positions, then torch.quantile
        torch.manual_seed(77)
        if mode == "adaptive_threshold":
            sample, quant = min(100000, max(10000, total // 10)), 1.0 - budget
        else:
            sample, quant = min(100000, max(10000, int(total * 0.05))), 1.0 - int(total * budget) / total
        chunk = min(512, rows)
        per = max(1, (sample * chunk) // rows)
        pos = []
        for s in range(0, rows, chunk):
            n_el = (min(s + chunk, rows) - s) * d_in
            pos.append(torch.randint(0, n_el, (min(per, n_el),), device=dev).cpu().numpy() + s * d_in)
        samp = torch.from_numpy(np.abs(resid.reshape(-1)[np.concatenate(pos)])).to(dev).to(tdt)
        thr_t = torch.quantile(samp.float(), quant).to(tdt) if tdt != torch.float32 else torch.quantile(samp, quant)
        thr = float(thr_t)
    oidx, oval = orc.adaptive_select_above(resid, thr, dtype)
    assert idx.dtype == torch.int32 and values.dtype == tdt
    got = idx.cpu().numpy().astype(np.int64)
    orc.check_indices(got, total, ascending=True)
    assert 0 < oidx.size < total
    assert np.array_equal(got, oidx)
    assert np.array_equal(_np(values), oval)
    g = make_grad(rows, d_out).to(dev, tdt)
    y.backward(g)
    odw, _ = _oracle_dw(g, _np(coeff), used_basis, oidx, oval, d_in)
    assert rel_l2(_np(lin.weight.grad), odw) <= (1e-5 if dtype == "f32" else 4e-3)


@pytest.mark.parametrize("thr", [0.0, -0.0])
def test_threshold_mode_at_zero(dev, thr):
    """residual_threshold 0 and -0 (the config accepts no negative value) keep every nonzero
    residual, as torch's abs() > 0 does; rows of X in the basis's span (here zero rows) give exact
    zeros, which stay out."""
    from stacr_amd import adaptive as ad

    rows, d_in, d_out = 256, 64, 32
    x = make_activation(rows, d_in).to(dev)
    x[::3] = 0.0
    basis = make_basis(d_in, 4).to(dev)
    lin = nn.Linear(d_in, d_out).to(dev)
    cfg = ad.STACRConfig(rank=4, residual_mode="threshold", residual_threshold=thr, warmup_steps=0,
                         quantize_coefficients=False, quantize_residuals=False).to_dict()
    y = ad.STACRFunction.apply(x, lin.weight, lin.bias, basis, cfg, torch.zeros(1, dtype=torch.long),
                               {"_schedule_step": 0})
    saved = y.grad_fn.saved_tensors
    coeff, values, idx = saved[0], saved[3], saved[4]
    resid = orc.residual_act(_np(x), _np(coeff), _np(y.grad_fn.basis), "f32")
    oidx, oval = orc.adaptive_select_above(resid, thr, "f32")
    assert np.array_equal(idx.cpu().numpy().astype(np.int64), oidx)
    assert np.array_equal(_np(values), oval)
    assert 0 < oidx.size < rows * d_in


def test_threshold_mode_keeps_an_empty_residual_and_adaptive_threshold_k0_has_none(dev):
    """A threshold above every residual keeps an empty residual (the reference's empty tensors,
    int16 indices for a small layer, quantized as its empty-input rule says); adaptive_threshold
    with k = int(n * budget) = 0 keeps none and reports zero residual energy."""
    from stacr_amd import adaptive as ad

    x = torch.randn(8, 16, device=dev)
    lin = nn.Linear(16, 7).to(dev)
    basis = make_basis(16, 4).to(dev)
    cfg = ad.STACRConfig(rank=4, residual_mode="threshold", residual_threshold=1e6, warmup_steps=0,
                         quantize_coefficients=False, quantize_residuals=True).to_dict()
    y = ad.STACRFunction.apply(x, lin.weight, lin.bias, basis, cfg, torch.zeros(1, dtype=torch.long),
                               {"_schedule_step": 0})
    saved = y.grad_fn.saved_tensors
    assert saved[4].numel() == 0 and saved[4].dtype == torch.int16 and saved[3].numel() == 0
    y.sum().backward()
    assert torch.isfinite(lin.weight.grad).all()
    state = {"_schedule_step": 0}
    cfg = ad.STACRConfig(rank=4, residual_mode="adaptive_threshold", residual_budget=0.001, warmup_steps=0,
                         quantize_coefficients=False).to_dict()
    y = ad.STACRFunction.apply(x, lin.weight, lin.bias, basis, cfg, torch.zeros(1, dtype=torch.long), state)
    assert len(y.grad_fn.saved_tensors) == 3 and state["last_residual_energy"] == 0.0


def test_state_restores_runtime_controller_and_basis(dev):
    """Reference tests/test_adaptive.py:39-67."""
    from stacr_amd.adaptive import STACRLinear, set_stacr_runtime_state

    announce("adaptive state restore")
    cfg = _cfg(rank=4, residual_mode="topk", rank_mode="sensitivity", rank_min=1, rank_max=4, rank_adjust_interval=1,
               freeze_basis_after_warmup=False, update_interval=1, lazy_update_enabled=False,
               oja_update_per_optimizer_step=True)
    first = _layer(dev, 16, 7, cfg)
    set_stacr_runtime_state(first, 3)
    first(torch.randn(8, 16, device=dev)).sum().backward()
    state = copy.deepcopy(first.state_dict())
    second = STACRLinear(16, 7, copy.deepcopy(cfg)).to(dev)
    second.load_state_dict(state)
    assert second.layer_state == first.layer_state
    assert torch.equal(second.basis, first.basis)
    for layer in (first, second):
        layer.zero_grad()
        set_stacr_runtime_state(layer, 4)
    x = torch.randn(8, 16, device=dev)
    first(x).sum().backward()
    second(x).sum().backward()
    assert torch.equal(second.basis, first.basis)
    assert torch.equal(second.linear.weight.grad, first.linear.weight.grad)


def test_variance_rank_checkpoint_restores_changed_shape(dev):
    """Reference tests/test_adaptive.py:70-81."""
    from stacr_amd.adaptive import STACRLinear

    cfg = _cfg(rank=8, rank_mode="variance", rank_min=1, rank_max=8, rank_variance_threshold=0.9)
    first = _layer(dev, 16, 7, cfg)
    x = torch.randn(12, 1, device=dev) @ torch.randn(1, 16, device=dev)
    first(x).sum().backward()
    assert first.basis.shape[1] == 1
    second = STACRLinear(16, 7, copy.deepcopy(cfg)).to(dev)
    second.load_state_dict(first.state_dict())
    assert torch.equal(first.basis, second.basis) and second.basis_initialized


def test_repeated_forward_preserves_saved_basis(dev):
    """Reference tests/test_adaptive.py:84-103: an Oja update between forward and backward does not
    change the basis the first backward uses."""
    layer = _layer(dev, 16, 7, _cfg(rank=4, residual_mode="topk", freeze_basis_after_warmup=False,
                                    update_trigger="fixed", update_interval=2, lazy_update_enabled=False))
    x = torch.randn(8, 16, device=dev)
    out = layer(x)
    saved = out.grad_fn.basis.clone()
    layer(x * 2).sum().backward()
    assert torch.equal(out.grad_fn.basis, saved)
    out.sum().backward()


@pytest.mark.parametrize("frozen", [False, True])
def test_checkpoint_guard_preserves_gradient(dev, frozen):
    """Reference tests/test_adaptive.py:106-124."""
    from stacr_amd.adaptive_checkpointing import checkpoint

    cfg = _cfg(rank=4, residual_mode="topk", residual_budget=0.2, freeze_basis_after_warmup=frozen,
               update_interval=1, lazy_update_enabled=False)
    first = _layer(dev, 16, 7, cfg)
    second = copy.deepcopy(first)
    x = torch.randn(8, 16, device=dev, requires_grad=True)
    y = x.detach().clone().requires_grad_(True)
    first(x).square().sum().backward()
    checkpoint(second, y).square().sum().backward()
    assert torch.allclose(first.linear.weight.grad, second.linear.weight.grad)
    assert torch.equal(x.grad, y.grad)
    assert int(first.step_counter) == int(second.step_counter) == 1


def test_surgery_training_step_and_conv1d_identity(dev):
    """Reference tests/test_adaptive.py:140-170 with the training step."""
    from stacr_amd.adaptive import apply_adaptive_stacr

    class Conv1D(nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = nn.Parameter(torch.randn(16, 7))
            self.bias = nn.Parameter(torch.randn(7))

        def forward(self, x):
            return torch.addmm(self.bias, x, self.weight)

    model = nn.Sequential(Conv1D(), nn.Linear(7, 16)).to(dev)
    weight = model[0].weight
    x = torch.randn(8, 16, device=dev)
    expected = model(x)
    rng = torch.get_rng_state()
    apply_adaptive_stacr(model, rank=4, surface="all", min_features=1)
    assert torch.equal(rng, torch.get_rng_state())
    assert weight is model[0].linear.source_weight
    out = model(x)
    assert torch.allclose(out, expected, atol=1e-5)
    out.sum().backward()
    assert weight.grad is not None and torch.isfinite(weight.grad).all()


def _oracle_dw(g, coeff, basis, idx, vals, d_in):
    return orc.weight_grad(_np(g), coeff, _np(basis), idx, vals, d_in)


def _saved_factors(out, cfg, rows, d_in):
    """(coefficients as the backward dequantizes them, flat indices, values) read back from an
    adaptive STACRFunction's saved tensors, in the reference's order."""
    from stacr_amd.adaptive import dequantize_int4, dequantize_int8, decompress_indices, CompressedIndices, \
        IndexCompressionMode

    saved = list(out.grad_fn.saved_tensors)
    saved = [t.to(saved[1].device) for t in saved]  # offloaded factors come back to the weight's device
    pos = 2
    if cfg.quantize_coefficients:
        coeff = dequantize_int8(saved[0], saved[2])
        pos = 3
    else:
        coeff = saved[0]
    pos += 1  # bias
    values = saved[pos]
    pos += 1
    fn = out.grad_fn
    if cfg.index_compression == "none":
        idx = saved[pos]
        pos += 1
    else:
        a, b = saved[pos], saved[pos + 1]
        pos += 2
        csr = cfg.index_compression == "csr"
        comp = CompressedIndices(IndexCompressionMode.CSR if csr else IndexCompressionMode.DELTA,
                                 row_ptrs=a if csr else None, col_indices=b if csr else a,
                                 delta_base=None if csr else b, nnz=fn.index_compression_nnz, B_flat=rows, N=d_in,
                                 original_dtype=fn.index_compression_original_dtype)
        idx = decompress_indices(comp, restore_order=False)
    if cfg.quantize_residuals:
        scale = saved[pos]
        values = dequantize_int8(values, scale) if cfg.residual_quantize_bits == 8 else \
            dequantize_int4(values, scale, fn.residual_orig_len)
    return coeff, idx, values


def test_training_forward_reads_the_gpu_once(dev, monkeypatch):
    """After the first forward (which fits the basis), a training forward with int8 coefficients and
    int8 residual values reads the GPU once: the energies and both scales' dtype codes in one
    transfer (the step counter and the initialization flag have host mirrors)."""
    announce("adaptive host reads")
    cfg = _cfg(rank=8, residual_mode="topk", residual_budget=0.01, quantize_coefficients=True,
               quantize_residuals=True, residual_quantize_bits=8, freeze_basis_after_warmup=True)
    layer = _layer(dev, 512, 384, cfg)
    x = make_activation(1024, 512).to(dev)
    layer(x).sum().backward()
    reads = []
    for name in ("item", "tolist", "__bool__", "__int__", "__float__", "__index__"):
        orig = getattr(torch.Tensor, name)

        def counted(t, *a, _orig=orig, _name=name, **k):
            if t.is_cuda:
                reads.append(_name)
            return _orig(t, *a, **k)

        monkeypatch.setattr(torch.Tensor, name, counted)
    out = layer(x)
    monkeypatch.undo()
    assert reads == ["tolist"]
    saved = out.grad_fn.saved_tensors
    assert saved[2].dtype == torch.float32 and saved[-1].dtype == torch.float32  # both scales, x's dtype
    assert int(layer.step_counter) == 2 and layer.basis_initialized
    layer.step_counter.fill_(7)  # a write from outside: the mirror notices the version change
    assert layer._get_schedule_step() == 7 or layer._use_optimizer_step_schedule()


@pytest.mark.parametrize("compression,bits,offload", [("none", 8, False), ("csr", 4, False), ("delta", 8, True),
                                                      ("csr", 8, True)])
def test_saved_layout_and_weight_gradient_against_oracle(dev, compression, bits, offload):
    """int8 coefficients, CSR / delta index streams, int4 / int8 residual values and CPU offload:
    the saved tensors follow the reference's order and dtypes, and dW from them matches the fp64
    oracle on the same factors."""
    announce("adaptive layout", compression, bits, offload)
    rows, d_in, d_out = 1024, 512, 384
    cfg = _cfg(rank=8, residual_mode="topk", residual_budget=0.01, quantize_coefficients=True,
               quantize_residuals=True, residual_quantize_bits=bits, index_compression=compression,
               cpu_offload=offload, freeze_basis_after_warmup=True)
    layer = _layer(dev, d_in, d_out, cfg)
    x = make_activation(rows, d_in).to(dev)
    out = layer(x)
    saved = out.grad_fn.saved_tensors
    assert saved[0].dtype == torch.int8 and saved[0].shape == (rows, 8)
    assert saved[2].dtype == torch.float32 and saved[2].shape == (1,)  # coefficient scale in x's dtype
    k = int(rows * d_in * 0.01)
    expected_streams = {"none": 1, "csr": 2, "delta": 2}[compression]
    assert len(saved) == 4 + 1 + expected_streams + 1
    if offload:
        assert saved[0].device.type == "cpu" and saved[4].device.type == "cpu"
    coeff, idx, values = _saved_factors(out, cfg, rows, d_in)
    assert idx.numel() == k
    g = make_grad(rows, d_out).to(dev)
    out.backward(g)
    oidx = idx.cpu().numpy().astype(np.int64)
    orc.check_indices(oidx, rows * d_in, ascending=True)
    odw, odb = _oracle_dw(g, _np(coeff), out.grad_fn.basis, oidx, _np(values), d_in)
    assert rel_l2(_np(layer.linear.weight.grad), odw) <= 1e-5
    assert torch.allclose(layer.linear.bias.grad.double().cpu(), torch.from_numpy(odb), rtol=1e-5, atol=1e-4)


def test_low_rank_only_route_and_baseline_warmup(dev):
    from stacr_amd.adaptive import STACRLowRankOnlyFunction

    announce("adaptive routes")
    layer = _layer(dev, 256, 96, _cfg(rank=8, residual_mode="none", warmup_steps=1))
    x = make_activation(300, 256).to(dev)
    out = layer(x)  # step 0 < warmup: the full input is saved
    assert out.grad_fn.saved_tensors[0].shape == (300, 256)
    g = make_grad(300, 96).to(dev)
    out.backward(g)
    assert torch.allclose(layer.linear.weight.grad, g.t() @ x, rtol=1e-4, atol=1e-3)
    layer.zero_grad()
    out = layer(x)  # step 1: residuals off -> the low-rank-only route
    assert type(out.grad_fn).__name__.startswith(STACRLowRankOnlyFunction.__name__)
    assert layer.layer_state["b1_route_step_count"] == 1
    q = out.grad_fn.basis
    coeff = out.grad_fn.saved_tensors[0]
    out.backward(g)
    odw, _ = _oracle_dw(g, _np(coeff), q, np.zeros(0, np.int64), np.zeros(0, np.float32), 256)
    assert rel_l2(_np(layer.linear.weight.grad), odw) <= 1e-5


# ------------------------------------------------------------------ BASELINE config 4
def _drifting_activation(rows, d, step, seed, dev, latent=8, drift=0.02):
    """X = Z B_t^T + 0.05 E, 0.1% of entries x20, with B_t = B cos(drift t) + P sin(drift t) turning B
    towards a fixed random P (a slow rotation of the latent directions); seeded, generated on the GPU."""
    g = torch.Generator(device=dev).manual_seed(seed)
    b = torch.randn(d, latent, generator=g, device=dev)
    p = torch.randn(d, latent, generator=g, device=dev)
    gs = torch.Generator(device=dev).manual_seed(seed * 1000 + step)
    z = torch.randn(rows, latent, generator=gs, device=dev)
    bt = b * np.cos(drift * step) + p * np.sin(drift * step)
    x = z @ bt.t() + 0.05 * torch.randn(rows, d, generator=gs, device=dev)
    mask = torch.rand(rows, d, generator=gs, device=dev) < 0.001
    return torch.where(mask, x * 20.0, x)


@pytest.mark.timeout(900)
def test_config4_fifty_steps_refresh_rank_and_parity(dev):
    """Pythia-1.4B-shaped MLP pair (2048 -> 8192, 8192 -> 2048), bf16, N = 16 x 2048
    tokens, int8 coefficients, rank from the sensitivity controller capped at 16, chunk top-k budget
    0.005, fixed-cadence (10 steps) hybrid refresh of a frozen basis, 50 seeded steps with drifting
    activations.  Checks: refresh fires exactly on the layer's scheduled steps (plus any energy
    triggers, which are recorded as such), the active rank stays in [rank_min, 16], the save is
    bit-exact against the oracle at step 0 and on the first step after each layer's first scheduled
    refresh, the basis that refresh installs (a rank-16 Oja step on the layer's own 32768-row X,
    d_in 2048 and 8192, then QR) matches the fp64 Oja step of the oracle on the same X, prior basis
    and rate, and dW matches the oracle on sampled output features at steps 0, 10, 25 and 49."""
    from stacr_amd import adaptive
    from stacr_amd.rank_controller import is_fixed_refresh_step

    def check_save(out, x, li, step):
        announce("cfg4 save parity", li, step)
        basis = out.grad_fn.basis
        coeff, idx, values, _ = adaptive.save(x, basis, 0.005)
        xf, qf, cf = _np(x), _np(basis), _np(coeff)
        _, oidx, oval = orc.adaptive_save(xf, qf, "bf16", 0.005, 512, coeff=cf)
        assert np.array_equal(idx.cpu().numpy().astype(np.int64), oidx.astype(np.int64))
        assert np.array_equal(_np(values), oval)
        oq, oscale, odt = orc.adaptive_quantize(cf, "bf16", 8)
        assert np.array_equal(out.grad_fn.saved_tensors[0].cpu().numpy().reshape(-1), oq)
        assert out.grad_fn.saved_tensors[2].item() == oscale and odt == "bf16"

    def check_refresh(layer, x, prior, li, step):
        """The installed basis against orthonormalize(oja_step) in fp64 by projector distance.  The
        layer keeps its basis in bf16, so each entry carries a relative rounding of at most 2^-9:
        the projector of 16 orthonormal columns (Frobenius norm 4) then moves by at most about
        2 * 2^-9 * 4, 0.4 % of its norm; the bound is 1 %.  The step must also have moved the basis
        well beyond that bound (so a refresh on the wrong X, basis or rate would show)."""
        announce("cfg4 refresh basis", li, step)
        lr = float(layer.layer_state["last_oja_lr"])
        _, m64 = orc.oja_step(_np(x), _np(prior), lr)
        ref = orc.orthonormalize(m64)
        got = layer.effective_basis.detach().double().cpu().numpy()
        assert got.shape == ref.shape == (x.shape[1], 16)
        p_ref = ref @ ref.T
        dist = np.linalg.norm(got @ got.T - p_ref) / np.linalg.norm(p_ref)
        q0 = _np(prior).astype(np.float64)
        moved = np.linalg.norm(q0 @ q0.T - p_ref) / np.linalg.norm(p_ref)
        print(f"refresh layer {li} step {step}: projector distance {dist:.3g}, prior basis {moved:.3g}", flush=True)
        assert dist <= 1e-2, dist
        assert moved >= 5e-2, moved

    rows, dims = 16 * 2048, ((2048, 8192), (8192, 2048))
    cfg = _cfg(rank=16, rank_mode="sensitivity", rank_min=4, rank_max=16, rank_adjust_interval=5,
               residual_mode="topk", residual_budget=0.005, quantize_coefficients=True, quantize_residuals=True,
               residual_quantize_bits=8, freeze_basis_after_warmup=True, warmup_steps=0, refresh_trigger="hybrid",
               refresh_period=10, refresh_energy_threshold=0.1, basis_dtype="bfloat16")
    model = nn.Sequential(nn.Linear(*dims[0]), nn.Linear(*dims[1])).to(dev, torch.bfloat16)
    layers = adaptive.apply_adaptive_stacr(model, cfg, surface="all", min_features=1)
    assert len(layers) == 2 and [lay.layer_index for lay in layers] == [0, 1]
    check_steps = {0, 10, 25, 49}
    first_refresh = {li: min(s for s in range(1, 50) if is_fixed_refresh_step(s, 0, 10, li, 2)) for li in (0, 1)}
    energy_refresh_steps = {0: [], 1: []}
    for step in range(50):
        adaptive.set_stacr_runtime_state(model, step)
        for li, (layer, (d_in, d_out)) in enumerate(zip(layers, dims)):
            before = layer.layer_state["refresh_count_total"]
            x = _drifting_activation(rows, d_in, step, 11 + li, dev).to(torch.bfloat16)
            prior = layer.effective_basis.detach().clone() if step == first_refresh[li] else None
            out = layer(x)
            fixed = is_fixed_refresh_step(step, 0, 10, li, 2)
            fired = layer.layer_state["refresh_count_total"] - before
            energy = layer.layer_state["last_residual_energy"]
            if fixed:
                assert fired == 1, f"layer {li} step {step}: scheduled refresh did not fire"
            elif fired:
                assert energy > 0.1, f"layer {li} step {step}: refresh fired without a trigger"
                energy_refresh_steps[li].append(step)
            active = layer.layer_state["active_rank"]
            assert 4 <= active <= 16
            g = torch.randn(rows, d_out, generator=torch.Generator(device=dev).manual_seed(500 + step),
                            device=dev).to(torch.bfloat16)
            if step == first_refresh[li]:
                check_refresh(layer, x, prior, li, step)
            if step in (0, first_refresh[li] + 1):
                check_save(out, x, li, step)
            if step in check_steps:
                announce("cfg4 dW", li, step)
                coeff, idx, values = _saved_factors(out, cfg, rows, d_in)
                cols = torch.randperm(d_out, generator=torch.Generator().manual_seed(step))[:256]
                basis = out.grad_fn.basis
                out.backward(g)
                oidx = idx.cpu().numpy().astype(np.int64)
                orc.check_indices(oidx, rows * d_in, ascending=True)
                odw, _ = orc.weight_grad(_np(g)[:, cols.numpy()], _np(coeff), _np(basis), oidx, _np(values), d_in)
                got = _np(layer.linear.weight.grad)[cols.numpy()]
                assert_rounded_once_bf16(got, odw, what=f"cfg4 layer {li} step {step} dW")
                layer.zero_grad(set_to_none=True)
            else:
                out.backward(g)
                layer.zero_grad(set_to_none=True)
    for li, layer in enumerate(layers):
        scheduled = sum(is_fixed_refresh_step(s, 0, 10, li, 2) for s in range(50))
        assert layer.layer_state["refresh_count_total"] == scheduled + len(energy_refresh_steps[li])
        assert int(layer.step_counter) == 50
        assert layer.layer_state["rank_trajectory"], "the controller never ran"
        # the scheduled refreshes took Y from their forward's save (X read once more, not twice)
        assert layer.layer_state.get("oja_given_y_steps", 0) >= scheduled, layer.layer_state.get("oja_given_y_steps")
    print("energy-triggered refreshes:", energy_refresh_steps, flush=True)


ABLOCK_CASES = [
    # rows, d, chunk, block, budget, dtype
    (1024, 512, 512, 16, 0.01, "bf16"),    # whole blocks, two chunks, global cut
    (1000, 100, 256, 16, 0.02, "f32"),     # padded row ends, partial last chunk
    (300, 40, 64, 8, 0.05, "f16"),         # int16 indices (12,000 elements), padding
    (2048, 1000, 512, 16, 0.003, "bf16"),  # padded, per-chunk candidates cut to k_blocks
    (16 * 2048, 2048, 512, 16, 0.005, "bf16"),  # config 4's input width at its token count
]


@pytest.mark.parametrize("case", ABLOCK_CASES, ids=[f"{c[0]}x{c[1]}_{c[5]}" for c in ABLOCK_CASES])
def test_adaptive_block_sparse_matches_oracle(dev, case):
    from stacr_amd import adaptive

    rows, d, chunk, bs, budget, dtype = case
    announce("adaptive block_sparse", *case)
    tdt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    x = make_activation(rows, d, lognormal=True).to(dev, tdt)
    q = make_basis(d, 8).to(dev, tdt)
    coeff, _, _, _ = adaptive.save(x, q, 0.0)
    idx, values = adaptive.select_block_sparse(x, coeff, q, budget, chunk, bs)
    total = rows * d
    assert idx.dtype == (torch.int16 if total < 32768 else torch.int32)
    resid = orc.residual_act(_np(x), _np(coeff), _np(q), dtype)
    oidx, oval = orc.adaptive_select_block_sparse(resid, budget, chunk, bs, dtype)
    got = idx.cpu().numpy().astype(np.int64)
    orc.check_indices(got, total, ascending=True)
    assert np.array_equal(got, oidx)
    assert np.array_equal(_np(values), oval)


def test_adaptive_default_block_sparse_layer_weight_gradient(dev):
    """The adaptive engine's defaults (block_sparse, int8 coefficients, int4 residual values) through
    the layer: dW from the saved factors against the oracle."""
    announce("adaptive default layer")
    rows, d_in, d_out = 2048, 1000, 300
    cfg = _cfg(rank=16)  # residual_mode block_sparse, quantized coefficients and int4 residuals
    layer = _layer(dev, d_in, d_out, cfg)
    out = layer(make_activation(rows, d_in, lognormal=True).to(dev))
    coeff, idx, values = _saved_factors(out, cfg, rows, d_in)
    assert out.grad_fn.saved_tensors[0].dtype == torch.int8
    assert idx.numel() > 0
    g = make_grad(rows, d_out).to(dev)
    out.backward(g)
    oidx = idx.cpu().numpy().astype(np.int64)
    orc.check_indices(oidx, rows * d_in, ascending=True)
    odw, _ = _oracle_dw(g, _np(coeff), out.grad_fn.basis, oidx, _np(values), d_in)
    assert rel_l2(_np(layer.linear.weight.grad), odw) <= 1e-5


def test_basis_sharing_layers_use_and_refresh_one_basis(dev):
    """basis_sharing="every_2" (stacr/adaptive.py:2735-2792, 3100-3115, 3555-3580, 3368-3378): the
    group's first layer fits the basis from its batch and the second uses that basis without
    fitting its own; an Oja step by either layer replaces the group's basis for both; the basis
    travels in _shared_basis_state through state_dict into an empty pool; and dW on the shared
    basis matches the fp64 oracle on the saved factors."""
    from stacr_amd.adaptive import STACRLinear, get_basis_pool

    announce("adaptive basis sharing")
    pool = get_basis_pool()
    pool.clear()
    rows, d_in, d_out = 512, 256, 128
    cfg = _cfg(rank=8, basis_sharing="every_2", rank_mode="fixed", residual_mode="topk", residual_budget=0.01,
               quantize_coefficients=False)
    torch.manual_seed(3)
    first = STACRLinear(d_in, d_out, cfg, layer_index=0).to(dev)
    second = STACRLinear(d_in, d_out, cfg, layer_index=1).to(dev)
    assert first.basis is None and second.basis is None and not pool.is_initialized(0, d_in, 8)
    first(make_activation(rows, d_in).to(dev)).sum().backward()
    assert pool.is_initialized(0, d_in, 8) and first.basis_initialized
    before = second.effective_basis.clone()
    x = make_activation(rows, d_in, seed=99).to(dev)
    out = second(x)
    assert torch.equal(out.grad_fn.basis, before)  # the group's basis, not a fit of its own batch
    assert first.effective_basis is second.effective_basis
    shared = first.effective_basis.clone()
    second._update_basis_oja(x)
    assert not torch.equal(first.effective_basis, shared)
    assert first.effective_basis is second.effective_basis
    state = first.state_dict()
    assert torch.equal(state["_shared_basis_state"], first.effective_basis)
    pool.clear()
    fresh = STACRLinear(d_in, d_out, cfg, layer_index=1).to(dev)
    fresh.load_state_dict(state)
    assert torch.equal(fresh.effective_basis, state["_shared_basis_state"])
    g = make_grad(rows, d_out).to(dev)
    coeff, idx, values = _saved_factors(out, cfg, rows, d_in)
    used = out.grad_fn.basis
    out.backward(g)
    oidx = idx.cpu().numpy().astype(np.int64)
    orc.check_indices(oidx, rows * d_in, ascending=True)
    odw, _ = _oracle_dw(g, _np(coeff), used, oidx, _np(values), d_in)
    assert rel_l2(_np(second.linear.weight.grad), odw) <= 1e-5
    pool.clear()
