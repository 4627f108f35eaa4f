"""Host-side contract of the drop-in API, on CPU (no kernel launches).

Mirrors the reference's CPU tests for what runs without the save/backward arithmetic:
option validation before any mutation (tests/test_integration.py:170-175), surface selection
(tests/test_surgery.py, tests/test_layers.py:72-84), Turbo configuration (tests/test_surgery.py:
141-160), exact native paths (tests/test_integration.py:59-71), stored_bytes rules
(stacr/layers.py:402-473).  Training forwards on CPU tensors must fail loudly: the product path has
no CPU implementation.
"""
import pytest
import torch
from torch import nn
from torch.nn import functional as F

import stacr_amd
from stacr_amd import STACRLinear, apply_stacr, classify, select_target_names, set_step
from stacr_amd.memory import stacr_stored_bytes
from oracle import oracle as orc


class _Proj(nn.Module):
    """GPT-2 Conv1D convention: weight stored (in, out)."""

    def __init__(self, nin, nout):
        super().__init__()
        self.weight = nn.Parameter(torch.randn(nin, nout) * 0.02)
        self.bias = nn.Parameter(torch.zeros(nout))

    def forward(self, x):
        return x @ self.weight + self.bias


_Proj.__name__ = "Conv1D"


def _gpt2_like(hidden=512):
    block = nn.Module()
    block.attn = nn.Module()
    block.attn.c_attn = nn.Linear(hidden, 3 * hidden)
    block.attn.c_proj = nn.Linear(hidden, hidden)
    block.mlp = nn.Module()
    block.mlp.c_fc = nn.Linear(hidden, 4 * hidden)
    block.mlp.c_proj = nn.Linear(4 * hidden, hidden)
    root = nn.Module()
    root.h = nn.ModuleList([block])
    return root


def make_layer(**options):
    return STACRLinear.from_linear(nn.Linear(16, 7), rank=4, **options)


@pytest.mark.parametrize(
    "options",
    [dict(rank=0), dict(rank=1.5), dict(residual_bits=7), dict(residual_budget=-1), dict(residual_budget=1.1),
     dict(update_interval=0), dict(chunk_rows=0), dict(residual_mode="typo"), dict(basis_dtype="typo"),
     dict(turbo_after_step=-1), dict(oja_lr=float("nan")), dict(residual_sample_ratio=0.0)],
)
def test_invalid_layer_options_fail_before_wrapping(options):
    model = nn.Sequential(nn.Linear(16, 7), nn.Linear(7, 2))
    with pytest.raises((ValueError, TypeError)):
        apply_stacr(model, surface="all", min_features=1, **options)
    assert isinstance(model[0], nn.Linear) and isinstance(model[1], nn.Linear)


def test_mlp_surface_excludes_attention_projections():
    names = select_target_names(_gpt2_like(), surface="mlp", min_features=256)
    assert any(n.endswith("mlp.c_fc") for n in names)
    assert any(n.endswith("mlp.c_proj") for n in names)
    assert not any("attn" in n for n in names)
    names = select_target_names(_gpt2_like(), surface="attention", min_features=256)
    assert names and all("attn" in n for n in names)


def test_classify_by_parent_block():
    assert classify("encoder.layer.0.attention.output.dense") == "attention"
    assert classify("encoder.layer.0.output.dense") == "mlp"
    assert classify("encoder.layer.0.intermediate.dense") == "mlp"
    assert classify("model.decoder.layers.3.fc1") == "mlp"
    assert classify("model.decoder.layers.3.self_attn.fc1") is None
    assert classify("lm_head") is None


def test_min_features_and_explicit_selection():
    model = nn.Sequential(nn.Linear(64, 256), nn.GELU(), nn.Linear(256, 64))
    assert select_target_names(model, surface="all", min_features=1024) == []
    assert select_target_names(model, surface="all", min_features=128) == ["2"]
    assert select_target_names(model, surface="none", extra_names=["0"]) == ["0"]
    with pytest.raises(ValueError, match="Unknown target"):
        select_target_names(model, target_names=["nope"])
    with pytest.raises(ValueError, match="not supported"):
        select_target_names(model, target_names=["1"])


def test_surgery_keeps_parameters_and_aliases():
    shared = nn.Linear(16, 16)
    model = nn.Sequential(shared, shared)
    before = shared.weight.detach().clone()
    layers = apply_stacr(model, surface="all", min_features=1, rank=4)
    assert len(layers) == 1 and model[0] is model[1]
    assert layers[0].weight is shared.weight and torch.equal(layers[0].weight, before)


def test_custom_target_selection_and_step_helper():
    model = nn.Sequential(nn.Linear(16, 7), nn.Linear(7, 2))
    layers = apply_stacr(model, target_names=["1"], rank=2)
    assert len(layers) == 1 and isinstance(model[0], nn.Linear)
    set_step(model, 4)
    assert model[1].step == 4
    with pytest.raises(ValueError, match="Unknown STAC-R"):
        apply_stacr(model, rnak=2)
    with pytest.raises(ValueError):
        set_step(model, -1)
    with pytest.raises(ValueError):
        set_step(model, 1, microbatch_index=2, accum_steps=2)


def test_empty_selection_is_explicit_and_frozen_weights_are_skipped():
    model = nn.Sequential(nn.Linear(16, 7))
    with pytest.raises(ValueError, match="No trainable"):
        apply_stacr(model)
    assert apply_stacr(model, allow_empty=True) == []
    model[0].weight.requires_grad_(False)
    assert apply_stacr(model, surface="all", min_features=1, allow_empty=True) == []


@pytest.mark.parametrize(
    "config,overrides,expected",
    [(None, {}, 50), ({}, {}, 50), ({"turbo_after_step": None}, {}, None), ({"turbo_after_step": 17}, {}, 17),
     ({"turbo_after_step": 17}, {"turbo_after_step": None}, None),
     (stacr_amd.STACRConfig(), {}, None), (stacr_amd.STACRConfig(), {"turbo_after_step": 50}, 50)],
)
def test_apply_stacr_honors_explicit_turbo_configuration(config, overrides, expected):
    """Reference tests/test_surgery.py:130-148, including the compressor's config dataclass."""
    model = nn.Sequential(nn.Linear(12, 7))
    layers = apply_stacr(model, config, surface="all", min_features=1, rank=3, **overrides)
    assert layers[0].turbo_after_step == expected
    assert STACRLinear.from_linear(nn.Linear(12, 7), rank=3).turbo_after_step is None
    assert stacr_amd.STACRConfig().turbo_after_step is None


def test_saved_tensor_hooks_never_compress_parameter_views():
    """Reference tests/test_adaptive.py:222-226: a parameter, or a view of one (linear autograd
    saves the transposed weight), is never compressed; activations of the right size are."""
    from stacr_amd.compressor import STACRCompressor, STACRConfig

    weight = nn.Parameter(torch.randn(7, 16))
    compressor = STACRCompressor(STACRConfig(min_features=1, min_numel=1))
    assert not compressor.should_compress(weight.t())
    assert not compressor.should_compress(weight)
    assert compressor.should_compress(torch.randn(3, 16))
    assert not compressor.should_compress(torch.randn(16))  # one dimension
    assert not compressor.should_compress(torch.arange(48).reshape(3, 16))  # integer
    big = STACRCompressor(STACRConfig())  # defaults: >= 128 features and >= 4096 elements
    assert not big.should_compress(torch.randn(64, 64)) and not big.should_compress(torch.randn(8, 128))
    assert big.should_compress(torch.randn(32, 128))
    # pack passes ineligible tensors (and everything during warmup) through untouched
    assert compressor.pack(weight) is weight
    warm = STACRCompressor(STACRConfig(min_features=1, min_numel=1, warmup_steps=3))
    t = torch.randn(4, 16)
    assert warm.pack(t) is t and warm.unpack(t) is t


def test_sparse_residual_dense_scatters_flat_indices():
    """stacr/residual.py:13-20: zeros away from the entries, the values at their flat indices."""
    from stacr_amd.compressor import SparseResidual

    r = SparseResidual((2, 3), torch.tensor([5, 0, 3]), torch.tensor([1.5, -2.0, 4.0]))
    d = r.dense(device=torch.device("cpu"), dtype=torch.float32)
    assert torch.equal(d, torch.tensor([[-2.0, 0.0, 0.0], [4.0, 0.0, 1.5]]))
    empty = SparseResidual((2, 2), torch.empty(0, dtype=torch.long), torch.empty(0))
    assert torch.equal(empty.dense(device=torch.device("cpu"), dtype=torch.bfloat16), torch.zeros(2, 2, dtype=torch.bfloat16))


def test_conv1d_is_wrapped_transposed_and_basis_follows_weight_device():
    root = nn.Module()
    root.mlp = nn.Module()
    root.mlp.c_fc = _Proj(256, 512)
    layers = apply_stacr(root, surface="mlp", min_features=128, rank=8)
    assert layers[0].transposed and layers[0].in_features == 256 and layers[0].out_features == 512
    assert layers[0].basis.device == layers[0].weight.device
    with pytest.raises(TypeError):
        STACRLinear.from_linear(nn.Conv2d(3, 3, 1))


@pytest.mark.parametrize("mode", ["eval", "no_grad", "frozen"])
def test_exact_paths_do_not_initialize_or_refresh_basis(mode):
    layer = make_layer()
    if mode == "eval":
        layer.eval()
    if mode == "frozen":
        layer.weight.requires_grad_(False)
    x = torch.randn(5, 16, requires_grad=True)
    with torch.set_grad_enabled(mode != "no_grad"):
        actual = layer(x)
        expected = F.linear(x, layer.weight, layer.bias)
    assert torch.equal(actual, expected)
    assert not bool(layer.basis_ready)
    if mode != "no_grad":
        actual.sum().backward()
        assert x.grad is not None


def test_cpu_training_forward_fails_loudly():
    layer = make_layer()
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        layer(torch.randn(5, 16))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        stacr_amd.quantize_values(torch.randn(4), 8)
    q = stacr_amd.quantize_values(torch.randn(4), 0)  # bits 0 is a passthrough
    assert q.bits == 0 and q.scale.item() == 1.0


@pytest.mark.parametrize("bits", [0, 4, 8])
def test_stored_bytes_matches_payload_estimate(bits):
    layer = STACRLinear.from_linear(nn.Linear(16, 7), rank=4, residual_budget=0.25, residual_bits=bits)
    estimate = stacr_stored_bytes((5, 16), rank=4, dtype=torch.float32, residual_budget=0.25, residual_bits=bits,
                                  basis_dtype=torch.float32, include_basis=True)
    assert estimate == layer.stored_bytes(5, value_bytes=4)["total"]


@pytest.mark.parametrize("rows,chunk,budget", [(5, 1, 0.17), (8192, 512, 0.005), (37, 8, 0.05), (5, 2, 0.25)])
def test_stored_bytes_count_equals_selected_count(rows, chunk, budget):
    layer = STACRLinear.from_linear(nn.Linear(16, 7), rank=4, residual_mode="chunk_topk", chunk_rows=chunk,
                                    residual_budget=budget)
    k_total, k_sum = orc.residual_plan(rows, 16, "chunk_topk", budget, chunk)
    assert layer.stored_bytes(rows)["residual_count"] == min(k_total, k_sum)
    layer.residual_mode = "global_topk"
    assert layer.stored_bytes(rows)["residual_count"] == k_total


def test_turbo_schedule_and_step_property():
    layer = make_layer(turbo_after_step=2)
    assert not layer._turbo()
    layer.step = 2
    assert layer._turbo() and layer.step == 2
    assert layer.stored_bytes(5)["residual_count"] == 0
    with pytest.raises(ValueError):
        layer.set_step(True)


def test_stored_bytes_closed_forms_and_reference_known_answers():
    from stacr_amd.memory import dense_bytes, saved_surface_predictor

    # reference tests/test_memory.py:7-15
    assert stacr_stored_bytes((8, 512), rank=8, dtype=torch.float16, residual_budget=0.005) < dense_bytes(
        (8, 512), torch.float16)
    assert saved_surface_predictor(10, 100) == 0.1
    assert saved_surface_predictor(-3, 100) == 0.0
    with pytest.raises(ValueError):
        saved_surface_predictor(1, 0)
    # (5, 16), rank 4, fp32, budget 0.25, int8 residual: 80 B coeff; 20 entries x (4 idx + 1) + 4 scale
    assert stacr_stored_bytes((5, 16), 4, torch.float32, 0.25, residual_bits=8) == 80 + 20 * 5 + 4
    # + an fp32 basis 16 x 4; int4 coefficients pack two per byte and add a scale
    assert stacr_stored_bytes((5, 16), 4, torch.float32, 0.25, residual_bits=8, include_basis=True) == 184 + 256
    assert stacr_stored_bytes((5, 16), 4, torch.float32, 0.0, coeff_bits=4) == 10 + 4
    assert stacr_stored_bytes((5, 16), 4, torch.float32, 0.0, coeff_bits=4, include_scales=False) == 10
    # residual_bits=0 keeps dtype values plus a unit scale; None keeps values without a scale
    assert stacr_stored_bytes((5, 16), 4, torch.bfloat16, 0.25, residual_bits=0) == 40 + 20 * 6 + 4
    assert stacr_stored_bytes((5, 16), 4, torch.bfloat16, 0.25) == 40 + 20 * 6
    assert stacr_stored_bytes((2, 3, 64), 100, torch.float16, 0.0) == 6 * 64 * 2  # rank capped at features
    assert stacr_stored_bytes((3, 0), 4) == 0 and stacr_stored_bytes((), 4) == 2
    for bad in (dict(rank=0), dict(rank=True), dict(residual_budget=1.5), dict(index_bytes=3),
                dict(coeff_bits=2), dict(residual_bits=16)):
        args = dict(shape=(5, 16), rank=4) | bad
        with pytest.raises(ValueError):
            stacr_stored_bytes(**args)
    with pytest.raises(ValueError, match="nonnegative"):
        dense_bytes((2, -1), torch.float32)
