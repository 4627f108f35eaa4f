"""Adaptive engine host logic on the CPU (no kernel launches): configuration, surgery, schedule
and persistent state.  Mirrors the reference's CPU-runnable adaptive tests
(tests/test_adaptive.py:127-208, 242-247); training forwards need the HIP save and are GPU tests.
"""
import copy

import pytest
import torch
from torch import nn

import stacr_amd
from stacr_amd.adaptive import (STACRConfig, STACRLinear, apply_adaptive_stacr, profile_layer_spectrum,
                                set_stacr_runtime_state)


def test_config_rejects_unimplemented_or_invalid_settings():
    """Reference tests/test_adaptive.py:197-208."""
    for options in [dict(streaming_algorithm="incremental_svd"), dict(update_interval=0), dict(residual_budget=2),
                    dict(rank=0), dict(residual_quantize_bits=2), dict(basis_sharing="all", rank_mode="sensitivity"),
                    dict(rank_min=9, rank_max=8), dict(oja_learning_rate=float("inf")), dict(quantize_bits=4),
                    dict(residual_mode="typo"), dict(warmup_steps=-1), dict(basis_dtype="int8")]:
        with pytest.raises(ValueError):
            STACRConfig(**options)


def test_config_dict_and_schedules():
    cfg = STACRConfig(rank=16, residual_schedule="linear", residual_start=0.05, residual_end=0.01)
    d = cfg.to_dict()
    assert "chunk_size" not in d and "joint_qk" not in d and d["rank"] == 16 and len(d) == 62
    assert cfg.get_residual_budget(0, 100) == 0.05
    assert cfg.get_residual_budget(100, 100) == pytest.approx(0.01)
    cos = STACRConfig(residual_schedule="cosine", residual_start=0.05, residual_end=0.01)
    assert cos.get_residual_budget(50, 100) == pytest.approx(0.03)
    heur = STACRConfig(adaptive_layer_rank="heuristic", rank=32)
    assert [heur.get_layer_rank(i, 32, 12) for i in (0, 3, 4, 7, 8, 11)] == [32, 32, 22, 22, 12, 12]
    assert heur.get_layer_rank(11, 16, 12) == 8  # floor of 8


def test_spectrum_profile_closed_form():
    # singular values 4, 2, 1 (energies 16, 4, 1 of 21): 90% needs two directions, 76% one
    x = torch.zeros(6, 5)
    x[0, 0], x[1, 1], x[2, 2] = 4.0, 2.0, 1.0
    assert profile_layer_spectrum(x, 0.90)["adaptive_rank"] == 2
    assert profile_layer_spectrum(x, 0.76)["adaptive_rank"] == 1
    assert profile_layer_spectrum(x, 0.999)["adaptive_rank"] == 3
    assert profile_layer_spectrum(torch.zeros(4, 3), 0.9)["adaptive_rank"] == 1
    assert profile_layer_spectrum(torch.zeros(0, 3), 0.9)["adaptive_rank"] == 1


@pytest.mark.parametrize("mode", ["eval", "no_grad", "frozen"])
def test_exact_paths_do_not_initialize(mode):
    """Reference tests/test_adaptive.py:127-137."""
    layer = STACRLinear(16, 7, STACRConfig(rank=4))
    if mode == "eval":
        layer.eval()
    if mode == "frozen":
        layer.linear.weight.requires_grad_(False)
    with torch.set_grad_enabled(mode != "no_grad"):
        x = torch.randn(3, 16)
        assert torch.equal(layer(x), layer.linear(x))
    assert not layer.basis_initialized and int(layer.step_counter) == 0


def test_surgery_preserves_parameters_and_rng():
    """Reference tests/test_adaptive.py:140-148 (without the training step, which needs a GPU)."""
    model = nn.Sequential(nn.Linear(16, 7))
    parameters = list(model.parameters())
    rng = torch.get_rng_state()
    layers = apply_adaptive_stacr(model, {"rank": 4}, target_names=["0"])
    assert torch.equal(rng, torch.get_rng_state())
    assert all(a is b for a, b in zip(parameters, model.parameters()))
    assert layers[0].source_name == "0" and layers[0].layer_index == 0 and layers[0].num_layers == 1


def test_conv1d_surgery_keeps_original_parameter_identity():
    """Reference tests/test_adaptive.py:151-170 (eval forward; training forwards are GPU tests)."""
    class Conv1D(nn.Module):
        def __init__(self):
            super().__init__()
            self.weight = nn.Parameter(torch.randn(16, 7))
            self.bias = nn.Parameter(torch.randn(7))

        def forward(self, x):
            return torch.addmm(self.bias, x, self.weight)

    model = nn.Sequential(Conv1D())
    weight = model[0].weight
    x = torch.randn(8, 16)
    expected = model(x)
    apply_adaptive_stacr(model, rank=4, target_names=["0"])
    assert weight is model[0].linear.source_weight
    assert model[0].in_features == 16 and model[0].out_features == 7
    model.eval()
    assert torch.allclose(model(x), expected, atol=1e-5)


def test_apply_adaptive_validates_before_mutation():
    model = nn.Sequential(nn.Linear(16, 7), nn.Linear(7, 300))
    for options in (dict(rank=0), dict(joint_qk=True), dict(min_adaptation_steps=3),
                    dict(use_random_qr_init=True, warmup_steps=2), dict(target_names=["nope"])):
        with pytest.raises(ValueError):
            apply_adaptive_stacr(model, **options)
        assert isinstance(model[0], nn.Linear) and isinstance(model[1], nn.Linear)
    with pytest.raises(ValueError, match="No trainable"):
        apply_adaptive_stacr(model, surface="mlp")
    assert apply_adaptive_stacr(model, surface="mlp", allow_empty=True) == []
    assert isinstance(model[0], nn.Linear)


def test_basis_sharing_groups_and_pool():
    """Sharing groups from the layer index (stacr/adaptive.py:2735-2792) and the pool's contract:
    zero until fitted, replaced (not written into) by an update, keyed by (group, in_features, rank)."""
    from stacr_amd.adaptive import STACRConfig, STACRLinear, get_basis_pool

    pool = get_basis_pool()
    pool.clear()
    groups = {}
    for mode, expect in (("all", [0, 0, 0, 0, 0]), ("every_2", [0, 0, 1, 1, 2]), ("every_3", [0, 0, 0, 1, 1]),
                         ("every_4", [0, 0, 0, 0, 1])):
        cfg = STACRConfig(rank=4, basis_sharing=mode, rank_mode="fixed")
        layers = [STACRLinear(16, 7, cfg, layer_index=i) for i in range(5)]
        assert [lyr.basis_group_id for lyr in layers] == expect and all(lyr.basis is None for lyr in layers)
        groups[mode] = layers
    explicit = STACRLinear(16, 7, STACRConfig(rank=4, basis_sharing="all", basis_sharing_group=9), layer_index=3)
    assert explicit.basis_group_id == 9
    with pytest.warns(UserWarning, match="layer_index not provided"):
        alone = STACRLinear(16, 7, STACRConfig(rank=4, basis_sharing="all"))
    assert not alone.use_basis_sharing and alone.basis is not None
    a, b = groups["every_2"][0], groups["every_2"][1]
    first = a.effective_basis
    assert first is b.effective_basis and not pool.is_initialized(0, 16, 4) and not first.any()
    fitted = torch.linalg.qr(torch.randn(16, 4))[0]
    a._install_basis(fitted)
    assert pool.is_initialized(0, 16, 4) and torch.equal(b.effective_basis, fitted)
    assert not first.any()  # the tensor an earlier forward took is left as it was
    assert not pool.is_initialized(1, 16, 4)
    pool.clear()


def test_runtime_state_and_set_step_reach_adaptive_layers():
    model = nn.Sequential(nn.Linear(16, 7), nn.Linear(7, 3))
    layers = apply_adaptive_stacr(model, surface="all", min_features=1, rank=2, refresh_trigger="fixed")
    set_stacr_runtime_state(model, 7, microbatch_index=1, accum_steps=4)
    for layer in layers:
        assert layer.layer_state["optimizer_step"] == 7 and layer.layer_state["microbatch_index"] == 1
        assert layer._get_schedule_step() == 7 and layer._get_accum_steps() == 4
    stacr_amd.set_step(model, 9)
    assert all(layer.layer_state["optimizer_step"] == 9 for layer in layers)
    assert [layer.layer_index for layer in layers] == [0, 1]
    # without an optimizer-step schedule the layer's own counter drives the schedule
    plain = STACRLinear(16, 7, STACRConfig(rank=2))
    set_stacr_runtime_state(plain, 5)
    assert plain._get_schedule_step() == 0


def test_state_dict_round_trip_restores_runtime_state_and_basis_shape():
    """Reference tests/test_adaptive.py:39-82, 242-247 for the persistence part."""
    cfg = STACRConfig(rank=8, rank_mode="variance", rank_min=1, rank_max=8, basis_dtype=torch.float32)
    first = STACRLinear(16, 7, cfg)
    first.basis = torch.linalg.qr(torch.randn(16, 3))[0]  # as a fitted variance-rank basis would be
    first.basis_initialized = True
    first.layer_state["rank_trajectory"].append({"step": 0, "active_rank": 3, "reason_code": "x",
                                                  "metric_value": None})
    set_stacr_runtime_state(first, 4)
    second = STACRLinear(16, 7, STACRConfig(rank=8))
    second.load_state_dict(copy.deepcopy(first.state_dict()))
    assert second.basis.shape == (16, 3) and torch.equal(second.basis, first.basis)
    assert second.basis_initialized
    assert second.layer_state == first.layer_state
    assert second.config.rank_mode == "variance"
    # a checkpoint written before the initialized flag existed: a non-zero basis counts as fitted
    old = {k: v for k, v in first.state_dict().items() if k != "_basis_initialized"}
    third = STACRLinear(16, 7, STACRConfig(rank=8))
    third.load_state_dict(old)
    assert third.basis_initialized


def test_training_forward_on_cpu_fails_loudly():
    layer = STACRLinear(16, 7, STACRConfig(rank=4, residual_mode="topk"))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        layer(torch.randn(8, 16))
