"""Model surgery: choose linear projections by surface and swap in STACRLinear in place.

Behaviour of stacr/surgery.py: ``classify`` (:241-251) places a module on the MLP or attention
surface by its parent block, since GPT-2 names both the MLP and attention output "c_proj" and
BERT names both feed-forward and attention outputs "dense"; ``select_target_names`` (:254-315);
``apply_stacr`` (:318-399) builds the whole replacement plan before mutating anything and
defaults to Turbo after optimizer step 50; ``set_step`` (:402-430).  The name tables below are the
reference's, kept identical so the same modules are selected.
"""
from __future__ import annotations

import inspect
import re
from dataclasses import asdict, is_dataclass
from typing import Any, Iterable

from torch import nn

from .layers import STACRLinear

MLP_PARENTS = ("mlp", "ffn", "feed_forward", "intermediate")
ATTENTION_PARENTS = ("attn", "attention", "self_attn", "self_attention", "crossattention")
MLP_LEAVES = ("c_fc", "c_proj", "dense", "dense_h_to_4h", "dense_4h_to_h", "gate_proj", "up_proj", "down_proj",
              "fc1", "fc2", "w1", "w2", "w3")
ATTENTION_LEAVES = ("c_attn", "c_proj", "dense", "q_proj", "k_proj", "v_proj", "o_proj", "out_proj", "query", "key",
                    "value", "query_key_value")
# OPT keeps fc1/fc2 directly on the decoder layer (no "mlp" parent); these two leaf names never
# denote attention projections, so they are MLP by name alone once no attention parent matched.
UNAMBIGUOUS_MLP_LEAVES = ("fc1", "fc2")

SURFACES = {"mlp": {"mlp"}, "attention": {"attention"}, "mlp+attention": {"mlp", "attention"}, "all": None,
            "none": None}


def _is_conv1d(module: nn.Module) -> bool:
    return type(module).__name__ == "Conv1D" and hasattr(module, "weight") and module.weight.dim() == 2


def _feature_count(module: nn.Module) -> int | None:
    if isinstance(module, nn.Linear):
        return int(module.in_features)
    if _is_conv1d(module):
        return int(module.weight.shape[0])
    return None


def classify(name: str) -> str | None:
    """'attention', 'mlp' or None for the module at dotted path ``name``."""
    *parents, leaf = name.split(".")
    parents = set(parents)
    if parents.intersection(ATTENTION_PARENTS):
        return "attention" if leaf in ATTENTION_LEAVES else None
    if parents.intersection(MLP_PARENTS) or "output" in parents:
        return "mlp" if leaf in MLP_LEAVES else None
    return "mlp" if leaf in UNAMBIGUOUS_MLP_LEAVES else None


def _as_set(values) -> set:
    return {values} if isinstance(values, str) else set(values)


def select_target_names(model: nn.Module, *, surface: str = "mlp", min_features: int = 256,
                        extra_names: Iterable[str] = (), target_names: Iterable[str] | None = None,
                        target_pattern: str | None = None, exclude_names: Iterable[str] = (),
                        trainable_only: bool = True) -> list[str]:
    """Names of trainable linear projections on ``surface``, or matching explicit names / a regex.

    ``target_names`` and ``target_pattern`` restrict; ``extra_names`` add (explicit names bypass
    ``min_features``).
    """
    if surface not in SURFACES:
        raise ValueError(f"Unknown surface: {surface!r}")
    if isinstance(min_features, bool) or int(min_features) != min_features or min_features < 1:
        raise ValueError("min_features must be a positive integer")
    extras = _as_set(extra_names)
    targets = None if target_names is None else _as_set(target_names)
    excluded = _as_set(exclude_names)
    regex = None if target_pattern is None else re.compile(target_pattern)
    modules = dict(model.named_modules(remove_duplicate=False))
    explicit = extras | (targets or set())
    unknown = explicit - modules.keys()
    if unknown:
        raise ValueError(f"Unknown target module names: {sorted(unknown)}")
    unsupported = [n for n in explicit if _feature_count(modules[n]) is None]
    if unsupported:
        raise ValueError(f"Targets are not supported linear projections: {sorted(unsupported)}")
    wanted = SURFACES[surface]
    chosen = []
    for name, module in modules.items():
        feats = _feature_count(module)
        if feats is None or name in excluded:
            continue
        if trainable_only and not module.weight.requires_grad:
            continue
        if targets is not None and name not in targets:
            continue
        if regex is not None and regex.search(name) is None:
            continue
        if feats < int(min_features) and name not in explicit:
            continue
        if surface == "all" or name in explicit or targets is not None or regex is not None:
            chosen.append(name)
        elif wanted is not None and classify(name) in wanted:
            chosen.append(name)
    return chosen


_SELECTION_KEYS = {"surface", "min_features", "extra_names", "target_names", "target_pattern", "exclude_names",
                   "trainable_only", "allow_empty"}
# accepted for compatibility with the saved-tensor storage config; only their defaults are valid
_COMPAT_KEYS = {"min_numel", "post_warmup_mode"}


def _layer_keys() -> set:
    params = set(inspect.signature(STACRLinear.__init__).parameters)
    return params - {"self", "weight", "bias", "transposed"}


def apply_stacr(model: nn.Module, config: dict[str, Any] | None = None, **overrides: Any) -> list[STACRLinear]:
    """Replace the selected projections with STACRLinear in place; returns the new layers.

    Defaults to Turbo after optimizer step 50 (basis frozen, residual dropped; weights keep
    training).  Pass turbo_after_step=None for full STAC-R.  A config object (dataclass) is
    taken as given, so its own turbo_after_step (None) wins over the default.
    """
    cfg: dict[str, Any] = asdict(config) if is_dataclass(config) else dict(config or {})
    cfg.update(overrides)
    cfg.setdefault("turbo_after_step", 50)
    layer_keys = _layer_keys()
    unknown = cfg.keys() - layer_keys - _SELECTION_KEYS - _COMPAT_KEYS
    if unknown:
        raise ValueError(f"Unknown STAC-R options: {sorted(unknown)}")
    if cfg.get("post_warmup_mode", "full") != "full":
        raise ValueError("Use turbo_after_step to switch the factor-native layer to Turbo")
    names = select_target_names(
        model,
        surface=str(cfg.get("surface", "mlp")),
        min_features=cfg.get("min_features", 256),
        extra_names=cfg.get("extra_names", ()),
        target_names=cfg.get("target_names"),
        target_pattern=cfg.get("target_pattern"),
        exclude_names=cfg.get("exclude_names", ()),
        trainable_only=cfg.get("trainable_only", True),
    )
    if "" in names:
        raise ValueError("For a standalone linear module use STACRLinear.from_linear(model, ...)")
    if not names and not cfg.get("allow_empty", False) and cfg.get("surface") != "none":
        raise ValueError("No trainable linear projections matched. Select surface='all', supply target_names, "
                         "lower min_features, or explicitly set allow_empty=True.")
    options = {k: cfg[k] for k in layer_keys if k in cfg}
    # every layer is constructed (and validated) before the model is touched
    plan, built = [], {}
    for name in names:
        *path, leaf = name.split(".")
        parent = model
        for part in path:
            parent = getattr(parent, part)
        module = getattr(parent, leaf)
        layer = built.get(id(module))
        if layer is None:
            layer = STACRLinear.from_linear(module, **options)
            layer.source_name = name
            built[id(module)] = layer
        plan.append((parent, leaf, layer))
    wrapped: list[STACRLinear] = []
    for parent, leaf, layer in plan:
        setattr(parent, leaf, layer)
        if all(layer is not w for w in wrapped):
            wrapped.append(layer)
    return wrapped


def set_step(layers: Iterable[STACRLinear] | nn.Module, step: int, *, microbatch_index: int = 0,
             accum_steps: int = 1) -> None:
    """Set the optimizer step on every STACRLinear in ``layers`` (or in a model)."""
    if isinstance(step, bool) or int(step) != step or step < 0:
        raise ValueError("step must be a nonnegative integer")
    if int(accum_steps) != accum_steps or accum_steps < 1:
        raise ValueError("accum_steps must be a positive integer")
    if int(microbatch_index) != microbatch_index or not 0 <= microbatch_index < accum_steps:
        raise ValueError("microbatch_index must be in [0, accum_steps)")
    if isinstance(layers, nn.Module):
        layers = [m for m in layers.modules() if isinstance(m, STACRLinear)]
    for layer in layers:
        layer.set_step(step)
