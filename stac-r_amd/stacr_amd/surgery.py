"""Model surgery: pick linear projections by surface and swap in STACRLinear in place.

Interface of stacr/surgery.py: `classify` (:70-80), `select_target_names` (:83-144),
`apply_stacr` (:147-228), `set_step` (:231-259), with the same options, defaults (Turbo after
optimizer step 50), error types and messages.  The name tables are the reference's, kept
identical so the same modules land on the same surface (GPT-2 names both its MLP and attention
output projections "c_proj" and BERT both its outputs "dense", so a module is placed by its
parent block, not its leaf name alone).

Structure: `classify` walks an ordered rule table; `select_target_names` builds one `_Criteria`
object that decides each module; `apply_stacr` resolves options, plans every replacement
(constructing, and so validating, every new layer) and only then mutates the model.
"""
from __future__ import annotations

import inspect
import re
from dataclasses import asdict, dataclass, is_dataclass
from typing import Any, Iterable

from torch import nn

from .layers import STACRLinear

MLP_PARENTS = ("mlp", "ffn", "feed_forward", "intermediate")
ATTENTION_PARENTS = ("attn", "attention", "self_attn", "self_attention", "crossattention")
MLP_LEAVES = ("c_fc", "c_proj", "dense", "dense_h_to_4h", "dense_4h_to_h", "gate_proj", "up_proj", "down_proj",
              "fc1", "fc2", "w1", "w2", "w3")
ATTENTION_LEAVES = ("c_attn", "c_proj", "dense", "q_proj", "k_proj", "v_proj", "o_proj", "out_proj", "query", "key",
                    "value", "query_key_value")
# OPT keeps fc1 / fc2 on the decoder layer itself (no MLP parent); those two leaf names never
# name an attention projection, so the leaf alone places them once no parent rule applied.
UNAMBIGUOUS_MLP_LEAVES = ("fc1", "fc2")

# (surface, parent names that claim the module, leaf names accepted under them); the first rule
# whose parents appear on the path decides, so attention wins over an enclosing MLP-like name.
_PARENT_RULES = (
    ("attention", frozenset(ATTENTION_PARENTS), frozenset(ATTENTION_LEAVES)),
    ("mlp", frozenset(MLP_PARENTS) | {"output"}, frozenset(MLP_LEAVES)),
)

SURFACES = {"mlp": frozenset({"mlp"}), "attention": frozenset({"attention"}),
            "mlp+attention": frozenset({"mlp", "attention"}), "all": None, "none": None}


def _in_features(module: nn.Module) -> int | None:
    """Input features of an nn.Linear or a Transformers Conv1D (weight in x out); else None."""
    if isinstance(module, nn.Linear):
        return int(module.in_features)
    weight = getattr(module, "weight", None)
    if type(module).__name__ == "Conv1D" and weight is not None and weight.dim() == 2:
        return int(weight.shape[0])
    return None


def classify(name: str) -> str | None:
    """'attention', 'mlp' or None for the module at dotted path `name`."""
    path = name.split(".")
    parents, leaf = frozenset(path[:-1]), path[-1]
    for surface, claim, leaves in _PARENT_RULES:
        if parents & claim:
            return surface if leaf in leaves else None
    return "mlp" if leaf in UNAMBIGUOUS_MLP_LEAVES else None


def _names(values) -> frozenset:
    return frozenset((values,)) if isinstance(values, str) else frozenset(values)


@dataclass(frozen=True)
class _Criteria:
    surface: str
    min_features: int
    extra: frozenset
    targets: frozenset | None
    pattern: re.Pattern | None
    excluded: frozenset
    trainable_only: bool

    @property
    def explicit(self) -> frozenset:
        return self.extra | (self.targets or frozenset())

    @property
    def restricted(self) -> bool:
        """True when names / a pattern, not the surface, choose among the admitted modules."""
        return self.targets is not None or self.pattern is not None

    def admits(self, name: str, module: nn.Module) -> bool:
        feats = _in_features(module)
        explicit = name in self.explicit
        eligible = (
            feats is not None
            and name not in self.excluded
            and (module.weight.requires_grad or not self.trainable_only)
            and (self.targets is None or name in self.targets)
            and (self.pattern is None or self.pattern.search(name) is not None)
            and (explicit or feats >= self.min_features)
        )
        if not eligible:
            return False
        if self.surface == "all" or explicit or self.restricted:
            return True
        wanted = SURFACES[self.surface]
        return wanted is not None and classify(name) in wanted


def select_target_names(model: nn.Module, *, surface: str = "mlp", min_features: int = 256,
                        extra_names: Iterable[str] = (), target_names: Iterable[str] | None = None,
                        target_pattern: str | None = None, exclude_names: Iterable[str] = (),
                        trainable_only: bool = True) -> list[str]:
    """Names (in module order) of trainable linear projections on `surface`.

    `target_names` and `target_pattern` restrict the choice; `extra_names` add modules (explicit
    names bypass `min_features`); `surface="none"` with `extra_names` gives a custom list.
    """
    if surface not in SURFACES:
        raise ValueError(f"Unknown surface: {surface!r}")
    if isinstance(min_features, bool) or int(min_features) != min_features or min_features < 1:
        raise ValueError("min_features must be a positive integer")
    criteria = _Criteria(surface=surface, min_features=int(min_features), extra=_names(extra_names),
                         targets=None if target_names is None else _names(target_names),
                         pattern=None if target_pattern is None else re.compile(target_pattern),
                         excluded=_names(exclude_names), trainable_only=bool(trainable_only))
    modules = dict(model.named_modules(remove_duplicate=False))
    unknown = criteria.explicit - modules.keys()
    if unknown:
        raise ValueError(f"Unknown target module names: {sorted(unknown)}")
    unsupported = sorted(n for n in criteria.explicit if _in_features(modules[n]) is None)
    if unsupported:
        raise ValueError(f"Targets are not supported linear projections: {unsupported}")
    return [name for name, module in modules.items() if criteria.admits(name, module)]


_SELECTION_OPTIONS = frozenset({"surface", "min_features", "extra_names", "target_names", "target_pattern",
                                "exclude_names", "trainable_only", "allow_empty"})
# keys of the saved-tensor storage config, accepted here with their default values only
_STORAGE_OPTIONS = frozenset({"min_numel", "post_warmup_mode"})
_SELECTION_DEFAULTS = {"surface": "mlp", "min_features": 256, "extra_names": (), "target_names": None,
                       "target_pattern": None, "exclude_names": (), "trainable_only": True}


def _layer_options() -> frozenset:
    return frozenset(inspect.signature(STACRLinear.__init__).parameters) - {"self", "weight", "bias", "transposed"}


def _resolve(config, overrides: dict) -> tuple[dict, dict, dict]:
    """(all options, STACRLinear options, selection options) with Turbo after step 50 unless set."""
    options: dict[str, Any] = asdict(config) if is_dataclass(config) else dict(config or {})
    options.update(overrides)
    options.setdefault("turbo_after_step", 50)
    layer_keys = _layer_options()
    unknown = options.keys() - layer_keys - _SELECTION_OPTIONS - _STORAGE_OPTIONS
    if unknown:
        raise ValueError(f"Unknown STAC-R options: {sorted(unknown)}")
    if options.get("post_warmup_mode", "full") != "full":
        raise ValueError("Use turbo_after_step to switch the factor-native layer to Turbo")
    layer = {k: v for k, v in options.items() if k in layer_keys}
    selection = {k: options.get(k, default) for k, default in _SELECTION_DEFAULTS.items()}
    selection["surface"] = str(selection["surface"])
    return options, layer, selection


def apply_stacr(model: nn.Module, config: dict[str, Any] | None = None, **overrides: Any) -> list[STACRLinear]:
    """Replace the selected projections with STACRLinear in place and return the new layers.

    Defaults to Turbo after optimizer step 50 (basis frozen, residual dropped; the weights keep
    training); pass turbo_after_step=None for full STAC-R.  A config dataclass is taken as given,
    so its own turbo_after_step wins over that default.  Nothing is replaced unless every new
    layer could be built, and a module reached under several names becomes one layer.
    """
    options, layer_options, selection = _resolve(config, overrides)
    names = select_target_names(model, **selection)
    if "" in names:
        raise ValueError("For a standalone linear module use STACRLinear.from_linear(model, ...)")
    if not names and not options.get("allow_empty", False) and options.get("surface") != "none":
        raise ValueError("No trainable linear projections matched. Select surface='all', supply target_names, "
                         "lower min_features, or explicitly set allow_empty=True.")
    by_module: dict[int, STACRLinear] = {}
    plan = []
    for name in names:
        parent_name, _, leaf = name.rpartition(".")
        parent = model.get_submodule(parent_name)
        module = getattr(parent, leaf)
        if id(module) not in by_module:
            layer = STACRLinear.from_linear(module, **layer_options)
            layer.source_name = name
            by_module[id(module)] = layer
        plan.append((parent, leaf, by_module[id(module)]))
    for parent, leaf, layer in plan:
        setattr(parent, leaf, layer)
    # each new layer once, in order of first selection
    return list({id(layer): layer for _, _, layer in plan}.values())


def set_step(layers: Iterable[nn.Module] | nn.Module, step: int, *, microbatch_index: int = 0,
             accum_steps: int = 1) -> None:
    """Set the optimizer step on every STAC-R layer of either engine in `layers` (or a model);
    adaptive layers also take the micro-batch position."""
    from .adaptive import AdaptiveSTACRLinear

    if isinstance(step, bool) or int(step) != step or step < 0:
        raise ValueError("step must be a nonnegative integer")
    if int(accum_steps) != accum_steps or accum_steps < 1:
        raise ValueError("accum_steps must be a positive integer")
    if int(microbatch_index) != microbatch_index or not 0 <= microbatch_index < accum_steps:
        raise ValueError("microbatch_index must be in [0, accum_steps)")
    if isinstance(layers, nn.Module):
        layers = [m for m in layers.modules() if isinstance(m, (STACRLinear, AdaptiveSTACRLinear))]
    for layer in layers:
        if isinstance(layer, AdaptiveSTACRLinear):
            layer.set_runtime_state(optimizer_step=step, microbatch_index=microbatch_index,
                                    accum_steps=accum_steps)
        else:
            layer.set_step(step)


__all__ = ["MLP_PARENTS", "ATTENTION_PARENTS", "MLP_LEAVES", "ATTENTION_LEAVES", "UNAMBIGUOUS_MLP_LEAVES", "classify",
           "select_target_names", "apply_stacr", "set_step"]
