"""Runtime rank control and basis-refresh triggers of the adaptive engine (host policy).

Same names, arguments, reason codes and errors as stacr/rank_controller.py:15-210, the refresh
schedule helpers stacr/adaptive.py:561-595, and the two per-layer decisions the adaptive layer
makes each forward: the active prefix rank (stacr/adaptive.py:3041-3095) and whether to update
the basis (stacr/adaptive.py:3397-3516).  The inputs are the energies the HIP save kernel
reports (layer_state["last_residual_energy"], layer_state["last_coeff_energy_by_rank"]); the
decisions are plain Python on scalars and run on the host.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from enum import Enum
from typing import Any, Iterable, Mapping, MutableMapping, Optional

TRAJECTORY_LIMIT = 128  # rank_trajectory entries kept per layer (stacr/adaptive.py:3093)


@dataclass(frozen=True)
class RankDecision:
    active_rank: int
    reason_code: str
    changed: bool
    metric_value: Optional[float] = None


def _clamp_rank(rank: int, rank_min: int, rank_max: int, max_available_rank: int) -> int:
    """rank limited to [max(1, rank_min), max(floor, rank_max)], then to the allocated rank."""
    floor = max(1, int(rank_min))
    ceiling = max(floor, int(rank_max))
    return min(max(1, int(max_available_rank)), max(floor, min(int(rank), ceiling)))


def should_adjust_rank(schedule_step: int, last_adjust_step: int, adjust_interval: int) -> bool:
    """True on the first call (last_adjust_step < 0) and then every adjust_interval steps."""
    if last_adjust_step < 0:
        return True
    return int(schedule_step) - int(last_adjust_step) >= max(1, int(adjust_interval))


def _keep_grow_shrink(prefix: str, target: int, current: int) -> str:
    if target == current:
        return prefix + "_keep"
    return prefix + ("_grow" if target > current else "_shrink")


def choose_variance_rank(coeff_energy_by_rank: Optional[Iterable[float]], current_rank: int, rank_min: int,
                         rank_max: int, max_available_rank: int, variance_threshold: float) -> RankDecision:
    """Smallest prefix of the per-rank coefficient energies holding ``variance_threshold`` of their sum."""
    current = _clamp_rank(current_rank, rank_min, rank_max, max_available_rank)
    if coeff_energy_by_rank is None:
        return RankDecision(current, "variance_cold_start", False, None)
    energies = []
    for raw in coeff_energy_by_rank:
        e = float(raw)
        if not math.isfinite(e):
            raise ValueError(f"Invalid coefficient energy: {raw!r}")
        energies.append(e if e > 0.0 else 0.0)
    if not energies:
        return RankDecision(current, "variance_empty", False, 0.0)
    energies = energies[:max_available_rank]
    total = float(sum(energies))
    if total <= 0.0:
        target = _clamp_rank(rank_min, rank_min, rank_max, max_available_rank)
        return RankDecision(target, "variance_zero_energy", target != current, 0.0)
    goal = total * min(1.0, max(0.0, float(variance_threshold)))
    captured, prefix = 0.0, 1
    for prefix, e in enumerate(energies, start=1):
        captured += e
        if captured >= goal:
            break
    target = _clamp_rank(prefix, rank_min, rank_max, max_available_rank)
    return RankDecision(target, _keep_grow_shrink("variance", target, current), target != current,
                        captured / total)


def choose_sensitivity_rank(residual_energy: float, current_rank: int, rank_min: int, rank_max: int,
                            max_available_rank: int, low_threshold: float, high_threshold: float,
                            step_fraction: float) -> RankDecision:
    """Step the rank up at or above the high band, down at or below the low band, else keep."""
    current = _clamp_rank(current_rank, rank_min, rank_max, max_available_rank)
    low, high = sorted((float(low_threshold), float(high_threshold)))
    energy = float(residual_energy)
    step = max(1, int(round(current * max(0.01, float(step_fraction)))))
    if energy >= high:
        target = _clamp_rank(current + step, rank_min, rank_max, max_available_rank)
        return RankDecision(target, "sensitivity_grow" if target != current else "sensitivity_keep_high",
                            target != current, energy)
    if energy <= low:
        target = _clamp_rank(current - step, rank_min, rank_max, max_available_rank)
        return RankDecision(target, "sensitivity_shrink" if target != current else "sensitivity_keep_low",
                            target != current, energy)
    return RankDecision(current, "sensitivity_keep_band", False, energy)


def choose_runtime_rank(rank_mode: str, current_rank: int, rank_min: int, rank_max: int, max_available_rank: int,
                        layer_state: Mapping[str, object], variance_threshold: float = 0.95,
                        sensitivity_low: float = 0.03, sensitivity_high: float = 0.10,
                        step_fraction: float = 0.125) -> RankDecision:
    """Dispatch on rank_mode: "fixed", "variance" or "sensitivity"."""
    if rank_mode == "fixed":
        target = _clamp_rank(current_rank, rank_min, rank_max, max_available_rank)
        return RankDecision(target, "fixed", target != current_rank, None)
    if rank_mode == "variance":
        return choose_variance_rank(layer_state.get("last_coeff_energy_by_rank"), current_rank, rank_min, rank_max,
                                    max_available_rank, variance_threshold)
    if rank_mode == "sensitivity":
        return choose_sensitivity_rank(float(layer_state.get("last_residual_energy", 0.0)), current_rank, rank_min,
                                       rank_max, max_available_rank, sensitivity_low, sensitivity_high,
                                       step_fraction)
    raise ValueError(f"Unsupported rank_mode: {rank_mode}")


# ---------------------------------------------------------------- per-layer decisions
RANK_DEFAULTS = {"rank_mode": "fixed", "rank_variance_threshold": 0.95, "rank_min": 4, "rank_max": 64,
                 "rank_adjust_interval": 100, "rank_sensitivity_low": 0.03, "rank_sensitivity_high": 0.10,
                 "rank_step_fraction": 0.125}
REFRESH_DEFAULTS = {"update_trigger": "hybrid", "update_interval": 100, "energy_threshold": 0.05,
                    "warmup_steps": 0, "freeze_basis_after_warmup": True, "lazy_update_enabled": True,
                    "lazy_update_threshold": 0.01, "refresh_trigger": "off", "refresh_period": 1000,
                    "refresh_energy_threshold": 0.1, "cache_basis_per_optimizer_step": False}


def _cfg(config: Mapping[str, Any], key: str, defaults: Mapping[str, Any]):
    return config.get(key, defaults[key])


def select_active_rank(config: Mapping[str, Any], layer_state: MutableMapping[str, Any], schedule_step: int,
                       allocated_rank: int, use_basis_sharing: bool = False) -> int:
    """The active prefix rank for this forward (stacr/adaptive.py:3041-3095); records the decision
    (last_rank_reason, rank_reason_code_counts, rank_trajectory) in layer_state."""
    allocated = max(1, int(allocated_rank))
    mode = _cfg(config, "rank_mode", RANK_DEFAULTS)
    if use_basis_sharing and mode != "fixed":
        raise RuntimeError("Adaptive runtime rank is incompatible with basis sharing.")
    rank_min = _cfg(config, "rank_min", RANK_DEFAULTS)
    current = max(rank_min, min(int(layer_state.get("active_rank", allocated)), allocated))
    if mode == "fixed":
        layer_state["last_rank_reason"] = "fixed"
        return allocated
    if not should_adjust_rank(schedule_step, int(layer_state.get("_last_rank_adjust_step", -1)),
                              _cfg(config, "rank_adjust_interval", RANK_DEFAULTS)):
        return current
    decision = choose_runtime_rank(mode, current, rank_min, _cfg(config, "rank_max", RANK_DEFAULTS), allocated,
                                   layer_state,
                                   variance_threshold=_cfg(config, "rank_variance_threshold", RANK_DEFAULTS),
                                   sensitivity_low=_cfg(config, "rank_sensitivity_low", RANK_DEFAULTS),
                                   sensitivity_high=_cfg(config, "rank_sensitivity_high", RANK_DEFAULTS),
                                   step_fraction=_cfg(config, "rank_step_fraction", RANK_DEFAULTS))
    target = max(1, min(int(decision.active_rank), allocated))
    layer_state["_last_rank_adjust_step"] = int(schedule_step)
    layer_state["last_rank_reason"] = decision.reason_code
    counts = layer_state.setdefault("rank_reason_code_counts", {})
    counts[decision.reason_code] = int(counts.get(decision.reason_code, 0)) + 1
    trajectory = layer_state.setdefault("rank_trajectory", [])
    trajectory.append({"step": int(schedule_step), "active_rank": int(target), "reason_code": decision.reason_code,
                       "metric_value": None if decision.metric_value is None else float(decision.metric_value)})
    if len(trajectory) > TRAJECTORY_LIMIT:
        del trajectory[:-TRAJECTORY_LIMIT]
    return target


class BasisRefreshTrigger(Enum):
    """When a basis frozen after warmup is refreshed (stacr/adaptive.py:561-566)."""

    OFF = "off"
    FIXED = "fixed"
    RESIDUAL_ENERGY = "residual_energy"
    HYBRID = "hybrid"


def compute_refresh_offset(layer_index: Optional[int], num_layers: int, refresh_period: int) -> int:
    """Layer i of L refreshes at offset floor(i * period / L) within each period (0 without an index)."""
    if layer_index is None:
        return 0
    layers = max(1, int(num_layers))
    period = max(1, int(refresh_period))
    return int(((int(layer_index) % layers) * period) / layers) % period


def is_fixed_refresh_step(schedule_step: int, warmup_steps: int, refresh_period: int,
                          layer_index: Optional[int] = None, num_layers: int = 1) -> bool:
    """True on this layer's fixed-cadence refresh steps, the first one a full period after warmup."""
    since = max(0, int(schedule_step) - int(warmup_steps))
    period = max(1, int(refresh_period))
    return since >= period and since % period == compute_refresh_offset(layer_index, num_layers, period)


def _microbatch_cached(layer_state: MutableMapping[str, Any], cache: bool, microbatch_index: int) -> bool:
    if cache and microbatch_index > 0:
        layer_state["microbatch_cache_hits"] = layer_state.get("microbatch_cache_hits", 0) + 1
        layer_state["last_skip_reason"] = "cache_hit"
        return True
    return False


def basis_update_outlook(config: Mapping[str, Any], schedule_step: int, microbatch_index: int = 0,
                         accum_steps: int = 1, layer_index: Optional[int] = None, num_layers: int = 1) -> str:
    """What should_update_basis can decide after this step's forward, known before it: "never",
    "certain" (a cadence fires whatever the forward's energy) or "maybe" (it depends on the energy).
    Reads and writes no layer state."""
    step = int(schedule_step)
    cache = bool(_cfg(config, "cache_basis_per_optimizer_step", REFRESH_DEFAULTS) and accum_steps > 1)
    if cache and microbatch_index > 0:
        return "never"
    warmup = _cfg(config, "warmup_steps", REFRESH_DEFAULTS)
    if _cfg(config, "freeze_basis_after_warmup", REFRESH_DEFAULTS) and step >= warmup:
        trigger = _cfg(config, "refresh_trigger", REFRESH_DEFAULTS)
        fixed = is_fixed_refresh_step(step, warmup, max(1, int(_cfg(config, "refresh_period", REFRESH_DEFAULTS))),
                                      layer_index, num_layers)
        if trigger in (BasisRefreshTrigger.FIXED.value, BasisRefreshTrigger.HYBRID.value) and fixed:
            return "certain"
        if trigger in (BasisRefreshTrigger.RESIDUAL_ENERGY.value, BasisRefreshTrigger.HYBRID.value):
            return "maybe"
        return "never"
    lazy = bool(_cfg(config, "lazy_update_enabled", REFRESH_DEFAULTS))
    trigger = _cfg(config, "update_trigger", REFRESH_DEFAULTS)
    interval = _cfg(config, "update_interval", REFRESH_DEFAULTS)
    on_interval = step > 0 and step % interval == 0
    if trigger in ("fixed", "hybrid") and on_interval:
        return "maybe" if lazy else "certain"
    if trigger in ("adaptive", "hybrid"):
        return "maybe"
    return "never"


def should_update_basis(config: Mapping[str, Any], layer_state: MutableMapping[str, Any], schedule_step: int,
                        microbatch_index: int = 0, accum_steps: int = 1, layer_index: Optional[int] = None,
                        num_layers: int = 1) -> bool:
    """Whether this forward updates the basis (stacr/adaptive.py:3397-3516).

    Reads layer_state["last_residual_energy"]; records skips (frozen_updates, skipped_updates,
    microbatch_cache_hits, last_skip_reason), _last_update_schedule_step and the pending update
    reason (_pending_update_reason) as the reference does.
    """
    step = int(schedule_step)
    energy = layer_state["last_residual_energy"]
    cache = bool(_cfg(config, "cache_basis_per_optimizer_step", REFRESH_DEFAULTS) and accum_steps > 1)
    warmup = _cfg(config, "warmup_steps", REFRESH_DEFAULTS)

    def fire(reason: str) -> bool:
        if _microbatch_cached(layer_state, cache, microbatch_index):
            return False
        layer_state["_last_update_schedule_step"] = step
        layer_state["_pending_update_reason"] = reason
        return True

    if _cfg(config, "freeze_basis_after_warmup", REFRESH_DEFAULTS) and step >= warmup:
        trigger = _cfg(config, "refresh_trigger", REFRESH_DEFAULTS)
        fixed = is_fixed_refresh_step(step, warmup, max(1, int(_cfg(config, "refresh_period", REFRESH_DEFAULTS))),
                                      layer_index, num_layers)
        rises = energy > float(_cfg(config, "refresh_energy_threshold", REFRESH_DEFAULTS))
        reason = None
        if trigger == BasisRefreshTrigger.FIXED.value and fixed:
            reason = "fixed"
        elif trigger == BasisRefreshTrigger.RESIDUAL_ENERGY.value and rises:
            reason = "residual_energy"
        elif trigger == BasisRefreshTrigger.HYBRID.value and (fixed or rises):
            reason = "hybrid_both" if fixed and rises else ("fixed" if fixed else "residual_energy")
        if reason is not None:
            return fire(f"refresh_{reason}")
        layer_state["frozen_updates"] = layer_state.get("frozen_updates", 0) + 1
        layer_state["last_skip_reason"] = "frozen_after_warmup"
        return False

    if _cfg(config, "lazy_update_enabled", REFRESH_DEFAULTS) and \
            energy < _cfg(config, "lazy_update_threshold", REFRESH_DEFAULTS):
        layer_state["skipped_updates"] = layer_state.get("skipped_updates", 0) + 1
        layer_state["last_skip_reason"] = "lazy_update_skip"
        return False

    trigger = _cfg(config, "update_trigger", REFRESH_DEFAULTS)
    interval = _cfg(config, "update_interval", REFRESH_DEFAULTS)
    on_interval = step > 0 and step % interval == 0
    above = energy > _cfg(config, "energy_threshold", REFRESH_DEFAULTS)
    if trigger == "fixed":
        return fire("fixed") if on_interval else False
    if trigger == "adaptive":
        return fire("adaptive") if above else False
    if trigger == "hybrid":
        if not (on_interval or above):
            return False
        return fire("hybrid_both" if on_interval and above else ("fixed" if on_interval else "adaptive"))
    return False
