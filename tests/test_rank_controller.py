"""Host policy of the adaptive engine: runtime rank control and basis-refresh triggers.

Known answers from the reference's tests/test_rank_controller.py:11-150 (same inputs, same
expected decisions), plus brute-force checks of the variance prefix rule and the clamp, and the
refresh schedule (stacr/adaptive.py:568-595,3397-3516) on hand-computed cases.
"""
import itertools
import math

import pytest

from stacr_amd.rank_controller import (
    RankDecision,
    _clamp_rank,
    choose_runtime_rank,
    choose_sensitivity_rank,
    choose_variance_rank,
    compute_refresh_offset,
    is_fixed_refresh_step,
    select_active_rank,
    should_adjust_rank,
    should_update_basis,
)


# ---------------------------------------------------------------- reference known answers
def test_should_adjust_rank_known_answers():
    assert should_adjust_rank(schedule_step=0, last_adjust_step=-1, adjust_interval=100) is True
    assert should_adjust_rank(schedule_step=50, last_adjust_step=0, adjust_interval=100) is False
    assert should_adjust_rank(schedule_step=100, last_adjust_step=0, adjust_interval=100) is True
    assert should_adjust_rank(schedule_step=3, last_adjust_step=2, adjust_interval=0) is True  # interval floor 1


def test_variance_known_answers():
    d = choose_variance_rank([9.0, 1.0, 0.2, 0.1], 4, 1, 4, 4, 0.90)
    assert (d.active_rank, d.reason_code) == (2, "variance_shrink")
    d = choose_variance_rank(None, 8, 4, 16, 16, 0.95)
    assert (d.active_rank, d.reason_code, d.changed, d.metric_value) == (8, "variance_cold_start", False, None)
    d = choose_variance_rank([1.0, 1.0, 100.0], 3, 1, 8, 2, 0.9)
    assert d.active_rank == 2 and d.reason_code in {"variance_keep", "variance_shrink", "variance_grow"}
    with pytest.raises(ValueError, match="Invalid coefficient energy"):
        choose_variance_rank([1.0, float("nan")], 2, 1, 8, 8, 0.9)


def test_sensitivity_known_answers():
    d = choose_sensitivity_rank(0.30, 8, 4, 16, 16, 0.03, 0.10, 0.25)
    assert (d.active_rank, d.reason_code) == (10, "sensitivity_grow")
    d = choose_sensitivity_rank(0.01, 8, 4, 16, 16, 0.03, 0.10, 0.25)
    assert (d.active_rank, d.reason_code) == (6, "sensitivity_shrink")


def test_runtime_dispatch_known_answers():
    d = choose_runtime_rank("variance", 8, 4, 16, 16, {"last_coeff_energy_by_rank": [10.0, 1.0, 0.1, 0.1, 0.1]},
                            variance_threshold=0.9)
    assert d.active_rank == 4 and d.reason_code.startswith("variance_")
    d = choose_runtime_rank("sensitivity", 8, 4, 16, 16, {"last_residual_energy": 0.20}, sensitivity_low=0.03,
                            sensitivity_high=0.10, step_fraction=0.25)
    assert (d.active_rank, d.reason_code) == (10, "sensitivity_grow")
    d = choose_runtime_rank("fixed", 32, 4, 16, 16, {})
    assert d.active_rank == 16 and d.changed is True and d.reason_code == "fixed"
    with pytest.raises(ValueError, match="Unsupported rank_mode"):
        choose_runtime_rank("bogus", 8, 4, 16, 16, {})


# ---------------------------------------------------------------- brute force
def test_clamp_matches_brute_force_definition():
    for rank, lo, hi, avail in itertools.product(range(-2, 12), range(-1, 6), range(-1, 9), range(-1, 8)):
        floor = max(1, lo)
        allowed = [r for r in range(floor, max(floor, hi) + 1)]  # the rank range, nearest to `rank`
        nearest = min(allowed, key=lambda r: (abs(r - rank), r))
        assert _clamp_rank(rank, lo, hi, avail) == min(max(1, avail), nearest)


def test_variance_prefix_matches_brute_force():
    grids = [[0.5, 0.25, 0.125, 0.0625], [1, 1, 1, 1, 1], [0, 3, 0, 1], [2, 0, 0, 0], [1e-3, 5, 1e-3]]
    for energies, thr in itertools.product(grids, [0.0, 0.5, 0.8, 0.95, 1.0, 1.5]):
        total = sum(max(0.0, e) for e in energies)
        t = min(1.0, max(0.0, thr))
        prefix = next(k for k in range(1, len(energies) + 1) if sum(energies[:k]) >= total * t)
        d = choose_variance_rank(energies, 2, 1, 8, 8, thr)
        assert d.active_rank == prefix
        assert math.isclose(d.metric_value, sum(energies[:prefix]) / total)
        assert d.changed == (prefix != 2)


def test_variance_edge_rules():
    d = choose_variance_rank([], 3, 1, 8, 8, 0.9)
    assert (d.active_rank, d.reason_code, d.metric_value) == (3, "variance_empty", 0.0)
    d = choose_variance_rank([0.0, -1.0], 3, 2, 8, 8, 0.9)  # negatives count as 0: all-zero energy
    assert (d.active_rank, d.reason_code, d.changed) == (2, "variance_zero_energy", True)
    with pytest.raises(ValueError):
        choose_variance_rank([float("inf")], 3, 1, 8, 8, 0.9)


def test_sensitivity_band_and_rounding():
    # step = max(1, round(current * fraction)) with Python's half-to-even round
    assert choose_sensitivity_rank(0.5, 10, 1, 64, 64, 0.03, 0.1, 0.25).active_rank == 12  # round(2.5) = 2
    assert choose_sensitivity_rank(0.5, 14, 1, 64, 64, 0.03, 0.1, 0.25).active_rank == 18  # round(3.5) = 4
    assert choose_sensitivity_rank(0.5, 4, 1, 64, 64, 0.03, 0.1, 0.001).active_rank == 5   # fraction floor 0.01
    d = choose_sensitivity_rank(0.05, 8, 4, 16, 16, 0.10, 0.03, 0.25)  # swapped thresholds
    assert (d.active_rank, d.reason_code) == (8, "sensitivity_keep_band")
    d = choose_sensitivity_rank(0.5, 16, 4, 16, 16, 0.03, 0.1, 0.25)
    assert (d.active_rank, d.reason_code, d.changed) == (16, "sensitivity_keep_high", False)
    d = choose_sensitivity_rank(0.0, 4, 4, 16, 16, 0.03, 0.1, 0.25)
    assert (d.active_rank, d.reason_code) == (4, "sensitivity_keep_low")
    assert isinstance(d, RankDecision) and d.metric_value == 0.0


def test_select_active_rank_records_trajectory():
    cfg = {"rank_mode": "sensitivity", "rank_min": 2, "rank_max": 16, "rank_adjust_interval": 10}
    state = {"last_residual_energy": 0.5}
    assert select_active_rank(cfg, state, 0, 8) == 8  # current 8 + round(8 * 0.125) = 9 > allocated 8
    assert state["last_rank_reason"] == "sensitivity_keep_high"
    state["last_residual_energy"] = 0.0
    state["active_rank"] = 8
    assert select_active_rank(cfg, state, 5, 8) == 8  # inside the adjust interval: unchanged
    assert select_active_rank(cfg, state, 10, 8) == 7
    assert state["rank_reason_code_counts"] == {"sensitivity_keep_high": 1, "sensitivity_shrink": 1}
    assert [t["active_rank"] for t in state["rank_trajectory"]] == [8, 7]
    for s in range(20, 20 + 10 * 200, 10):
        select_active_rank(cfg, state, s, 8)
    assert len(state["rank_trajectory"]) == 128
    assert select_active_rank({"rank_mode": "fixed"}, {}, 3, 8) == 8
    with pytest.raises(RuntimeError):
        select_active_rank(cfg, {}, 0, 8, use_basis_sharing=True)


# ---------------------------------------------------------------- refresh triggers
def test_refresh_offsets_spread_layers_over_the_period():
    assert compute_refresh_offset(None, 12, 1000) == 0
    assert [compute_refresh_offset(i, 4, 100) for i in range(5)] == [0, 25, 50, 75, 0]
    assert [compute_refresh_offset(i, 3, 10) for i in range(3)] == [0, 3, 6]
    assert not is_fixed_refresh_step(105, 100, 10)        # first refresh a full period after warmup
    assert is_fixed_refresh_step(110, 100, 10)
    assert is_fixed_refresh_step(113, 100, 10, layer_index=1, num_layers=3)
    assert not is_fixed_refresh_step(110, 100, 10, layer_index=1, num_layers=3)


def test_should_update_basis_schedules():
    base = {"freeze_basis_after_warmup": False, "lazy_update_enabled": False}
    st = {"last_residual_energy": 0.0}
    fixed = dict(base, update_trigger="fixed", update_interval=5)
    assert [s for s in range(12) if should_update_basis(fixed, st, s)] == [5, 10]
    assert st["_pending_update_reason"] == "fixed" and st["_last_update_schedule_step"] == 10
    adaptive = dict(base, update_trigger="adaptive", energy_threshold=0.05)
    assert not should_update_basis(adaptive, {"last_residual_energy": 0.05}, 3)
    st = {"last_residual_energy": 0.06}
    assert should_update_basis(adaptive, st, 3) and st["_pending_update_reason"] == "adaptive"
    hybrid = dict(base, update_trigger="hybrid", update_interval=4, energy_threshold=0.05)
    st = {"last_residual_energy": 0.5}
    assert should_update_basis(hybrid, st, 8) and st["_pending_update_reason"] == "hybrid_both"
    st = {"last_residual_energy": 0.0}
    assert should_update_basis(hybrid, st, 8) and st["_pending_update_reason"] == "fixed"
    # lazy skip before the trigger; grad-accumulation cache on later microbatches
    st = {"last_residual_energy": 0.001}
    assert not should_update_basis({"freeze_basis_after_warmup": False}, st, 100)
    assert st["last_skip_reason"] == "lazy_update_skip" and st["skipped_updates"] == 1
    st = {"last_residual_energy": 0.5}
    cached = dict(base, update_trigger="adaptive", cache_basis_per_optimizer_step=True)
    assert not should_update_basis(cached, st, 7, microbatch_index=1, accum_steps=4)
    assert st["microbatch_cache_hits"] == 1 and st["last_skip_reason"] == "cache_hit"
    assert should_update_basis(cached, st, 7, microbatch_index=0, accum_steps=4)


def test_should_update_basis_after_warmup_freeze():
    st = {"last_residual_energy": 0.5}
    frozen = {"warmup_steps": 10}  # defaults: frozen after warmup, refresh off
    assert not should_update_basis(frozen, st, 10)
    assert st["frozen_updates"] == 1 and st["last_skip_reason"] == "frozen_after_warmup"
    refresh = {"warmup_steps": 10, "refresh_trigger": "hybrid", "refresh_period": 5,
               "refresh_energy_threshold": 0.1}
    st = {"last_residual_energy": 0.0}
    assert [s for s in range(10, 26) if should_update_basis(refresh, st, s)] == [15, 20, 25]
    assert st["_pending_update_reason"] == "refresh_fixed"
    st = {"last_residual_energy": 0.2}
    assert should_update_basis(refresh, st, 12) and st["_pending_update_reason"] == "refresh_residual_energy"
    assert should_update_basis(refresh, st, 15) and st["_pending_update_reason"] == "refresh_hybrid_both"
    energy_only = dict(refresh, refresh_trigger="residual_energy")
    assert not should_update_basis(energy_only, {"last_residual_energy": 0.1}, 15)
