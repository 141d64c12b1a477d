"""Noise-floor statistics and environment records (host logic, no GPU).

Known answers are worked by hand from the definitions the reference states
(``src/bench_poly.py:59-129``): the floor is the A/A gap between the minima,
the within-variant spread only without a control pair.
"""

from __future__ import annotations

import json

import pytest

from techjam_amd.infra.environment import collect_environment, collect_git, collect_gpu_state
from techjam_amd.infra.timing import is_resolvable, summarise_timings, time_interleaved


def test_floor_is_the_gap_between_aa_minima():
    samples = {"a": [12.0, 10.0, 11.0], "a_ctl": [10.5, 11.0, 13.0], "b": [20.0, 22.0]}
    out = summarise_timings(samples, [("a", "a_ctl")])
    va = out["variants"]["a"]
    assert (va["min_ms"], va["median_ms"], va["max_ms"], va["reps"]) == (10.0, 11.0, 12.0, 3)
    assert va["spread"] == pytest.approx(0.2)
    assert out["variants"]["b"]["median_ms"] == pytest.approx(21.0)  # even count: mean of the middle two
    noise = out["noise"]
    assert noise["aa_discrepancy"] == pytest.approx(0.05)             # |10 - 10.5| / 10
    # per-repetition pairs in sample order: (12, 10.5), (10, 11), (11, 13)
    assert noise["worst_paired_aa_discrepancy"] == pytest.approx(2.0 / 11.0)
    assert noise["worst_within_variant_spread"] == pytest.approx(2.5 / 10.5)
    assert noise["minimum_detectable_effect"] == pytest.approx(1.05)


def test_without_a_control_pair_the_spread_is_the_floor():
    out = summarise_timings({"a": [4.0, 5.0], "b": [2.0, 2.2]})
    assert out["noise"]["aa_discrepancy"] is None
    assert out["noise"]["worst_paired_aa_discrepancy"] is None
    assert out["noise"]["minimum_detectable_effect"] == pytest.approx(1.25)


def test_several_control_pairs_take_the_worst():
    samples = {"a": [1.0], "a2": [1.1], "b": [2.0], "b2": [2.0]}
    out = summarise_timings(samples, [("a", "a2"), ("b", "b2")])
    assert out["noise"]["aa_discrepancy"] == pytest.approx(0.1)


def test_empty_variant_is_refused():
    with pytest.raises(ValueError):
        summarise_timings({"a": []})


def test_resolvable_in_both_directions():
    assert is_resolvable(1.10, 1.05)
    assert is_resolvable(1 / 1.10, 1.05)
    assert not is_resolvable(1.04, 1.05)
    assert not is_resolvable(0.96, 1.05)     # 1 / 0.96 = 1.0417
    assert not is_resolvable(0.0, 1.05)
    assert not is_resolvable(-2.0, 1.05)


def test_interleaved_order_and_sample_counts():
    calls = []
    variants = {"x": lambda: calls.append("x"), "y": lambda: calls.append("y")}
    samples = time_interleaved(variants, reps=3, sync=lambda: None)
    assert calls == ["x", "y"] + ["x", "y"] * 3   # one warm call each, then alternating
    assert {k: len(v) for k, v in samples.items()} == {"x": 3, "y": 3}
    assert all(t >= 0.0 for v in samples.values() for t in v)
    with pytest.raises(ValueError):
        time_interleaved(variants, reps=0, sync=lambda: None)


def test_environment_record_on_a_host_without_gpu():
    import torch

    env = collect_environment(torch, torch.device("cpu"))
    json.dumps(env)
    assert set(env) >= {"cpu", "os", "python", "pytorch", "gpu", "disk"}
    assert env["pytorch"] == torch.__version__
    assert env["gpu"]["name"] is None and env["gpu"]["hip_runtime"] == torch.version.hip
    assert collect_gpu_state(torch.device("cpu")) is None
    git = collect_git()
    assert set(git) == {"commit", "dirty", "status"}
