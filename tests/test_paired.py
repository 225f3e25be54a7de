"""Paired A/B harness statistics (lab/paired.py) on synthetic rounds: rotation balance, ratio pairing,
bootstrap interval, A/A control and the summary table."""
import math
import statistics

from lab import paired as PA


def test_rotation_puts_every_arm_at_every_position():
    names = ["a", "b", "c", "d"]
    orders = PA.round_orders(names, 4, seed=0)
    for o in orders:
        assert sorted(o) == names
    for pos in range(4):
        assert sorted(o[pos] for o in orders) == names
    assert orders[1] == orders[0][1:] + orders[0][:1]


def test_collect_runs_each_arm_once_per_round_in_order():
    calls = []

    def arm(name, v):
        def f():
            calls.append(name)
            return {"tg_b1": v}
        return f
    arms = {"x": arm("x", 100.0), "y": arm("y", 120.0), "z": arm("z", 80.0)}
    raw = PA.collect(arms, 3, seed=5)
    assert len(calls) == 9
    for r, rec in enumerate(raw["rounds"]):
        assert calls[3 * r:3 * r + 3] == rec["order"]
    assert PA.ratios(raw["rounds"], ("y", "tg_b1"), ("x", "tg_b1")) == [1.2] * 3


def test_ratios_skip_missing_and_zero():
    R = [{"a": {"k": 2.0}, "b": {"k": 1.0}}, {"a": {}, "b": {"k": 1.0}}, {"a": {"k": 3.0}, "b": {"k": 0.0}}]
    assert PA.ratios(R, ("a", "k"), ("b", "k")) == [2.0]


def test_bootstrap_interval_brackets_the_mean_and_is_degenerate_for_constants():
    xs = [0.9, 1.1, 1.0, 1.05, 0.95, 1.02]
    lo, hi = PA.boot_ci(xs)
    assert lo <= statistics.mean(xs) <= hi
    assert min(xs) <= lo and hi <= max(xs)
    assert PA.boot_ci([2.0] * 5) == (2.0, 2.0)


def test_summary_geometric_mean_and_table():
    # per-round drift multiplies both arms alike: the ratio is exactly 1.25 every round
    R = [{"round": r, "graph": {"tg_b1": 1000.0 * (1 + 0.1 * r)}, "graph_dup": {"tg_b1": 1000.0 * (1 + 0.1 * r)},
          "mega": {"tg_b1": 1250.0 * (1 + 0.1 * r)}} for r in range(5)]
    res, table = PA.summarize({"rounds": R, "order_seed": 0}, PA.DECODE_PAIRS)
    assert set(res) == {"A/A: graph_dup / graph", "mega / graph"}      # no llama rounds: pair left out
    assert math.isclose(res["mega / graph"]["median"], 1.25)
    assert math.isclose(res["mega / graph"]["gmean"], 1.25)
    assert all(math.isclose(c, 1.25) for c in res["mega / graph"]["ci95"])
    assert math.isclose(res["A/A: graph_dup / graph"]["median"], 1.0)
    assert "| mega / graph | 1500.0 | 1200.0 | 1.2500" in table
