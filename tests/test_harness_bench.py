"""The interleaved A/B harness's arithmetic, on the CPU with an injected timer (no device)."""

from __future__ import annotations

import json

import pytest

from deltaforge_amd.harness.bench import (
    BenchConfig,
    ResultRecord,
    calibration_holds,
    median,
    outcome,
    quantile,
    run_interleaved,
)


class ScriptedTimer:
    """Returns the next scripted duration for each call, recording which column ran."""

    def __init__(self, script: dict[str, list[float]]) -> None:
        self.script = {k: list(v) for k, v in script.items()}
        self.calls: list[str] = []

    def time_ms(self, fn) -> float:
        label = fn()
        self.calls.append(label)
        return self.script[label].pop(0)


def _columns(*labels):
    return {label: (lambda label=label: label) for label in labels}


def test_quantile_matches_linear_interpolation():
    import numpy as np

    xs = [5.0, 1.0, 4.0, 2.0, 3.0, 9.5]
    for q in (0.0, 0.1, 0.25, 0.5, 0.75, 0.9, 1.0):
        assert quantile(xs, q) == pytest.approx(float(np.quantile(xs, q)))
    assert median([3.0, 1.0, 2.0]) == 2.0 and median([1.0, 2.0, 3.0, 4.0]) == 2.5
    with pytest.raises(ValueError):
        quantile([], 0.5)
    with pytest.raises(ValueError):
        quantile([1.0], 1.5)


def test_rounds_are_interleaved_and_ratios_are_per_round():
    # The candidate is 2x faster in every round while the whole box drifts 10x slower:
    # per-round ratios see 2.0 throughout; a sequential design would not.
    drift = [1.0, 2.0, 4.0, 8.0, 10.0]
    timer = ScriptedTimer({"baseline": [2.0 * d for d in drift], "candidate": [1.0 * d for d in drift],
                           "identity": [2.0 * d for d in drift]})
    cfg = BenchConfig(rounds=5, warmup_rounds=2, baseline="baseline", bytes_per_call={"candidate": 8e6})
    res = run_interleaved(_columns("baseline", "candidate", "identity"), cfg, timer)
    assert res.call_order == tuple(["baseline", "candidate", "identity"] * 5)
    assert res.ratios["candidate"] == [2.0, 2.0, 2.0]
    assert res.median_ratio["identity"] == 1.0 and res.iqr_ratio["identity"] == 0.0
    assert res.scoring_timings_ms["candidate"] == [4.0, 8.0, 10.0]
    assert res.median_ms["candidate"] == 8.0
    assert res.achieved_gbps["candidate"] == pytest.approx(8e6 / 8e-3 / 1e9)
    d = res.to_dict()
    assert d["median_ratio"]["candidate"] == 2.0 and len(d["timings_ms"]["baseline"]) == 5


def test_setups_run_untimed_before_each_call_and_warmup_calls_are_hidden():
    events = []
    cols = {"baseline": lambda: events.append("run-b") or "baseline",
            "candidate": lambda: events.append("run-c") or "candidate"}
    setups = {"candidate": lambda: events.append("setup-c")}
    timer = ScriptedTimer({"baseline": [1.0] * 2, "candidate": [1.0] * 2})
    cfg = BenchConfig(rounds=2, warmup_rounds=1, untimed_warmup_calls=1)
    run_interleaved(cols, cfg, timer, setups=setups)
    assert events == ["run-b", "setup-c", "run-c", "run-b", "setup-c", "run-c", "run-b", "setup-c", "run-c"]
    assert timer.calls == ["baseline", "candidate"] * 2


def test_configuration_errors():
    with pytest.raises(ValueError):
        BenchConfig(rounds=2, warmup_rounds=2)
    with pytest.raises(ValueError):
        run_interleaved(_columns("a", "b"), BenchConfig(baseline="zzz"), ScriptedTimer({}))
    with pytest.raises(ValueError):
        run_interleaved(_columns("baseline"), BenchConfig(), ScriptedTimer({}), setups={"nope": lambda: None})
    timer = ScriptedTimer({"baseline": [1.0] * 3, "c": [0.0] * 3})
    res = run_interleaved(_columns("baseline", "c"), BenchConfig(rounds=3, warmup_rounds=0), timer)
    with pytest.raises(ValueError):
        _ = res.ratios


def test_outcome_needs_a_margin_beyond_the_noise_band():
    assert outcome(1.05, 0.01) == "win"
    assert outcome(0.95, 0.01) == "loss"
    assert outcome(1.005, 0.01) == "inconclusive"
    assert outcome(1.5, 0.01, correct=False) == "incorrect"
    assert outcome(None, 0.0) == "error"


def test_calibration_floor():
    assert calibration_holds(1.01, 0.0)  # inside the 2 % floor
    assert not calibration_holds(1.05, 0.01)
    assert calibration_holds(1.05, 0.06)  # a noisy run admits more, and says so by its IQR
    assert not calibration_holds(None, 0.0)


def test_result_record_serialises_and_rejects_unknown_outcomes(tmp_path):
    rec = ResultRecord(kind="ab", outcome="win", config_name="config5", workload={"tokens": 64})
    path = tmp_path / "records.jsonl"
    rec.append_to(path)
    rec.append_to(path)
    lines = path.read_text().splitlines()
    assert len(lines) == 2
    d = json.loads(lines[0])
    assert d["outcome"] == "win" and d["schema_version"] == 1 and "git" in d and "environment" in d
    with pytest.raises(ValueError):
        ResultRecord(kind="ab", outcome="great", config_name="x")
    with pytest.raises(ValueError):
        ResultRecord(kind="other", outcome="win", config_name="x")


def test_phase_trace_report_attributes_time_to_phases():
    from deltaforge_amd.harness.phase_trace import layer_windows, phase_totals, decode_stamps, report

    def st(us, tag):
        return (int(round(us * 100)) << 8) | tag

    ctl = [st(0, 10)]
    t = 1.0
    for layer in range(4):
        kinds = ((1, 5), (4, 12), (6, 3), (11, 3), (7, 7), (8, 6), (11, 3)) if layer == 3 else \
            ((1, 5), (2, 4), (3, 3), (11, 3), (7, 7), (8, 6), (11, 3))
        for tag, d in kinds:
            ctl.append(st(t, tag))
            t += d
    ctl.append(st(t, 9))
    dec = decode_stamps(ctl)
    totals = {n: (tot, c) for n, tot, c in phase_totals(dec)}
    assert totals["reduce"] == (24.0, 8) and totals["attn"] == (12.0, 1) and totals["embed"] == (1.0, 1)
    layers = layer_windows(dec)
    assert [round(e - s, 2) for s, e, _ in layers] == [31.0, 31.0, 31.0, 39.0]
    assert [a for _, _, a in layers] == [False, False, False, True]
    assert "no stamps" in report({"control": [], "waves": [[]] * 8})
