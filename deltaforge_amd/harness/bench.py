"""Interleaved A/B timing of opaque callables, with an identity calibration column.

The semantics are the reference's harness (reference src/deltaforge/harness/bench.py:
150-343 ``BenchResult`` / ``run_interleaved``; src/deltaforge/batch.py:560-591 outcome and
``calibration_holds``; harness/report.py:211 ``ResultRecord``):

* every column runs once per round, in a fixed order, so drift that affects a whole round
  (clocks, thermals, a neighbour on the box) divides out of that round's ratios;
* the first ``warmup_rounds`` rounds are discarded; the score of a column is the median over
  the scoring rounds of ``t_baseline / t_column`` taken within each round, and its noise band
  is the interquartile range of those ratios;
* a setup callable per column runs before each timed call and outside the timed region;
* a column that computes the baseline's own work (the identity) must score 1.00 within the
  noise band (floor 2 %), or the run measured something other than the kernels.

Timing uses HIP events on the current stream with a device synchronisation on both sides
(``HipEventTimer``); ``WallClockTimer`` is for host-only runs. Nothing here knows what the
columns compute, so the arithmetic is tested on the CPU with an injected timer.
"""

from __future__ import annotations

import json
import os
import platform
import subprocess
import time
from collections.abc import Callable, Mapping, Sequence
from dataclasses import dataclass, field
from typing import Any, Protocol

__all__ = [
    "BenchConfig",
    "BenchResult",
    "HipEventTimer",
    "ResultRecord",
    "Timer",
    "WallClockTimer",
    "calibration_holds",
    "median",
    "outcome",
    "quantile",
    "run_interleaved",
]

OUTCOMES = ("win", "loss", "inconclusive", "incorrect", "error", "baseline")


class Timer(Protocol):
    def time_ms(self, fn: Callable[[], object]) -> float: ...


class HipEventTimer:
    """Milliseconds between two HIP events recorded on the current stream around ``fn``;
    the device is synchronised first (so earlier work is not counted) and after (so the end
    event has completed)."""

    def __init__(self, device: object | None = None) -> None:
        self.device = device

    def time_ms(self, fn: Callable[[], object]) -> float:
        import torch

        torch.cuda.synchronize(self.device)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        ev[0].record()
        fn()
        ev[1].record()
        torch.cuda.synchronize(self.device)
        return float(ev[0].elapsed_time(ev[1]))


class WallClockTimer:
    """``time.perf_counter`` around ``fn``, for runs with no device."""

    def time_ms(self, fn: Callable[[], object]) -> float:
        t0 = time.perf_counter()
        fn()
        return (time.perf_counter() - t0) * 1e3


def median(values: Sequence[float]) -> float:
    return quantile(values, 0.5)


def quantile(values: Sequence[float], q: float) -> float:
    """Linear interpolation between the order statistics at ``q * (n - 1)`` (numpy's default
    method), written out so the score does not depend on a library's convention."""
    if not values:
        raise ValueError("quantile of no values")
    if not 0.0 <= q <= 1.0:
        raise ValueError(f"q must lie in [0, 1], got {q}")
    xs = sorted(float(v) for v in values)
    at = q * (len(xs) - 1)
    lo = int(at)
    hi = min(lo + 1, len(xs) - 1)
    return xs[lo] + (xs[hi] - xs[lo]) * (at - lo)


@dataclass(frozen=True)
class BenchConfig:
    """``rounds`` timed rounds of which the first ``warmup_rounds`` are discarded;
    ``untimed_warmup_calls`` extra calls per column before round 0; ``bytes_per_call``
    (algorithmic bytes one call of a column moves) turns medians into GB/s."""

    rounds: int = 7
    warmup_rounds: int = 2
    baseline: str = "baseline"
    untimed_warmup_calls: int = 0
    bytes_per_call: dict[str, float] = field(default_factory=dict)

    def __post_init__(self) -> None:
        if self.warmup_rounds < 0 or self.untimed_warmup_calls < 0:
            raise ValueError("warmup counts cannot be negative")
        if self.rounds - self.warmup_rounds < 1:
            raise ValueError(f"{self.rounds} rounds with {self.warmup_rounds} discarded leaves none to score")


@dataclass(frozen=True)
class BenchResult:
    """The per-round timings of every column (warmup rounds included) and the order in which
    the calls were made, from which every score is derived."""

    labels: tuple[str, ...]
    config: BenchConfig
    rounds_ms: tuple[dict[str, float], ...]  # one {label: ms} per round, in round order
    call_order: tuple[str, ...]
    metadata: dict[str, Any] = field(default_factory=dict)

    def _scored(self) -> tuple[dict[str, float], ...]:
        return self.rounds_ms[self.config.warmup_rounds:]

    @property
    def timings_ms(self) -> dict[str, list[float]]:
        return {label: [r[label] for r in self.rounds_ms] for label in self.labels}

    @property
    def scoring_timings_ms(self) -> dict[str, list[float]]:
        return {label: [r[label] for r in self._scored()] for label in self.labels}

    @property
    def ratios(self) -> dict[str, list[float]]:
        """Per scoring round, ``t_baseline / t_label`` (above 1: the column is faster)."""
        base = self.config.baseline
        out: dict[str, list[float]] = {}
        for label in self.labels:
            if label == base:
                continue
            per_round = []
            for i, r in enumerate(self._scored()):
                if r[label] <= 0.0:
                    raise ValueError(f"{label!r} timed {r[label]} ms in scoring round {i}: no ratio")
                per_round.append(r[base] / r[label])
            out[label] = per_round
        return out

    @property
    def median_ratio(self) -> dict[str, float]:
        return {label: median(v) for label, v in self.ratios.items()}

    @property
    def iqr_ratio(self) -> dict[str, float]:
        return {label: quantile(v, 0.75) - quantile(v, 0.25) for label, v in self.ratios.items()}

    @property
    def median_ms(self) -> dict[str, float]:
        return {label: median(v) for label, v in self.scoring_timings_ms.items()}

    @property
    def achieved_gbps(self) -> dict[str, float]:
        """Algorithmic bytes per call / median call time, for the columns that declared bytes."""
        med = self.median_ms
        return {label: b / (med[label] * 1e-3) / 1e9 for label, b in self.config.bytes_per_call.items()
                if label in med and med[label] > 0}

    def to_dict(self) -> dict[str, Any]:
        return {
            "labels": list(self.labels),
            "baseline": self.config.baseline,
            "rounds": self.config.rounds,
            "warmup_rounds": self.config.warmup_rounds,
            "timings_ms": self.timings_ms,
            "median_ms": self.median_ms,
            "ratios": self.ratios,
            "median_ratio": self.median_ratio,
            "iqr_ratio": self.iqr_ratio,
            "achieved_gbps": self.achieved_gbps,
            "call_order": list(self.call_order),
            "metadata": dict(self.metadata),
        }


def run_interleaved(
    columns: Mapping[str, Callable[[], object]],
    config: BenchConfig | None = None,
    timer: Timer | None = None,
    *,
    setups: Mapping[str, Callable[[], object]] | None = None,
    metadata: Mapping[str, Any] | None = None,
    progress: Callable[[int, str, float], None] | None = None,
) -> BenchResult:
    """Time each column once per round, in ``columns``' order, for ``config.rounds`` rounds."""
    config = config or BenchConfig()
    labels = tuple(columns)
    if not labels:
        raise ValueError("nothing to time")
    if config.baseline not in columns:
        raise ValueError(f"the baseline {config.baseline!r} is not a column ({list(labels)})")
    setups = dict(setups or {})
    for name, what in ((sorted(set(setups) - set(labels)), "setups"),
                       (sorted(set(config.bytes_per_call) - set(labels)), "bytes_per_call")):
        if name:
            raise ValueError(f"{what} name columns that do not exist: {name}")
    timer = timer or HipEventTimer()
    no_setup = lambda: None  # noqa: E731

    try:
        import torch

        grad_off = torch.no_grad()
    except ModuleNotFoundError:  # host-only use of the arithmetic
        from contextlib import nullcontext

        grad_off = nullcontext()

    rounds: list[dict[str, float]] = []
    order: list[str] = []
    with grad_off:
        for label in labels:
            for _ in range(config.untimed_warmup_calls):
                setups.get(label, no_setup)()
                columns[label]()
        for i in range(config.rounds):
            this_round: dict[str, float] = {}
            for label in labels:
                setups.get(label, no_setup)()
                order.append(label)
                this_round[label] = timer.time_ms(columns[label])
                if progress is not None:
                    progress(i, label, this_round[label])
            rounds.append(this_round)
    return BenchResult(labels, config, tuple(rounds), tuple(order), dict(metadata or {}))


def outcome(median_ratio: float | None, iqr: float, *, correct: bool = True) -> str:
    """``win`` / ``loss`` only when the ratio's distance from 1 exceeds the noise band
    (the ratios' IQR); otherwise ``inconclusive`` (reference batch.py:548-573)."""
    if not correct:
        return "incorrect"
    if median_ratio is None:
        return "error"
    if median_ratio - 1.0 > iqr:
        return "win"
    if 1.0 - median_ratio > iqr:
        return "loss"
    return "inconclusive"


def calibration_holds(median_ratio: float | None, iqr: float, *, floor: float = 0.02) -> bool:
    """The identity column scored 1.00 within max(IQR, floor) (reference batch.py:575-591);
    if not, no ratio of the same run means what it says."""
    return median_ratio is not None and abs(median_ratio - 1.0) <= max(iqr, floor)


def _git() -> dict[str, Any]:
    root = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    try:
        head = subprocess.run(["git", "rev-parse", "HEAD"], cwd=root, capture_output=True, text=True,
                              timeout=10).stdout.strip()
        dirty = bool(subprocess.run(["git", "status", "--porcelain"], cwd=root, capture_output=True, text=True,
                                    timeout=10).stdout.strip())
        return {"head": head or None, "dirty": dirty}
    except (OSError, subprocess.SubprocessError):
        return {"head": None, "dirty": None}


def _environment() -> dict[str, Any]:
    env: dict[str, Any] = {"host": platform.node(), "python": platform.python_version(), "cpus": os.cpu_count()}
    try:
        import torch

        env["torch"] = torch.__version__
        env["hip"] = getattr(torch.version, "hip", None)
        if torch.cuda.is_available():
            env["device"] = torch.cuda.get_device_name(0)
    except ModuleNotFoundError:
        pass
    return env


@dataclass
class ResultRecord:
    """One A/B run, whatever its outcome, as a JSON line: what ran (``workload``), the
    interleaved timings (``bench``, a ``BenchResult.to_dict()``), the correctness evidence,
    the calibration verdict, and where it ran (``environment``, ``git``)."""

    kind: str  # "baseline" (a measurement) or "ab" (a comparison)
    outcome: str
    config_name: str
    workload: dict[str, Any] = field(default_factory=dict)
    bench: dict[str, Any] | None = None
    correctness: dict[str, Any] | None = None
    calibration: dict[str, Any] | None = None
    environment: dict[str, Any] = field(default_factory=dict)
    git: dict[str, Any] = field(default_factory=dict)
    notes: str = ""
    timestamp: str = ""
    schema_version: int = 1

    def __post_init__(self) -> None:
        if self.outcome not in OUTCOMES:
            raise ValueError(f"outcome {self.outcome!r} is not one of {OUTCOMES}")
        if self.kind not in ("baseline", "ab"):
            raise ValueError(f"kind must be 'baseline' or 'ab', got {self.kind!r}")
        if not self.timestamp:
            self.timestamp = time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime())
        if not self.environment:
            self.environment = _environment()
        if not self.git:
            self.git = _git()

    def to_dict(self) -> dict[str, Any]:
        return {k: getattr(self, k) for k in ("schema_version", "kind", "outcome", "timestamp", "config_name",
                                              "workload", "bench", "correctness", "calibration", "environment",
                                              "git", "notes")}

    def append_to(self, path: str | os.PathLike) -> None:
        with open(path, "a", encoding="utf-8") as fh:
            fh.write(json.dumps(self.to_dict(), sort_keys=True) + "\n")
