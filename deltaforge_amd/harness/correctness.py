"""The two correctness gates, with the reference's semantics (harness/correctness.py).

* Layer 1, per kernel: ``check_kernel`` -- allclose at rtol/atol plus the recorded max
  absolute and max relative error, the relative error taken only where ``|ref| > atol``
  (reference correctness.py:112-194).
* Layer 2, end to end: ``kl_and_agreement`` (fp32 log-softmax KL(P_ref || P_cand) and argmax
  agreement, correctness.py:383-396) aggregated by ``DistributionCheck`` with a 95% Wilson
  interval on the agreement (correctness.py:297-380).
"""

from __future__ import annotations

import math
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

__all__ = [
    "DEFAULT_ATOL",
    "DEFAULT_RTOL",
    "DistributionCheck",
    "KernelCheck",
    "check_kernel",
    "error_magnitudes",
    "kl_and_agreement",
    "wilson",
]

DEFAULT_RTOL = 1e-2
DEFAULT_ATOL = 1e-2


@dataclass(frozen=True)
class KernelCheck:
    name: str
    replaces: str
    passed: bool
    max_abs_err: float
    max_rel_err: float
    rtol: float
    atol: float
    shape: tuple[int, ...]
    dtype: str
    excluded_near_zero: int = 0
    total_elements: int = 0
    note: str = ""


def error_magnitudes(reference: torch.Tensor, candidate: torch.Tensor, atol: float = DEFAULT_ATOL):
    """``(max_abs, max_rel, excluded_near_zero, total)``; relative error only where |ref| > atol."""
    if reference.shape != candidate.shape:
        raise ValueError(f"shape mismatch: {tuple(reference.shape)} vs {tuple(candidate.shape)}")
    ref = reference.detach().float().cpu()
    cand = candidate.detach().float().cpu()
    err = (cand - ref).abs()
    total = ref.numel()
    max_abs = float(err.max()) if total else 0.0
    significant = ref.abs() > atol
    excluded = int(total - int(significant.sum()))
    max_rel = float((err[significant] / ref.abs()[significant]).max()) if bool(significant.any()) else 0.0
    return max_abs, max_rel, excluded, total


def _tensors(out) -> tuple[torch.Tensor, ...]:
    if isinstance(out, torch.Tensor):
        return (out,)
    return tuple(t for t in out if isinstance(t, torch.Tensor))


def check_kernel(name: str, reference_fn: Callable, candidate_fn: Callable, args: Sequence = (), *,
                 replaces: str = "", rtol: float = DEFAULT_RTOL, atol: float = DEFAULT_ATOL,
                 note: str = "") -> KernelCheck:
    """Run both on the same inputs and record how far apart they are (every output compared)."""
    with torch.no_grad():
        refs = _tensors(reference_fn(*args))
        cands = _tensors(candidate_fn(*args))
    if len(refs) != len(cands):
        raise ValueError(f"{name}: {len(refs)} reference outputs vs {len(cands)} candidate outputs")
    worst_abs = worst_rel = 0.0
    excluded = total = 0
    passed = True
    for r, c in zip(refs, cands):
        a, rel, exc, tot = error_magnitudes(r, c, atol)
        worst_abs, worst_rel = max(worst_abs, a), max(worst_rel, rel)
        excluded += exc
        total += tot
        passed = passed and bool(torch.allclose(c.detach().float().cpu(), r.detach().float().cpu(),
                                                rtol=rtol, atol=atol))
    return KernelCheck(name, replaces, passed, worst_abs, worst_rel, rtol, atol, tuple(refs[0].shape),
                       str(refs[0].dtype), excluded, total, note)


def kl_and_agreement(ref_logits: torch.Tensor, cand_logits: torch.Tensor):
    """Per position ``(KL(P_ref || P_cand) nats, argmax match)`` in fp32 (correctness.py:383-396)."""
    ref = torch.log_softmax(ref_logits.float(), dim=-1)
    cand = torch.log_softmax(cand_logits.float(), dim=-1)
    kl = (ref.exp() * (ref - cand)).sum(dim=-1)
    return kl.reshape(-1), (ref.argmax(dim=-1) == cand.argmax(dim=-1)).reshape(-1)


def wilson(successes: int, n: int, z: float = 1.959964) -> tuple[float, float]:
    """95% Wilson score interval (correctness.py:367-380)."""
    if n == 0:
        return (0.0, 1.0)
    p = successes / n
    denom = 1.0 + z * z / n
    centre = (p + z * z / (2 * n)) / denom
    half = z * math.sqrt(p * (1 - p) / n + z * z / (4 * n * n)) / denom
    return (max(0.0, centre - half), min(1.0, centre + half))


@dataclass(frozen=True)
class DistributionCheck:
    """Layer 2 for an approximate candidate: agreement + mean KL, gated on thresholds."""

    top1_agreement: float
    mean_kl: float
    max_kl: float
    num_positions: int
    top1_threshold: float
    kl_threshold: float

    @classmethod
    def from_logits(cls, ref_logits, cand_logits, *, top1_threshold: float, kl_threshold: float):
        kl, match = kl_and_agreement(ref_logits, cand_logits)
        return cls(float(match.float().mean()), float(kl.mean()), float(kl.max()), int(kl.numel()),
                   top1_threshold, kl_threshold)

    @property
    def top1_interval(self) -> tuple[float, float]:
        return wilson(round(self.top1_agreement * self.num_positions), self.num_positions)

    @property
    def top1_resolved(self) -> bool:
        return self.top1_threshold > self.top1_interval[1]

    @property
    def passed(self) -> bool:
        if self.mean_kl > self.kl_threshold:
            return False
        return self.top1_agreement >= self.top1_threshold or not self.top1_resolved

    def to_dict(self) -> dict:
        return {"policy": "approximate", "passed": self.passed, "top1_agreement": self.top1_agreement,
                "top1_interval": list(self.top1_interval), "mean_kl": self.mean_kl, "max_kl": self.max_kl,
                "num_positions": self.num_positions, "top1_threshold": self.top1_threshold,
                "kl_threshold": self.kl_threshold}
