"""The kernel registry: ``name -> (impl, replaces, status)``, for the decode hot path.

Same surface and invariants as the reference's registry (reference
src/deltaforge/kernels/__init__.py:18-256): the ten replaceable operation names, at most one
CHAMPION per operation, ``promote`` that retires the incumbent in the same step, check
builders keyed by kernel name. The entries registered here are the gfx950 HIP kernels of
``deltaforge_amd`` (``hip_ops``), each the champion of the operation it replaces.
"""

from __future__ import annotations

from collections.abc import Callable, Iterator
from dataclasses import dataclass, replace
from enum import Enum

__all__ = [
    "CHECK_BUILDERS",
    "REGISTRY",
    "REPLACEABLE_OPS",
    "KernelEntry",
    "KernelRegistry",
    "KernelStatus",
    "RegistryError",
    "build_kernel_checks",
    "register_checks",
]


class KernelStatus(str, Enum):
    """``CANDIDATE`` correct but not assembled; ``CHAMPION`` the one implementation assembled
    for its operation; ``RETIRED`` kept registered so the dead end stays recorded."""

    CANDIDATE = "candidate"
    CHAMPION = "champion"
    RETIRED = "retired"


#: The reference operations a kernel may replace (reference kernels/__init__.py:56-80).
REPLACEABLE_OPS = frozenset(
    {
        "rms_norm",
        "rms_norm_residual",
        "swiglu_mlp",
        "qkv_projection_rope",
        "gated_delta_rule",
        "gqa_attention",
        "kv_cache_update",
        "decode_step",
        "causal_conv",
        "decode_cache",
    }
)


class RegistryError(RuntimeError):
    """A registration or lookup that would break the registry's rules."""


@dataclass(frozen=True)
class KernelEntry:
    name: str
    impl: Callable[..., object]
    replaces: str
    status: KernelStatus
    hypothesis: str | None = None
    notes: str = ""


class KernelRegistry:
    """Kernels by name, plus an index ``operation -> champion name``.

    The index is the only place a champion is recorded, so "at most one champion per
    operation" holds by construction: every status change goes through ``_set_status``,
    which keeps the entry and the index in step. ``check_invariants`` re-derives the index
    from the entries and compares, which catches an entry edited behind the registry's back.
    """

    def __init__(self, replaceable_ops: frozenset[str] = REPLACEABLE_OPS) -> None:
        self._replaceable_ops = frozenset(replaceable_ops)
        self._entries: dict[str, KernelEntry] = {}
        self._champion_of: dict[str, str] = {}  # operation -> name of its champion

    # -- mutation ------------------------------------------------------------------------

    def _set_status(self, entry: KernelEntry, status: KernelStatus) -> KernelEntry:
        op = entry.replaces
        if self._champion_of.get(op) == entry.name and status is not KernelStatus.CHAMPION:
            del self._champion_of[op]
        if status is KernelStatus.CHAMPION:
            self._champion_of[op] = entry.name
        updated = entry if entry.status is status else replace(entry, status=status)
        self._entries[entry.name] = updated
        return updated

    def register(
        self,
        name: str,
        impl: Callable[..., object],
        *,
        replaces: str,
        status: KernelStatus | str = KernelStatus.CANDIDATE,
        hypothesis: str | None = None,
        notes: str = "",
    ) -> KernelEntry:
        """Add a kernel. A new champion may only take an operation that has none; use
        ``promote`` to replace a sitting champion."""
        if name in self._entries:
            raise RegistryError(f"{name!r} is registered already; unregister it first to replace it")
        if replaces not in self._replaceable_ops:
            known = ", ".join(sorted(self._replaceable_ops))
            raise RegistryError(f"{name!r}: {replaces!r} is not a replaceable operation (one of: {known})")
        status = KernelStatus(status)
        sitting = self._champion_of.get(replaces)
        if status is KernelStatus.CHAMPION and sitting is not None:
            raise RegistryError(
                f"{replaces!r} already has the champion {sitting!r}; register {name!r} as a candidate "
                "and promote() it, which retires the sitting champion in the same step"
            )
        entry = KernelEntry(name=name, impl=impl, replaces=replaces, status=KernelStatus.CANDIDATE,
                            hypothesis=hypothesis, notes=notes)
        return self._set_status(entry, status)

    def promote(self, name: str) -> KernelEntry:
        """Make ``name`` its operation's champion; the previous champion (if any) is retired
        in the same call, so the operation never has two champions or, in between, none."""
        entry = self.get(name)
        sitting = self._champion_of.get(entry.replaces)
        if sitting == name:
            return entry
        if sitting is not None:
            self._set_status(self._entries[sitting], KernelStatus.RETIRED)
        return self._set_status(entry, KernelStatus.CHAMPION)

    def retire(self, name: str) -> KernelEntry:
        return self._set_status(self.get(name), KernelStatus.RETIRED)

    def unregister(self, name: str) -> None:
        entry = self.get(name)
        if self._champion_of.get(entry.replaces) == name:
            del self._champion_of[entry.replaces]
        del self._entries[name]

    def clear(self) -> None:
        self._entries = {}
        self._champion_of = {}

    # -- queries -------------------------------------------------------------------------

    def get(self, name: str) -> KernelEntry:
        entry = self._entries.get(name)
        if entry is None:
            raise RegistryError(f"unknown kernel {name!r}")
        return entry

    def champion(self, replaces: str) -> KernelEntry | None:
        name = self._champion_of.get(replaces)
        return None if name is None else self._entries[name]

    def champions(self) -> dict[str, KernelEntry]:
        """``operation -> champion`` for every operation that has one, in name order."""
        return {op: self._entries[self._champion_of[op]] for op in sorted(self._champion_of)}

    def for_op(self, replaces: str) -> tuple[KernelEntry, ...]:
        """Every kernel registered against ``replaces``, whatever its status, in
        registration order."""
        return tuple(e for e in self._entries.values() if e.replaces == replaces)

    def check_invariants(self) -> None:
        """Rebuild the champion index from the entries and compare it with the stored one."""
        derived: dict[str, str] = {}
        for key, entry in self._entries.items():
            if key != entry.name:
                raise RegistryError(f"the entry stored under {key!r} is named {entry.name!r}")
            if entry.replaces not in self._replaceable_ops:
                raise RegistryError(f"{key!r} replaces {entry.replaces!r}, which is not a replaceable operation")
            if entry.status is KernelStatus.CHAMPION:
                if entry.replaces in derived:
                    raise RegistryError(
                        f"{entry.replaces!r} has two champions: {derived[entry.replaces]!r} and {key!r}")
                derived[entry.replaces] = key
        if derived != self._champion_of:
            raise RegistryError(f"champion index {self._champion_of} disagrees with the entries {derived}")

    def __len__(self) -> int:
        return len(self._entries)

    def __contains__(self, name: object) -> bool:
        return name in self._entries

    def __iter__(self) -> Iterator[KernelEntry]:
        return iter(tuple(self._entries.values()))

    def __repr__(self) -> str:
        return f"<KernelRegistry: {len(self)} kernels, champions for {len(self._champion_of)} operations>"


#: The process-wide registry.
REGISTRY = KernelRegistry()

#: Kernel name -> builder ``(model, *, device, dtype, seed) -> tuple[KernelCheck, ...]``.
CHECK_BUILDERS: dict[str, Callable[..., tuple]] = {}


def register_checks(kernel_name: str, builder: Callable[..., tuple]) -> None:
    """Attach the per-op correctness checks of ``kernel_name`` (one builder per kernel)."""
    previous = CHECK_BUILDERS.setdefault(kernel_name, builder)
    if previous is not builder:
        raise ValueError(f"{kernel_name!r} has a check builder already")


def build_kernel_checks(model, *, registry: KernelRegistry | None = None, **kwargs) -> tuple:
    """The checks of every champion that has a builder, champions in operation order;
    ``kwargs`` (device, dtype, seed) go to each builder unchanged."""
    reg = REGISTRY if registry is None else registry
    builders = [CHECK_BUILDERS[e.name] for e in reg.champions().values() if e.name in CHECK_BUILDERS]
    return tuple(check for build in builders for check in build(model, **kwargs))


# -- registered kernels --------------------------------------------------------------------
# Importing ``hip_ops`` defines the torch.library ops; it does not load the HIP library, so
# the registry imports on a machine without a GPU (the ops raise when called there).

from . import hip_ops as _hip  # noqa: E402

_CHAMPIONS = (
    ("hip_tiled_gemv_int4", _hip.tiled_gemv_int4, "decode_step",
     "Group-128 int4 GEMV (tied head and every layer linear): exact bf16((n-8)*s) dequant, MFMA "
     "16x16x32 bf16, fp32 accumulation; the reference's tiled_gemv_int4 signature."),
    ("hip_silu_mul", _hip.silu_mul, "swiglu_mlp", "bf16(bf16(silu(g)) * u), one pass."),
    ("hip_rms_norm", _hip.rms_norm, "rms_norm", "RMSNorm with the (1 + w) scale, one workgroup per row."),
    ("hip_add_rms_norm", _hip.add_rms_norm, "rms_norm_residual", "(residual + x, rms_norm(residual + x))."),
    ("hip_partial_rope", _hip.apply_partial_rope, "qkv_projection_rope",
     "Partial RoPE in the reference's bf16 op order."),
    ("hip_causal_conv_step", _hip.fused_causal_conv_step, "causal_conv",
     "4-tap depthwise causal conv at seq_len 1, history advanced in place."),
    ("hip_gated_delta_decode", _hip.gated_delta_decode, "gated_delta_rule",
     "One fused token of GatedDeltaNet's middle: conv + SiLU, L2 norms, gates, delta rule."),
    ("hip_gated_attention_decode", _hip.gated_attention_decode, "gqa_attention",
     "Gated GQA decode: q/k norm + partial RoPE + cache write + split-KV attention + merge + gate."),
    ("hip_decode_engine", _hip.static_decode_engine, "decode_cache",
     "Static decode state at fixed addresses and the whole step captured in one HIP graph."),
)

for _name, _impl, _op, _notes in _CHAMPIONS:
    REGISTRY.register(_name, impl=_impl, replaces=_op, status=KernelStatus.CHAMPION, notes=_notes)

# Batch 1 only, and Qwen3.5-4B's head geometry only, so not the default champion of its
# operation; REGISTRY.promote("hip_persistent_decode") before apply_champions selects it.
REGISTRY.register(
    "hip_persistent_decode", impl=_hip.persistent_decoder, replaces="decode_cache", status=KernelStatus.CANDIDATE,
    notes="Every layer of every decode step in one persistent launch; the 8 XCDs act as 8 tensor-parallel "
          "ranks (column-parallel projections, row-parallel out/down with a cross-XCD all-reduce).")

# The reference's two standalone ops with their own signatures (its hypotheses 007 and 008):
# candidates beside the fused champions of the same operations, for call sites written
# against deltaforge::delta_rule_step / deltaforge::split_kv_decode_attention.
REGISTRY.register(
    "hip_delta_rule_step", impl=_hip.delta_rule_step, replaces="gated_delta_rule", status=KernelStatus.CANDIDATE,
    notes="deltaforge::delta_rule_step's signature: one step on normalised fp32 q/k/v, g, beta; "
          "(out, new_state) fp32.")
REGISTRY.register(
    "hip_split_kv_decode_attention", impl=_hip.split_kv_decode_attention, replaces="gqa_attention",
    status=KernelStatus.CANDIDATE,
    notes="deltaforge::split_kv_decode_attention's signature: single-token GQA over a whole cache, KV scan split "
          "and merged by log-sum-exp.")

register_checks("hip_tiled_gemv_int4", _hip.tiled_gemv_int4_checks)
register_checks("hip_delta_rule_step", _hip.delta_rule_step_checks)
register_checks("hip_split_kv_decode_attention", _hip.split_kv_decode_attention_checks)
