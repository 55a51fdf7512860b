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
    """Raised when a registration would violate a registry invariant."""


@dataclass(frozen=True)
class KernelEntry:
    name: str
    impl: Callable[..., object]
    replaces: str
    status: KernelStatus
    hypothesis: str | None = None
    notes: str = ""


class KernelRegistry:
    """Kernel name -> entry, with the one-champion-per-operation invariant enforced."""

    def __init__(self, replaceable_ops: frozenset[str] = REPLACEABLE_OPS) -> None:
        self._replaceable_ops = replaceable_ops
        self._entries: dict[str, KernelEntry] = {}

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
        if name in self._entries:
            raise RegistryError(f"kernel {name!r} is already registered")
        if replaces not in self._replaceable_ops:
            raise RegistryError(
                f"kernel {name!r} replaces unknown operation {replaces!r}; "
                f"known operations: {sorted(self._replaceable_ops)}"
            )
        status = KernelStatus(status)
        if status is KernelStatus.CHAMPION:
            incumbent = self.champion(replaces)
            if incumbent is not None:
                raise RegistryError(
                    f"cannot register {name!r} as champion of {replaces!r}: {incumbent.name!r} already "
                    "holds it; promote() demotes the incumbent in the same step"
                )
        entry = KernelEntry(name=name, impl=impl, replaces=replaces, status=status, hypothesis=hypothesis, notes=notes)
        self._entries[name] = entry
        return entry

    def promote(self, name: str) -> KernelEntry:
        """Make ``name`` the champion of its operation, retiring the incumbent (never two, never none)."""
        entry = self.get(name)
        if entry.status is KernelStatus.CHAMPION:
            return entry
        incumbent = self.champion(entry.replaces)
        if incumbent is not None:
            self._entries[incumbent.name] = replace(incumbent, status=KernelStatus.RETIRED)
        promoted = replace(entry, status=KernelStatus.CHAMPION)
        self._entries[name] = promoted
        return promoted

    def retire(self, name: str) -> KernelEntry:
        retired = replace(self.get(name), status=KernelStatus.RETIRED)
        self._entries[name] = retired
        return retired

    def unregister(self, name: str) -> None:
        del self._entries[name]

    def clear(self) -> None:
        self._entries.clear()

    def get(self, name: str) -> KernelEntry:
        try:
            return self._entries[name]
        except KeyError:
            raise RegistryError(f"no kernel registered as {name!r}") from None

    def champion(self, replaces: str) -> KernelEntry | None:
        found = [e for e in self._entries.values() if e.replaces == replaces and e.status is KernelStatus.CHAMPION]
        if len(found) > 1:  # pragma: no cover - register/promote make this unreachable
            raise RegistryError(f"registry invariant violated: {len(found)} champions for {replaces!r}")
        return found[0] if found else None

    def champions(self) -> dict[str, KernelEntry]:
        return {op: e for op in sorted(self._replaceable_ops) if (e := self.champion(op)) is not None}

    def for_op(self, replaces: str) -> tuple[KernelEntry, ...]:
        return tuple(e for e in self._entries.values() if e.replaces == replaces)

    def check_invariants(self) -> None:
        for op in self._replaceable_ops:
            self.champion(op)
        for name, entry in self._entries.items():
            if entry.name != name:
                raise RegistryError(f"entry keyed {name!r} carries name {entry.name!r}")
            if entry.replaces not in self._replaceable_ops:
                raise RegistryError(f"kernel {name!r} replaces unknown operation {entry.replaces!r}")

    def __len__(self) -> int:
        return len(self._entries)

    def __contains__(self, name: object) -> bool:
        return name in self._entries

    def __iter__(self) -> Iterator[KernelEntry]:
        return iter(self._entries.values())

    def __repr__(self) -> str:
        return f"KernelRegistry({len(self._entries)} kernels, {len(self.champions())} champions)"


#: The process-wide registry.
REGISTRY = KernelRegistry()

#: Kernel name -> builder ``(model, *, device, dtype, seed) -> tuple[KernelCheck, ...]``.
CHECK_BUILDERS: dict[str, Callable[..., tuple]] = {}


def register_checks(kernel_name: str, builder: Callable[..., tuple]) -> None:
    if kernel_name in CHECK_BUILDERS:
        raise ValueError(f"checks for kernel {kernel_name!r} are already registered")
    CHECK_BUILDERS[kernel_name] = builder


def build_kernel_checks(model, *, registry: KernelRegistry | None = None, **kwargs) -> tuple:
    """Every champion's per-op checks against ``model`` (kernels without a builder are skipped)."""
    registry = REGISTRY if registry is None else registry
    checks: list = []
    for entry in registry.champions().values():
        builder = CHECK_BUILDERS.get(entry.name)
        if builder is not None:
            checks.extend(builder(model, **kwargs))
    return tuple(checks)


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

register_checks("hip_tiled_gemv_int4", _hip.tiled_gemv_int4_checks)
