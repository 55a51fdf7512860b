"""Assembling the HIP champions into a decode path (reference src/deltaforge/model.py:25-148).

Same surface as the reference's model module: ``INSTALLERS`` keyed by kernel name,
``register_installer``, ``apply_champions`` (raises ``InstallerMissing`` rather than silently
running anything else), and ``greedy_decode`` with the ``model.decode_loop`` hook the
reference calls (model.py:131-147).

The model here is a ``SynthModel``-shaped object (a config, canonical int4 linears and bf16
small parameters). Each op-level installer checks that its kernel supports the model's
shapes and seats it at its operation's slot (``model.kernel_slots``); the ``decode_cache``
champion's installer sets ``model.decode_loop`` to a loop driving ``DecodeEngine`` (whose
step calls the kernel seated at each slot) or the persistent kernel. There is no path that
decodes without the HIP library.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping

import torch

from .kernels import REGISTRY, KernelEntry, KernelRegistry

__all__ = [
    "INSTALLERS",
    "STEP_SLOTS",
    "EngineDecodeLoop",
    "InstallerMissing",
    "PersistentDecodeLoop",
    "apply_champions",
    "greedy_decode",
    "installed_slots",
    "register_installer",
    "step_plan",
]


class InstallerMissing(RuntimeError):
    """A champion kernel exists for an operation, but nothing knows how to install it."""


#: Kernel name -> ``installer(model, entry)``.
INSTALLERS: dict[str, Callable[[object, KernelEntry], None]] = {}


def register_installer(kernel_name: str, installer: Callable[[object, KernelEntry], None]) -> None:
    if kernel_name in INSTALLERS:
        raise ValueError(f"installer for kernel {kernel_name!r} is already registered")
    INSTALLERS[kernel_name] = installer


def apply_champions(
    model,
    registry: KernelRegistry = REGISTRY,
    installers: Mapping[str, Callable[[object, KernelEntry], None]] | None = None,
) -> tuple[str, ...]:
    """Install every champion into ``model``; returns the kernel names installed."""
    registry.check_invariants()
    table = INSTALLERS if installers is None else installers
    applied: list[str] = []
    for op, entry in registry.champions().items():
        installer = table.get(entry.name)
        if installer is None:
            raise InstallerMissing(
                f"{entry.name!r} is champion of {op!r} but no installer is registered for it; refusing "
                "to run, because running anything else would report the wrong implementation"
            )
        installer(model, entry)
        applied.append(entry.name)
    return tuple(applied)


@torch.no_grad()
def greedy_decode(model, input_ids: torch.Tensor, max_new_tokens: int, cache=None) -> torch.Tensor:
    """Greedy-decode ``max_new_tokens`` and return only the generated ids ``[B, max_new_tokens]``."""
    if max_new_tokens < 1:
        raise ValueError("max_new_tokens must be at least 1")
    loop = getattr(model, "decode_loop", None)
    if loop is None:
        raise InstallerMissing("no decode loop installed: apply_champions(model) first")
    generated = loop(model, input_ids, max_new_tokens, cache)
    if generated.shape[-1] != max_new_tokens:
        raise RuntimeError(f"decode loop returned {generated.shape[-1]} tokens, expected {max_new_tokens}")
    return generated


# -- installers ------------------------------------------------------------------------------

#: The decode step's call sites: operation -> the kernels that can serve it. The graph step
#: fuses the first kernel of each slot into its launches (RMSNorm, the residual add and
#: SwiGLU run in the GEMV's prologue and epilogue, with the standalone kernels' arithmetic).
#: The second kernel of the delta and attention slots is the reference-signature standalone
#: op; with it installed the step composes that slot op by op, as the reference composes it
#: (kernels/gated_delta_step.py:231-300, kernels/flash_decode_splitkv.py:289-334). A decode
#: loop refuses to run unless every slot holds an installed kernel it can call.
STEP_SLOTS = {
    "decode_step": ("hip_tiled_gemv_int4",),
    "swiglu_mlp": ("hip_silu_mul",),
    "rms_norm": ("hip_rms_norm",),
    "rms_norm_residual": ("hip_add_rms_norm",),
    "qkv_projection_rope": ("hip_partial_rope",),
    "causal_conv": ("hip_causal_conv_step",),
    "gated_delta_rule": ("hip_gated_delta_decode", "hip_delta_rule_step"),
    "gqa_attention": ("hip_gated_attention_decode", "hip_split_kv_decode_attention"),
}

#: Every kernel some slot of the decode step accepts.
STEP_KERNELS = tuple(name for names in STEP_SLOTS.values() for name in names)

#: Slot -> the standalone op whose installation makes the step compose that slot.
_STANDALONE = {"gated_delta_rule": "hip_delta_rule_step", "gqa_attention": "hip_split_kv_decode_attention"}


def installed_slots(model) -> dict[str, KernelEntry]:
    """Operation -> the kernel the installers put at its call sites."""
    slots = getattr(model, "kernel_slots", None)
    if slots is None:
        slots = {}
        model.kernel_slots = slots
    return slots


def _installed(model) -> set:
    s = getattr(model, "installed_kernels", None)
    if s is None:
        s = set()
        model.installed_kernels = s
    return s


def _seat(model, entry: KernelEntry) -> None:
    installed_slots(model)[entry.replaces] = entry
    _installed(model).add(entry.name)


def step_plan(model) -> dict[str, Callable]:
    """The standalone compositions the graph step must run, ``slot -> impl`` (the installed
    entries' own callables) for ``DecodeEngine(standalone=...)``. Raises ``InstallerMissing``
    when a slot is empty or holds a kernel the step has no call site for."""
    from .engine import STANDALONE_SLOTS

    slots = installed_slots(model)
    empty = [op for op in STEP_SLOTS if op not in slots]
    if empty:
        raise InstallerMissing(f"decode step slots with no installed kernel: {empty} (apply_champions first)")
    foreign = {op: slots[op].name for op, names in STEP_SLOTS.items() if slots[op].name not in names}
    if foreign:
        raise InstallerMissing(f"the decode step has no call site for {foreign}; refusing to run something else")
    plan: dict[str, Callable] = {}
    for op, name in _STANDALONE.items():
        if slots[op].name == name:
            plan[op] = slots[op].impl
            for dep in STANDALONE_SLOTS[op]:
                plan[dep] = slots[dep].impl
    return plan


def _require(cond: bool, kernel: str, why: str) -> None:
    if not cond:
        raise ValueError(f"{kernel} does not support this model: {why}")


def _install_gemv(model, entry: KernelEntry) -> None:
    """Every linear needs K % 256; the launched matrices (the tied head, and per layer the
    fused input projection, gate|up, down, out) need N % 64. in_proj_a/b are 32 wide and only
    ever run inside the fused input projection."""
    c = model.config
    for name, w in model.linears.items():
        _require(w.K % 256 == 0 and w.N % 16 == 0, entry.name, f"{name} is {w.K} x {w.N} (needs K%256, N%16)")
    fused_in = (2 * c.linear_key_dim + 2 * c.linear_value_dim + 2 * c.linear_num_value_heads,
                2 * c.num_attention_heads * c.head_dim + 2 * c.num_key_value_heads * c.head_dim)
    for n in (*fused_in, 2 * c.intermediate_size, c.hidden_size, c.vocab_size):
        _require(n % 64 == 0, entry.name, f"a launched matrix is {n} wide (needs N%64)")
    _seat(model, entry)


def _install_delta(model, entry: KernelEntry) -> None:
    c = model.config
    _require(c.linear_key_head_dim == 128 and c.linear_value_head_dim == 128, entry.name, "128-wide heads only")
    _require(c.linear_num_value_heads % c.linear_num_key_heads == 0, entry.name, "value heads per key head")
    _require(c.linear_conv_kernel_dim == 4, entry.name, "4-tap conv only")
    _seat(model, entry)


def _install_attention(model, entry: KernelEntry) -> None:
    c = model.config
    _require(c.head_dim == 256, entry.name, "head_dim 256 only")
    _require(c.num_attention_heads == 4 * c.num_key_value_heads, entry.name, "4 query heads per KV head")
    _seat(model, entry)


def _install_rope(model, entry: KernelEntry) -> None:
    c = model.config
    _require(c.rotary_dim % 2 == 0 and c.rotary_dim <= c.head_dim, entry.name, "an even rotary width within the head")
    _seat(model, entry)


def _install_norm(model, entry: KernelEntry) -> None:
    _seat(model, entry)


def _prefiller(loop, model):
    """The loop's parallel prefill (built once per loop), or ``None`` when the prefill kernels
    do not cover the model's geometry; then the prompt is teacher-forced through the step."""
    from .prefill import Prefiller, unsupported_geometry

    if loop.prefiller is None and unsupported_geometry(model.config) is None:
        loop.prefiller = Prefiller(model, loop.device)
    return loop.prefiller


def _check_ids(input_ids: torch.Tensor) -> tuple[int, int]:
    if input_ids.dim() != 2 or input_ids.dtype != torch.int64:
        raise ValueError(f"input_ids must be int64 [B, P], got {input_ids.dtype} {tuple(input_ids.shape)}")
    return input_ids.shape[0], input_ids.shape[1]


class EngineDecodeLoop:
    """``model.decode_loop``: prefill the prompt in one parallel pass (``Prefiller``; the
    reference's forward over the prompt), then greedy-decode inside one ``DecodeEngine``
    sized for the request. Its step calls the kernels installed at each slot: the fused
    ones inside captured HIP graphs, a standalone delta or attention op eagerly at its call
    site. Models outside the prefill kernels' geometry are prefilled by teacher-forced
    decode steps instead; ``last_prefill`` says which ran."""

    def __init__(self, device: str | torch.device = "cuda") -> None:
        self.device = torch.device(device)
        self.engine = None
        self.prefiller = None
        self.last_prefill = None

    def __call__(self, model, input_ids: torch.Tensor, max_new_tokens: int, cache=None) -> torch.Tensor:
        from .engine import DecodeEngine

        plan = step_plan(model)
        batch, plen = _check_ids(input_ids)
        need = plen + max_new_tokens + 1
        e = self.engine
        if (e is None or e.batch != batch or e.max_seq_len < need or e.max_new_tokens < max_new_tokens
                or e.standalone != plan):
            e = DecodeEngine(model, batch=batch, max_seq_len=need, device=self.device, max_new_tokens=max_new_tokens,
                             standalone=plan)
            self.engine = e
        ids = input_ids.to(self.device)
        pre = _prefiller(self, model)
        if pre is not None:
            pre.fill_engine(e, ids)
            self.last_prefill = "parallel"
        else:
            e.prefill(ids)
            self.last_prefill = "teacher-forced"
        first = e.tokens.clone()  # argmax after the last prompt token
        if max_new_tokens > 1:
            e.decode(max_new_tokens - 1)
        generated = torch.cat((first[:, None], e.token_log[:, : max_new_tokens - 1]), dim=1)
        return generated.to(input_ids.device)


def _install_decode_loop(model, entry: KernelEntry) -> None:
    if getattr(model, "decode_loop", None) is None:
        model.decode_loop = EngineDecodeLoop()
    _seat(model, entry)


class PersistentDecodeLoop:
    """``model.decode_loop`` for batch 1: the prompt prefilled in one parallel pass
    (``Prefiller.fill``), then greedy decode in one persistent launch of
    ``df_decode_persistent`` (every layer of every step inside one kernel), in a
    ``PersistentDecoder`` sized for the request. Batch > 1 raises ``ValueError``: the
    persistent kernel decodes one sequence. It fuses every slot of the step itself, so it
    refuses to run when a standalone op holds a slot (the registry would be asking for a
    composition this kernel does not run)."""

    def __init__(self, device: str | torch.device = "cuda") -> None:
        self.device = torch.device(device)
        self.decoder = None
        self.prefiller = None
        self.last_prefill = None

    def __call__(self, model, input_ids: torch.Tensor, max_new_tokens: int, cache=None) -> torch.Tensor:
        from .persistent import PersistentDecoder

        standalone = {op: e.name for op, e in installed_slots(model).items() if _STANDALONE.get(op) == e.name}
        if standalone:
            raise InstallerMissing(f"the persistent kernel fuses every slot of the step, but {standalone} "
                                   "hold standalone ops; promote the graph engine to decode through them")
        batch, plen = _check_ids(input_ids)
        if batch != 1:
            raise ValueError(f"the persistent decode loop runs batch 1, got batch {batch}")
        need = plen + max_new_tokens + 1
        d = self.decoder
        if d is None or d.max_seq_len < need or d.max_new_tokens < max_new_tokens:
            d = PersistentDecoder(model, max_seq_len=need, device=self.device, max_new_tokens=max_new_tokens)
            self.decoder = d
        ids = input_ids.to(self.device)
        pre = _prefiller(self, model)
        if pre is not None:
            pre.fill(d, ids)
            self.last_prefill = "parallel"
        else:
            d.prefill(ids)
            self.last_prefill = "teacher-forced"
        first = d.tokens.clone()  # argmax after the last prompt token
        if max_new_tokens > 1:
            d.decode(max_new_tokens - 1)
        d.check()
        generated = torch.cat((first.view(1, 1), d.token_log[:, : max_new_tokens - 1]), dim=1)
        return generated.to(input_ids.device)


def _install_persistent_loop(model, entry: KernelEntry) -> None:
    """The persistent kernel replaces the whole step; it takes the decode loop over from any
    other ``decode_cache`` implementation."""
    from .persistent import check_geometry

    try:
        check_geometry(model.config)
    except ValueError as e:
        raise ValueError(f"{entry.name} does not support this model: {e}") from None
    model.decode_loop = PersistentDecodeLoop()
    _seat(model, entry)


register_installer("hip_tiled_gemv_int4", _install_gemv)
register_installer("hip_silu_mul", _install_norm)
register_installer("hip_rms_norm", _install_norm)
register_installer("hip_add_rms_norm", _install_norm)
register_installer("hip_partial_rope", _install_rope)
register_installer("hip_causal_conv_step", _install_delta)
register_installer("hip_gated_delta_decode", _install_delta)
register_installer("hip_gated_attention_decode", _install_attention)
register_installer("hip_decode_engine", _install_decode_loop)
register_installer("hip_persistent_decode", _install_persistent_loop)
register_installer("hip_delta_rule_step", _install_delta)
register_installer("hip_split_kv_decode_attention", _install_attention)
