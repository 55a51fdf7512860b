"""Assembling the HIP champions into a decode path (reference src/deltaforge/model.py:25-148).

Same surface as the reference's model module: ``INSTALLERS`` keyed by kernel name,
``register_installer``, ``apply_champions`` (raises ``InstallerMissing`` rather than silently
running anything else), and ``greedy_decode`` with the ``model.decode_loop`` hook the
reference calls (model.py:131-147).

The model here is a ``SynthModel``-shaped object (a config, canonical int4 linears and bf16
small parameters). Each op-level installer checks that its kernel supports the model's
shapes and records itself; the ``decode_cache`` champion's installer sets
``model.decode_loop`` to a loop driving ``DecodeEngine``, the graph-captured step that calls
every installed kernel. There is no path that decodes without the HIP library.
"""

from __future__ import annotations

from collections.abc import Callable, Mapping

import torch

from .kernels import REGISTRY, KernelEntry, KernelRegistry

__all__ = [
    "INSTALLERS",
    "EngineDecodeLoop",
    "InstallerMissing",
    "PersistentDecodeLoop",
    "apply_champions",
    "greedy_decode",
    "register_installer",
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

#: Kernels every decode step calls; the decode loop refuses to run unless all are installed.
STEP_KERNELS = (
    "hip_tiled_gemv_int4",
    "hip_silu_mul",
    "hip_rms_norm",
    "hip_add_rms_norm",
    "hip_partial_rope",
    "hip_causal_conv_step",
    "hip_gated_delta_decode",
    "hip_gated_attention_decode",
)


def _installed(model) -> set:
    s = getattr(model, "installed_kernels", None)
    if s is None:
        s = set()
        model.installed_kernels = s
    return s


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
    _installed(model).add(entry.name)


def _install_delta(model, entry: KernelEntry) -> None:
    c = model.config
    _require(c.linear_key_head_dim == 128 and c.linear_value_head_dim == 128, entry.name, "128-wide heads only")
    _require(c.linear_num_value_heads % c.linear_num_key_heads == 0, entry.name, "value heads per key head")
    _require(c.linear_conv_kernel_dim == 4, entry.name, "4-tap conv only")
    _installed(model).add(entry.name)


def _install_attention(model, entry: KernelEntry) -> None:
    c = model.config
    _require(c.head_dim == 256, entry.name, "head_dim 256 only")
    _require(c.num_attention_heads == 4 * c.num_key_value_heads, entry.name, "4 query heads per KV head")
    _installed(model).add(entry.name)


def _install_marker(model, entry: KernelEntry) -> None:
    _installed(model).add(entry.name)


class EngineDecodeLoop:
    """``model.decode_loop``: prefill the prompt through the captured decode step (teacher
    forced), then greedy-decode, all inside one ``DecodeEngine`` sized for the request."""

    def __init__(self, device: str | torch.device = "cuda") -> None:
        self.device = torch.device(device)
        self.engine = None

    def __call__(self, model, input_ids: torch.Tensor, max_new_tokens: int, cache=None) -> torch.Tensor:
        from .engine import DecodeEngine

        missing = [k for k in STEP_KERNELS if k not in _installed(model)]
        if missing:
            raise InstallerMissing(f"decode step kernels not installed: {missing}")
        if input_ids.dim() != 2 or input_ids.dtype != torch.int64:
            raise ValueError(f"input_ids must be int64 [B, P], got {input_ids.dtype} {tuple(input_ids.shape)}")
        batch, plen = input_ids.shape
        need = plen + max_new_tokens + 1
        e = self.engine
        if e is None or e.batch != batch or e.max_seq_len < need or e.max_new_tokens < max_new_tokens:
            e = DecodeEngine(model, batch=batch, max_seq_len=need, device=self.device, max_new_tokens=max_new_tokens)
            self.engine = e
        e.prefill(input_ids.to(self.device))
        first = e.tokens.clone()  # argmax after the last prompt token
        if max_new_tokens > 1:
            e.decode(max_new_tokens - 1)
        generated = torch.cat((first[:, None], e.token_log[:, : max_new_tokens - 1]), dim=1)
        return generated.to(input_ids.device)


def _install_decode_loop(model, entry: KernelEntry) -> None:
    if getattr(model, "decode_loop", None) is None:
        model.decode_loop = EngineDecodeLoop()
    _installed(model).add(entry.name)


class PersistentDecodeLoop:
    """``model.decode_loop`` for batch 1: prefill and greedy decode each run in one persistent
    launch of ``df_decode_persistent`` (every layer of every step inside one kernel), in a
    ``PersistentDecoder`` sized for the request. Batch > 1 raises ``ValueError``: the
    persistent kernel decodes one sequence."""

    def __init__(self, device: str | torch.device = "cuda") -> None:
        self.device = torch.device(device)
        self.decoder = None

    def __call__(self, model, input_ids: torch.Tensor, max_new_tokens: int, cache=None) -> torch.Tensor:
        from .persistent import PersistentDecoder

        if input_ids.dim() != 2 or input_ids.dtype != torch.int64:
            raise ValueError(f"input_ids must be int64 [B, P], got {input_ids.dtype} {tuple(input_ids.shape)}")
        batch, plen = input_ids.shape
        if batch != 1:
            raise ValueError(f"the persistent decode loop runs batch 1, got batch {batch}")
        need = plen + max_new_tokens + 1
        d = self.decoder
        if d is None or d.max_seq_len < need or d.max_new_tokens < max_new_tokens:
            d = PersistentDecoder(model, max_seq_len=need, device=self.device, max_new_tokens=max_new_tokens)
            self.decoder = d
        d.prefill(input_ids.to(self.device))
        first = d.tokens.clone()  # argmax after the last prompt token
        if max_new_tokens > 1:
            d.decode(max_new_tokens - 1)
        d.check()
        generated = torch.cat((first.view(1, 1), d.token_log[:, : max_new_tokens - 1]), dim=1)
        return generated.to(input_ids.device)


def _install_persistent_loop(model, entry: KernelEntry) -> None:
    """The persistent kernel replaces the whole step, so it needs none of ``STEP_KERNELS``; it
    takes the decode loop over from any other ``decode_cache`` implementation."""
    from .persistent import check_geometry

    try:
        check_geometry(model.config)
    except ValueError as e:
        raise ValueError(f"{entry.name} does not support this model: {e}") from None
    model.decode_loop = PersistentDecodeLoop()
    _installed(model).add(entry.name)


register_installer("hip_tiled_gemv_int4", _install_gemv)
register_installer("hip_silu_mul", _install_marker)
register_installer("hip_rms_norm", _install_marker)
register_installer("hip_add_rms_norm", _install_marker)
register_installer("hip_partial_rope", _install_marker)
register_installer("hip_causal_conv_step", _install_delta)
register_installer("hip_gated_delta_decode", _install_delta)
register_installer("hip_gated_attention_decode", _install_attention)
register_installer("hip_decode_engine", _install_decode_loop)
register_installer("hip_persistent_decode", _install_persistent_loop)
register_installer("hip_delta_rule_step", _install_delta)
register_installer("hip_split_kv_decode_attention", _install_attention)
