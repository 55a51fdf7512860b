"""``torch.library`` custom ops over the gfx950 HIP kernels, one per replaceable operation.

Each op has the signature of the reference op it replaces, a ``register_fake`` so it traces
under ``torch.compile``/meta tensors, and the reference's error order: shape and dtype
problems raise ``ValueError``, then a CPU tensor raises ``RuntimeError`` (no PyTorch fallback;
reference kernels/_triton.py:56-69). The work is done by ``deltaforge_amd.ops``, which calls
the C ABI of ``libdeltaforge_hip.so`` on the current stream.

| op (``deltaforge_amd::``) | reference op it mirrors |
|---|---|
| ``tiled_gemv_int4``        | ``deltaforge::tiled_gemv_int4`` (kernels/tiled_gemv.py:915-958) |
| ``silu_mul``               | ``deltaforge::silu_mul`` (kernels/fused_swiglu.py:51-80) |
| ``rms_norm``               | ``deltaforge::rms_norm`` (kernels/fused_rmsnorm_residual.py:201-230) |
| ``add_rms_norm``           | ``deltaforge::add_rms_norm`` (kernels/fused_rmsnorm_residual.py:164-198) |
| ``partial_rope``           | ``deltaforge::partial_rope`` (kernels/fused_rope.py:97-158) |
| ``fused_causal_conv_step`` | ``deltaforge::fused_causal_conv_step`` (kernels/fused_causal_conv.py:136-181) |
| ``delta_rule_step``        | ``deltaforge::delta_rule_step`` (kernels/gated_delta_step.py:109-186) |
| ``split_kv_decode_attention`` | ``deltaforge::split_kv_decode_attention`` (kernels/flash_decode_splitkv.py:177-261) |
| ``gated_delta_decode``     | ``GatedDeltaNet.forward``'s decode middle (reference.py:512-550) |
| ``gated_attention_decode`` | ``GatedAttention.forward``'s decode branch (reference.py:610-677) |
"""

from __future__ import annotations

import weakref

import torch
from torch import Tensor

from .. import ops

__all__ = [
    "add_rms_norm",
    "apply_partial_rope",
    "delta_rule_step",
    "delta_rule_step_checks",
    "fused_causal_conv_step",
    "gated_attention_decode",
    "gated_delta_decode",
    "rms_norm",
    "silu_mul",
    "split_kv_decode_attention",
    "split_kv_decode_attention_checks",
    "static_decode_engine",
    "tiled_gemv_int4",
    "tiled_gemv_int4_checks",
]

BF16 = torch.bfloat16
GROUP = 128
MAX_ROWS = 16  # rows per GEMV launch; more rows run as consecutive 16-row launches


# ---------------------------------------------------------------------------------------
# int4 GEMV over the canonical K-major format
# ---------------------------------------------------------------------------------------

# Canonical (packed, scale) -> device tiling, cached per live tensor pair. The entry holds
# weak references, so a freed weight can never alias a new one at the same address; the
# tensors' version counters catch in-place rewrites.
_REPACKED: dict[tuple[int, int], tuple] = {}


def _repacked(packed: Tensor, scale: Tensor) -> ops.Int4Weight:
    key = (id(packed), id(scale))
    hit = _REPACKED.get(key)
    if hit is not None:
        pref, sref, pver, sver, weight = hit
        if pref() is packed and sref() is scale and pver == packed._version and sver == scale._version:
            return weight
    weight = ops.int4_repack(packed, scale)
    _REPACKED[key] = (weakref.ref(packed), weakref.ref(scale), packed._version, scale._version, weight)
    for k in [k for k, v in _REPACKED.items() if v[0]() is None or v[1]() is None]:
        del _REPACKED[k]
    return weight


def _check_int4(x: Tensor, packed: Tensor, scale: Tensor, group_size: int) -> tuple[int, int]:
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError(f"packed must be uint8 [K/2, N], got {packed.dtype} {tuple(packed.shape)}")
    half, n = packed.shape
    k = 2 * half
    if group_size != GROUP:
        raise ValueError(f"the HIP GEMV is the group-128 format, got group_size {group_size}")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, packed holds K={k}")
    if x.dtype != BF16:
        raise ValueError(f"x must be bf16, got {x.dtype}")
    if k % 256 or n % 64:
        raise ValueError(f"the HIP tiling needs K % 256 == 0 and N % 64 == 0, got K={k} N={n}")
    if scale.dtype != BF16 or tuple(scale.shape) != (k // GROUP, n):
        raise ValueError(f"scale must be bf16 [{k // GROUP}, {n}], got {scale.dtype} {tuple(scale.shape)}")
    return k, n


@torch.library.custom_op("deltaforge_amd::tiled_gemv_int4", mutates_args=())
def tiled_gemv_int4(x: Tensor, packed: Tensor, scale: Tensor, group_size: int) -> Tensor:
    """``bf16(x.float() @ bf16((nibble - 8) * scale).float())`` for ``x [..., K]`` and the
    canonical K-major int4 weight ``packed [K/2, N]``, ``scale [K/128, N]`` bf16."""
    k, n = _check_int4(x, packed, scale, group_size)
    ops.require_gpu(x, "tiled_gemv_int4")
    weight = _repacked(packed, scale)
    flat = x.reshape(-1, k).contiguous()
    out = torch.empty((flat.shape[0], n), dtype=BF16, device=x.device)
    for r0 in range(0, flat.shape[0], MAX_ROWS):
        r1 = min(r0 + MAX_ROWS, flat.shape[0])
        ops.int4_gemv(flat[r0:r1], weight, out=out[r0:r1])
    return out.reshape(*x.shape[:-1], n)


@tiled_gemv_int4.register_fake
def _(x, packed, scale, group_size):
    return x.new_empty((*x.shape[:-1], packed.shape[1]))


def tiled_gemv_int4_checks(model=None, *, device="cuda", dtype=None, seed: int = 0) -> tuple:
    """Per-op check of the GEMV against the reference's expression at the head shape's K,
    through the harness's ``check_kernel`` (atol 2e-2, rtol 1e-2)."""
    from ..harness.correctness import check_kernel
    from ..synth import draw_int4

    gen = torch.Generator().manual_seed(seed)
    w = draw_int4(gen, 2560, 1024)
    x = torch.randn((4, 2560), generator=gen).to(BF16)
    dense = _dequant_reference(w.packed, w.scale)
    return (
        check_kernel(
            "hip_tiled_gemv_int4",
            lambda: (x.float() @ dense.float()).to(BF16),
            lambda: tiled_gemv_int4(x.to(device), w.packed.to(device), w.scale.to(device), GROUP).cpu(),
            replaces="decode_step", atol=2e-2, rtol=1e-2,
        ),
    )


def _dequant_reference(packed: Tensor, scale: Tensor) -> Tensor:
    """bf16((nibble - 8) * scale) in the canonical layout (reference tiled_gemv.py:281-288)."""
    half, n = packed.shape
    low = (packed & 0x0F).to(torch.int16) - 8
    high = (packed >> 4).to(torch.int16) - 8
    q = torch.cat((low, high), 0).float().reshape(2 * half // GROUP, GROUP, n)
    return (q * scale.float().unsqueeze(1)).reshape(2 * half, n).to(BF16)


# ---------------------------------------------------------------------------------------
# Elementwise ops
# ---------------------------------------------------------------------------------------


@torch.library.custom_op("deltaforge_amd::silu_mul", mutates_args=())
def silu_mul(gate: Tensor, up: Tensor) -> Tensor:
    """``bf16(bf16(silu(gate)) * up)``."""
    return ops.silu_mul(gate, up)


@silu_mul.register_fake
def _(gate, up):
    return torch.empty_like(up)


@torch.library.custom_op("deltaforge_amd::rms_norm", mutates_args=())
def rms_norm(x: Tensor, weight: Tensor, eps: float) -> Tensor:
    """RMSNorm with the ``(1 + w)`` scale over the last axis."""
    return ops.rms_norm(x, weight, eps)


@rms_norm.register_fake
def _(x, weight, eps):
    return torch.empty_like(x)


@torch.library.custom_op("deltaforge_amd::add_rms_norm", mutates_args=())
def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    """``(residual + x, rms_norm(residual + x))``."""
    return ops.add_rms_norm(x, residual, weight, eps)


@add_rms_norm.register_fake
def _(x, residual, weight, eps):
    return torch.empty_like(x), torch.empty_like(x)


@torch.library.custom_op("deltaforge_amd::partial_rope", mutates_args=())
def apply_partial_rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``x [B, H, S, D]`` rotated on its first ``R`` dims by ``cos``/``sin`` ``[B, S, R]``."""
    return ops.partial_rope(x, cos, sin)


@apply_partial_rope.register_fake
def _(x, cos, sin):
    return torch.empty_like(x)


@torch.library.custom_op("deltaforge_amd::fused_causal_conv_step", mutates_args=("conv_cache",))
def fused_causal_conv_step(x: Tensor, conv_cache: Tensor, weight: Tensor) -> Tensor:
    """``x [B, C, 1]``, history ``conv_cache [B, C, 3]`` (advanced in place), ``weight [C, 1, 4]``."""
    return ops.causal_conv_step(x, conv_cache, weight)


@fused_causal_conv_step.register_fake
def _(x, conv_cache, weight):
    return torch.empty_like(x)


# ---------------------------------------------------------------------------------------
# Module-level decode ops
# ---------------------------------------------------------------------------------------


@torch.library.custom_op("deltaforge_amd::gated_delta_decode", mutates_args=("conv_cache", "state"))
def gated_delta_decode(
    mixed_qkv: Tensor, a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Tensor, conv_weight: Tensor,
    conv_cache: Tensor, state: Tensor, num_k_heads: int,
) -> Tensor:
    """One decode token of GatedDeltaNet between in_proj and the gated norm.

    ``mixed_qkv [B, C]`` pre-conv (q | k | v), ``a``/``b`` ``[B, Hv]``, ``A_log``/``dt_bias``
    ``[Hv]``, ``conv_weight [C, 1, 4]``, ``conv_cache [B, C, 3]`` and ``state [B, Hv, 128, 128]``
    fp32 both advanced in place. Returns the core output ``[B, Hv, 128]`` bf16."""
    if conv_cache.dim() != 3 or conv_cache.shape[-1] != 3:
        raise ValueError(f"conv_cache must be [B, C, 3], got {tuple(conv_cache.shape)}")
    history_out = torch.empty_like(conv_cache) if conv_cache.is_cuda else conv_cache
    out = ops.gated_delta_step(mixed_qkv, a, b, A_log, dt_bias, conv_weight, state, num_k_heads=num_k_heads,
                               conv_in=conv_cache, conv_out=history_out)
    conv_cache.copy_(history_out)
    return out


@gated_delta_decode.register_fake
def _(mixed_qkv, a, b, A_log, dt_bias, conv_weight, conv_cache, state, num_k_heads):
    batch, heads, _, dv = state.shape
    return mixed_qkv.new_empty((batch, heads, dv))


@torch.library.custom_op("deltaforge_amd::gated_attention_decode", mutates_args=("k_cache", "v_cache"))
def gated_attention_decode(
    q_gate: Tensor, k: Tensor, v: Tensor, q_norm_w: Tensor, k_norm_w: Tensor, inv_freq: Tensor,
    k_cache: Tensor, v_cache: Tensor, position: Tensor, num_q_heads: int, sigmoid_gate: bool, eps: float,
) -> Tensor:
    """One decode token of gated GQA after the projections: q/k RMSNorm(1+w), partial RoPE at
    ``position`` (device int32 scalar), k/v written at ``position``, attention over
    ``position + 1`` keys, output gate. ``q_gate [B, Hq*2*D]`` holds per head ``[query | gate]``;
    returns ``[B, Hq*D]`` bf16."""
    return ops.attention_decode(q_gate, k, v, q_norm_w, k_norm_w, inv_freq, k_cache, v_cache, position,
                                num_q_heads=num_q_heads, gate=0 if sigmoid_gate else 1, eps=eps)


@gated_attention_decode.register_fake
def _(q_gate, k, v, q_norm_w, k_norm_w, inv_freq, k_cache, v_cache, position, num_q_heads, sigmoid_gate, eps):
    return q_gate.new_empty((q_gate.shape[0], num_q_heads * k_cache.shape[-1]))


@torch.library.custom_op("deltaforge_amd::delta_rule_step", mutates_args=())
def delta_rule_step(state: Tensor, query: Tensor, key: Tensor, value: Tensor, g: Tensor,
                    beta: Tensor) -> tuple[Tensor, Tensor]:
    """One delta-rule step, ``(output, new_state)``: ``state (B, H, Dk, Dv)`` fp32,
    ``query``/``key`` ``(B, H, Dk)`` already l2-normed (the query scaled by ``Dk**-0.5``),
    ``value (B, H, Dv)``, log-space decay ``g`` and ``beta`` ``(B, H)``; the output is fp32."""
    return ops.delta_rule_step(state, query, key, value, g, beta)


@delta_rule_step.register_fake
def _(state, query, key, value, g, beta):
    batch, heads, _, value_dim = state.shape
    return state.new_empty((batch, heads, value_dim)), torch.empty_like(state)


@torch.library.custom_op("deltaforge_amd::split_kv_decode_attention", mutates_args=())
def split_kv_decode_attention(query: Tensor, key: Tensor, value: Tensor, scale: float, splits: int) -> Tensor:
    """Single-token GQA attention, ``query (B, Hq, D)`` over ``key``/``value``
    ``(B, Hkv, L, D)`` with the KV scan split ``splits`` ways and merged by log-sum-exp."""
    return ops.split_kv_decode_attention(query, key, value, scale, splits)


@split_kv_decode_attention.register_fake
def _(query, key, value, scale, splits):
    return torch.empty_like(query)


def _delta_rule_definition(state: Tensor, q: Tensor, k: Tensor, v: Tensor, g: Tensor, beta: Tensor):
    """The op's definition in fp32, as matrix products per head: decay the state by exp(g),
    recall k^T S, write beta * (v - recall) along k, read q^T S (reference.py:450-458)."""
    s = state.float() * torch.exp(g.float())[..., None, None]
    kf, qf = k.float().unsqueeze(-2), q.float().unsqueeze(-2)  # (B, H, 1, Dk)
    recall = (kf @ s).squeeze(-2)
    s = s + kf.transpose(-1, -2) @ ((v.float() - recall) * beta.float().unsqueeze(-1)).unsqueeze(-2)
    return (qf @ s).squeeze(-2), s


def delta_rule_step_checks(model=None, *, device="cuda", dtype=None, seed: int = 0) -> tuple:
    """The step against its fp32 definition (reference.py:450-458) at Qwen3.5's DeltaNet head
    shape, batch 1 and 8: state within 1e-4 (the north star's bar for the fp32 state), output
    within atol 2e-2 / rtol 1e-2."""
    from ..harness.correctness import check_kernel

    gen = torch.Generator().manual_seed(seed)
    checks = []
    for batch in (1, 8):
        state = torch.randn((batch, 32, 128, 128), generator=gen) * 0.1
        q = torch.nn.functional.normalize(torch.randn((batch, 32, 128), generator=gen), dim=-1) / 128 ** 0.5
        k = torch.nn.functional.normalize(torch.randn((batch, 32, 128), generator=gen), dim=-1)
        v = torch.randn((batch, 32, 128), generator=gen)
        g = -torch.nn.functional.softplus(torch.randn((batch, 32), generator=gen))
        beta = torch.sigmoid(torch.randn((batch, 32), generator=gen))
        want_out, want_state = _delta_rule_definition(state, q, k, v, g, beta)
        got_out, got_state = delta_rule_step(*(t.to(device) for t in (state, q, k, v, g, beta)))
        checks.append(check_kernel(f"hip_delta_rule_step state B={batch}", lambda: want_state, lambda: got_state.cpu(),
                                   replaces="gated_delta_rule", atol=1e-4, rtol=0.0))
        checks.append(check_kernel(f"hip_delta_rule_step out B={batch}", lambda: want_out, lambda: got_out.cpu(),
                                   replaces="gated_delta_rule", atol=2e-2, rtol=1e-2))
    return tuple(checks)


def _attention_definition(query: Tensor, key: Tensor, value: Tensor, scale: float) -> Tensor:
    """Single-token GQA attention in fp32: query head h reads KV head h // (Hq / Hkv);
    softmax over every key, rounded to the query's dtype at the end."""
    batch, hq, dim = query.shape
    hkv = key.shape[1]
    q = query.float().reshape(batch, hkv, hq // hkv, dim)
    probs = torch.softmax((q @ key.float().transpose(-1, -2)) * scale, dim=-1)
    return (probs @ value.float()).reshape(batch, hq, dim).to(query.dtype)


def split_kv_decode_attention_checks(model=None, *, device="cuda", dtype=None, seed: int = 0) -> tuple:
    """The reference's own cases for the op (flash_decode_splitkv.py:365-372: batch 1 and 32
    at 2048 keys, fewer keys than splits, a key count no tile divides) at Qwen3.5's attention
    head shape, against the attention's fp32 definition (gqa_decode.py:322-335)."""
    from ..harness.correctness import check_kernel

    gen = torch.Generator().manual_seed(seed)
    scale = 256 ** -0.5
    checks = []
    for batch, key_len, label in ((1, 2048, "batch 1, context 2048"), (32, 2048, "batch 32, context 2048"),
                                  (1, 3, "context shorter than the split count"),
                                  (1, 33, "context that is not a multiple of the tile")):
        q = torch.randn((batch, 16, 256), generator=gen).to(BF16)
        k = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
        v = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
        want = _attention_definition(q, k, v, scale)
        got = split_kv_decode_attention(q.to(device), k.to(device), v.to(device), scale, 8).cpu()
        checks.append(check_kernel(f"hip_split_kv_decode_attention {label}", lambda: want, lambda: got,
                                   replaces="gqa_attention", atol=2e-2, rtol=1e-2))
    return tuple(checks)


def static_decode_engine(model, *, batch: int = 1, max_seq_len: int, device="cuda", max_new_tokens: int = 0):
    """The ``decode_cache`` champion: a ``DecodeEngine`` holding every cache at a fixed address
    with the whole decode step captured in one HIP graph (see ``deltaforge_amd.engine``)."""
    from ..engine import DecodeEngine

    return DecodeEngine(model, batch=batch, max_seq_len=max_seq_len, device=device, max_new_tokens=max_new_tokens)


def persistent_decoder(model, *, max_seq_len: int, device="cuda", max_new_tokens: int = 256):
    """The ``decode_cache`` candidate for batch 1: a ``PersistentDecoder`` whose launches run
    every layer of many decode steps inside one kernel (see ``deltaforge_amd.persistent``)."""
    from ..persistent import PersistentDecoder

    return PersistentDecoder(model, max_seq_len=max_seq_len, device=device, max_new_tokens=max_new_tokens)
