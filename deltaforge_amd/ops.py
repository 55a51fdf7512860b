"""Host side of the HIP kernels: argument checks, workspaces and the ``deltaforge::`` ops.

Two layers:

* plain functions (``int4_gemv``, ``gated_delta_step``, ``attention_decode``, ...) that
  check shapes, then call the C ABI on the current HIP stream, writing into caller-given or
  freshly allocated tensors. The decode engine uses these with preallocated buffers so the
  whole step can be captured in a HIP graph.
* ``torch.library.custom_op("deltaforge::...")`` ops with ``register_fake``, the same
  registration surface the reference's slots use (reference kernels/*.py), for callers that
  plug single ops into a reference-shaped model.

Checks follow the reference's order (kernels/fused_rmsnorm_residual.py:133-161): shape and
dtype problems raise ``ValueError`` before the device check; a CPU tensor raises
``RuntimeError`` and nothing falls back to PyTorch.
"""

from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch
from torch import Tensor

from . import _native as N

__all__ = [
    "Int4Weight",
    "add_rms_norm",
    "argmax_tokens",
    "attention_decode",
    "attention_splits",
    "causal_conv_step",
    "delta_rule_step",
    "embed_bf16",
    "embed_int4",
    "gated_delta_step",
    "int4_dequant",
    "int4_gemv",
    "int4_repack",
    "partial_rope",
    "require_gpu",
    "rms_norm",
    "silu_mul",
    "split_kv_decode_attention",
    "workspace",
]

BF16 = torch.bfloat16


def require_gpu(t: Tensor, op: str) -> None:
    """The no-silent-fallback rule (reference kernels/_triton.py:56-69)."""
    if not t.is_cuda:
        raise RuntimeError(
            f"deltaforge::{op} requires a GPU tensor and has no PyTorch fallback, on purpose: "
            "falling back would run the reference while the caller believes it ran the kernel."
        )


def require_gpus(op: str, *tensors: Tensor | None) -> None:
    """``require_gpu`` for every tensor a kernel dereferences, all on one device: a host
    pointer (or another device's) handed to a kernel is a memory fault, not an error."""
    device = None
    for t in tensors:
        if t is None:
            continue
        require_gpu(t, op)
        if device is None:
            device = t.device
        elif t.device != device:
            raise RuntimeError(f"deltaforge::{op}: tensors on {device} and {t.device}; one device per call")


def _check_dtype(op: str, name: str, t: Tensor, dtype: torch.dtype, numel: int | None = None) -> None:
    if t.dtype != dtype:
        raise ValueError(f"{op}: {name} must be {dtype}, got {t.dtype}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{op}: {name} must hold {numel} elements, got {t.numel()}")


def _stream(t: Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


_WORKSPACES: dict[tuple, Tensor] = {}


def workspace(device: torch.device, nbytes: int, tag: str = "default") -> Tensor:
    """A zero-filled byte buffer per (device, stream, tag), grown on demand and kept.

    Kernels that use a completion counter leave it at zero, so the buffer stays ready. Ops
    on one stream run in order; ops on different streams get different buffers.
    """
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream, tag)
    buf = _WORKSPACES.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = buf
    return buf


# ---------------------------------------------------------------------------------------
# int4
# ---------------------------------------------------------------------------------------


@dataclass
class Int4Weight:
    """A group-128 int4 weight in the device tiling, plus its logical ``[K, N]`` shape."""

    w: Tensor  # uint8, (N/16)*(K/128)*1024 bytes
    s: Tensor  # bf16, (N/16)*(K/128)*16
    K: int
    N: int

    @property
    def nbytes(self) -> int:
        return self.w.numel() + 2 * self.s.numel()


def int4_repack(packed: Tensor, scale: Tensor) -> Int4Weight:
    """Canonical K-major int4 (reference tiled_gemv.py:242-278 layout, bf16 scales) -> device tiling."""
    if packed.dtype != torch.uint8 or packed.dim() != 2:
        raise ValueError(f"packed must be uint8 [K/2, N], got {packed.dtype} {tuple(packed.shape)}")
    half, n = packed.shape
    k = 2 * half
    if k % 256 or n % 64:
        raise ValueError(f"int4 tiling needs K % 256 == 0 and N % 64 == 0, got K={k} N={n}")
    if scale.dtype != BF16 or tuple(scale.shape) != (k // 128, n):
        raise ValueError(f"scale must be bf16 [{k // 128}, {n}], got {scale.dtype} {tuple(scale.shape)}")
    require_gpu(packed, "int4_repack")
    packed = packed.contiguous()
    scale = scale.contiguous()
    w = torch.empty((n // 16) * (k // 128) * 1024, dtype=torch.uint8, device=packed.device)
    s = torch.empty((n // 16) * (k // 128) * 16, dtype=BF16, device=packed.device)
    N.check(N.lib().df_int4_repack(packed.data_ptr(), scale.data_ptr(), k, n, w.data_ptr(), s.data_ptr(),
                                   _stream(packed)), "int4_repack")
    return Int4Weight(w, s, k, n)


def interleave_gate_up(gate_packed: Tensor, gate_scale: Tensor, up_packed: Tensor, up_scale: Tensor):
    """Canonical gate ``[K/2, I]`` and up ``[K/2, I]`` -> one ``[K/2, 2I]`` matrix whose 16-column
    tiles alternate gate, up, gate, up ... (and the same for the scales), the layout
    ``DF_EPI_SWIGLU`` pairs. Each column keeps its own group scales.
    """
    half, inter = gate_packed.shape
    if up_packed.shape != gate_packed.shape or inter % 16:
        raise ValueError("gate and up must be the same [K/2, I] shape with I % 16 == 0")
    groups = gate_scale.shape[0]
    packed = torch.stack((gate_packed.reshape(half, inter // 16, 16), up_packed.reshape(half, inter // 16, 16)), 2)
    scale = torch.stack((gate_scale.reshape(groups, inter // 16, 16), up_scale.reshape(groups, inter // 16, 16)), 2)
    return packed.reshape(half, 2 * inter), scale.reshape(groups, 2 * inter)


def int4_dequant(weight: Int4Weight) -> Tensor:
    """bf16 ``[K, N]``: ``bf16((nibble - 8) * scale)`` (reference tiled_gemv.py:281-288 + .to(bf16))."""
    out = torch.empty((weight.K, weight.N), dtype=BF16, device=weight.w.device)
    N.check(N.lib().df_int4_dequant(weight.w.data_ptr(), weight.s.data_ptr(), weight.K, weight.N,
                                    out.data_ptr(), _stream(out)), "int4_dequant")
    return out


@dataclass(frozen=True)
class GemvPlan:
    """Launch shape of one GEMV: tiles per workgroup and the cross-workgroup K split."""

    tiles_per_workgroup: int
    ksplit: int
    groups_per_split: int
    workspace_bytes: int


_PLANS: dict[tuple, GemvPlan] = {}


def gemv_plan(rows: int, k: int, n: int, epilogue: int = N.EPI_STORE, target_waves: int = 2048) -> GemvPlan:
    """The library's launch shape for ``rows x K x N`` (cached per shape)."""
    key = (rows, k, n, epilogue, target_waves)
    if key not in _PLANS:
        nt, ks, gps, ws = C.c_int(), C.c_int(), C.c_int(), C.c_size_t()
        N.check(N.lib().df_int4_gemv_plan(rows, k, n, epilogue, target_waves, C.byref(nt), C.byref(ks),
                                          C.byref(gps), C.byref(ws)), "int4_gemv_plan")
        _PLANS[key] = GemvPlan(nt.value, ks.value, gps.value, ws.value)
    return _PLANS[key]


def int4_gemv(
    x: Tensor,
    weight: Int4Weight,
    *,
    prologue: int = N.PRO_NONE,
    epilogue: int = N.EPI_STORE,
    x2: Tensor | None = None,
    norm_w: Tensor | None = None,
    res: Tensor | None = None,
    eps: float = 1e-6,
    out: Tensor | None = None,
    h_out: Tensor | None = None,
    plan: GemvPlan | None = None,
    ws: Tensor | None = None,
) -> Tensor:
    """``x [rows, K] @ dequant(W) [K, N]`` with a fused prologue / epilogue (see the C header)."""
    if x.dim() != 2 or x.dtype != BF16:
        raise ValueError(f"x must be bf16 [rows, K], got {x.dtype} {tuple(x.shape)}")
    rows, k = x.shape
    if k != weight.K:
        raise ValueError(f"x has K={k}, weight has K={weight.K}")
    if not 1 <= rows <= 16:
        raise ValueError(f"int4_gemv handles 1..16 rows per launch, got {rows}")
    if x.stride(1) != 1 or x.stride(0) % 8:
        raise ValueError("x rows must be contiguous with a stride that is a multiple of 8")
    out_cols = weight.N // 2 if epilogue == N.EPI_SWIGLU else weight.N
    for name, t in (("x2", x2), ("res", res), ("norm_w", norm_w)):
        if t is not None and t.dtype != BF16:
            raise ValueError(f"{name} must be bf16, got {t.dtype}")
    require_gpu(x, "int4_gemv")
    if out is None:
        out = torch.empty((rows, out_cols), dtype=BF16, device=x.device)
    plan = plan if plan is not None else gemv_plan(rows, k, weight.N, epilogue)
    if ws is None and plan.workspace_bytes:
        ws = workspace(x.device, plan.workspace_bytes, "gemv")
    args = N.Int4GemvArgs(
        w=weight.w.data_ptr(), s=weight.s.data_ptr(), x=x.data_ptr(), x2=N.ptr(x2), norm_w=N.ptr(norm_w),
        res=N.ptr(res), out=out.data_ptr(), h_out=N.ptr(h_out), part=None,
        rows=rows, K=k, N=weight.N, ldx=x.stride(0), ldx2=x2.stride(0) if x2 is not None else 0,
        ldo=out.stride(0), tiles_per_workgroup=plan.tiles_per_workgroup, ksplit=plan.ksplit,
        groups_per_split=plan.groups_per_split, prologue=prologue, epilogue=epilogue, eps=eps,
    )
    N.check(N.lib().df_int4_gemv(C.byref(args), N.ptr(ws), ws.numel() if ws is not None else 0, _stream(x)),
            "int4_gemv")
    return out


# ---------------------------------------------------------------------------------------
# Gated DeltaNet step
# ---------------------------------------------------------------------------------------


def gated_delta_step(
    qkv: Tensor, a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Tensor, conv_w: Tensor, state: Tensor,
    *, num_k_heads: int, conv_in: Tensor | None = None, conv_out: Tensor | None = None,
    conv_ring: Tensor | None = None, position: Tensor | None = None, out: Tensor | None = None,
) -> Tensor:
    """One token of conv + L2-norm + gating + delta rule; ``state`` updated in place.

    ``qkv`` ``[B, C]`` pre-conv (rows may be strided), ``a``/``b`` ``[B, Hv]``, ``state``
    ``[B, Hv, 128, 128]`` fp32, ``conv_w`` ``[C, 4]`` (or ``[C, 1, 4]``). History: either
    ``conv_in``/``conv_out`` ``[B, C, 3]`` (reference layout) or ``conv_ring`` ``[B, C, 4]``
    with a device ``position``. Returns ``[B, Hv, 128]`` bf16.
    """
    if state.dim() != 4 or state.dtype != torch.float32:
        raise ValueError(
            f"the recurrent state is fp32 [B, Hv, Dk, Dv] by config (mamba_ssm_dtype), got "
            f"{state.dtype} {tuple(state.shape)}"
        )
    batch, hv, dk, dv = state.shape
    if dk != 128 or dv != 128:
        raise ValueError(f"this kernel is written for 128-wide heads, got Dk={dk} Dv={dv}")
    if hv % num_k_heads:
        raise ValueError(f"{hv} value heads do not divide into {num_k_heads} key heads")
    channels = 2 * num_k_heads * dk + hv * dv
    if qkv.dim() != 2 or qkv.shape[0] != batch or qkv.shape[1] < channels or qkv.stride(1) != 1:
        raise ValueError(f"qkv must be [B={batch}, >= {channels}] with unit column stride, got {tuple(qkv.shape)}")
    for name, t in (("a", a), ("b", b)):
        if t.dim() != 2 or t.shape[0] != batch or t.shape[1] < hv or t.stride(1) != 1:
            raise ValueError(f"{name} must be [B, >= {hv}], got {tuple(t.shape)}")
    if a.stride(0) != b.stride(0):
        raise ValueError("a and b must share a row stride")
    conv_w = conv_w.reshape(conv_w.shape[0], -1)
    if tuple(conv_w.shape) != (channels, 4):
        raise ValueError(f"conv weight must be [{channels}, 4] taps, got {tuple(conv_w.shape)}")
    op = "gated_delta_step"
    # the kernel reads every one of these as bf16 (A_log too: the reference model is cast to
    # bf16 as a whole, model.py:98); an fp32 tensor would be misread, not rejected, on the GPU
    for name, t in (("qkv", qkv), ("a", a), ("b", b), ("conv_w", conv_w)):
        _check_dtype(op, name, t, BF16)
    _check_dtype(op, "A_log", A_log, BF16, hv)
    _check_dtype(op, "dt_bias", dt_bias, BF16, hv)
    if not state.is_contiguous():
        raise ValueError("state must be contiguous (it is updated in place)")
    mode = 1 if conv_ring is not None else 0
    if mode == 0:
        if conv_in is None or conv_out is None or tuple(conv_in.shape) != (batch, channels, 3) \
                or tuple(conv_out.shape) != (batch, channels, 3):
            raise ValueError(f"conv history must be [B, {channels}, 3] in and out")
        if not conv_in.is_contiguous() or not conv_out.is_contiguous():
            raise ValueError("conv history must be contiguous")
        _check_dtype(op, "conv_in", conv_in, BF16)
        _check_dtype(op, "conv_out", conv_out, BF16)
    else:
        if position is None or tuple(conv_ring.shape) != (batch, channels, 4) or not conv_ring.is_contiguous():
            raise ValueError(f"conv ring must be a contiguous [B, {channels}, 4] with a device position")
        _check_dtype(op, "conv_ring", conv_ring, BF16)
        _check_dtype(op, "position", position, torch.int32, 1)
    if out is not None and (out.dtype != BF16 or tuple(out.shape) != (batch, hv, dv) or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous bf16 [{batch}, {hv}, {dv}]")
    require_gpus(op, state, qkv, a, b, A_log, dt_bias, conv_w, conv_in, conv_out, conv_ring, position, out)
    if out is None:
        out = torch.empty((batch, hv, dv), dtype=BF16, device=state.device)
    args = N.GatedDeltaArgs(
        qkv=qkv.data_ptr(), a=a.data_ptr(), b=b.data_ptr(), A_log=A_log.data_ptr(), dt_bias=dt_bias.data_ptr(),
        conv_w=conv_w.contiguous().data_ptr(), conv_in=N.ptr(conv_in), conv_out=N.ptr(conv_out),
        conv_ring=N.ptr(conv_ring), position=N.ptr(position), state=state.data_ptr(), out=out.data_ptr(),
        batch=batch, ld_qkv=qkv.stride(0), ld_ab=a.stride(0), num_k_heads=num_k_heads, num_v_heads=hv,
        head_k_dim=dk, head_v_dim=dv, conv_mode=mode,
    )
    N.check(N.lib().df_gated_delta_step(C.byref(args), _stream(state)), "gated_delta_step")
    return out


def delta_rule_step(state: Tensor, query: Tensor, key: Tensor, value: Tensor, g: Tensor, beta: Tensor,
                    *, state_out: Tensor | None = None, out: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """One delta-rule step on normalised fp32 inputs; returns ``(out, new_state)``.

    The contract of the reference's ``deltaforge::delta_rule_step``
    (kernels/gated_delta_step.py:109-186) and its checks in the same order: ``state``
    ``(B, H, Dk, Dv)`` fp32, ``query``/``key`` ``(B, H, Dk)`` (already l2-normed, the query
    already scaled by ``Dk**-0.5``), ``value (B, H, Dv)``, ``g``/``beta`` ``(B, H)``. The
    kernel is written for Dk = 128 and Dv a multiple of 32. ``state_out`` may be ``state``
    itself (an in-place step).
    """
    if state.dim() != 4:
        raise ValueError(f"expected state (batch, heads, key_dim, value_dim), got {tuple(state.shape)}")
    batch, heads, key_dim, value_dim = state.shape
    for name, t, shape in (("query", query, (batch, heads, key_dim)), ("key", key, (batch, heads, key_dim)),
                           ("value", value, (batch, heads, value_dim)), ("g", g, (batch, heads)),
                           ("beta", beta, (batch, heads))):
        if tuple(t.shape) != shape:
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {shape}")
    if state.dtype != torch.float32:
        raise ValueError(f"the recurrent state is fp32 by config (mamba_ssm_dtype), got {state.dtype}")
    if key_dim != 128 or value_dim < 32 or value_dim % 32:
        raise ValueError(f"the HIP step is written for key_dim 128 and value_dim % 32 == 0, got {key_dim}, {value_dim}")
    for name, t in (("state_out", state_out), ("out", out)):
        if t is not None and (t.dtype != torch.float32 or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous fp32 tensor")
    if state_out is not None and state_out.shape != state.shape:
        raise ValueError(f"state_out {tuple(state_out.shape)} must match state {tuple(state.shape)}")
    if out is not None and tuple(out.shape) != (batch, heads, value_dim):
        raise ValueError(f"out must be ({batch}, {heads}, {value_dim})")
    require_gpus("delta_rule_step", state, query, key, value, g, beta, state_out, out)
    state = state.contiguous()
    query, key, value, g, beta = (t.contiguous().float() for t in (query, key, value, g, beta))
    if state_out is None:
        state_out = torch.empty_like(state)
    if out is None:
        out = torch.empty((batch, heads, value_dim), dtype=torch.float32, device=state.device)
    args = N.DeltaRuleArgs(
        state_in=state.data_ptr(), state_out=state_out.data_ptr(), query=query.data_ptr(), key=key.data_ptr(),
        value=value.data_ptr(), g=g.data_ptr(), beta=beta.data_ptr(), out=out.data_ptr(),
        batch=batch, heads=heads, key_dim=key_dim, value_dim=value_dim,
    )
    N.check(N.lib().df_delta_rule_step(C.byref(args), _stream(state)), "delta_rule_step")
    return out, state_out


def delta_step_inputs(mixed: Tensor, a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Tensor, *, num_k_heads: int,
                      head_v_dim: int, eps: float = 1e-6) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """``delta_rule_step``'s ``(query, key, value, g, beta)`` from one token of Gated DeltaNet.

    ``mixed [B, C]`` is the conv + SiLU output (q | k | v, bf16), ``a``/``b`` ``[B, Hv]`` the
    gate projections (bf16 rows), ``A_log``/``dt_bias`` ``[Hv]`` bf16. The reference's
    prologue around its standalone step (kernels/gated_delta_step.py:189-213, 245-256): q and k
    L2-normed in fp32 and repeated from key heads to value heads, q scaled by ``Dk**-0.5``,
    ``beta = bf16(sigmoid(b))``, ``g = -exp(A_log) softplus(a + dt_bias)``; all fp32."""
    if mixed.dim() != 2 or a.dim() != 2 or b.dim() != 2:
        raise ValueError("mixed, a and b must be 2-D [B, ...] rows")
    batch = mixed.shape[0]
    hv = A_log.numel()
    if hv < 1 or hv % num_k_heads or dt_bias.numel() != hv:
        raise ValueError(f"{hv} value heads do not split over {num_k_heads} key heads (dt_bias {dt_bias.numel()})")
    channels = 2 * num_k_heads * 128 + hv * head_v_dim
    if mixed.shape[1] != channels:
        raise ValueError(f"mixed must be [B, {channels}] for 128-wide key heads, got {tuple(mixed.shape)}")
    for name, t in (("a", a), ("b", b)):
        if t.shape[0] != batch or t.shape[1] < hv:
            raise ValueError(f"{name} must be [{batch}, >= {hv}], got {tuple(t.shape)}")
    for name, t in (("mixed", mixed), ("a", a), ("b", b), ("A_log", A_log), ("dt_bias", dt_bias)):
        _check_dtype("delta_step_inputs", name, t, BF16)
    if a.stride(0) != b.stride(0) or a.stride(1) != 1 or b.stride(1) != 1 or mixed.stride(1) != 1:
        raise ValueError("a and b must be rows of one stride, and every row contiguous")
    require_gpus("delta_step_inputs", mixed, a, b, A_log, dt_bias)
    f32 = dict(dtype=torch.float32, device=mixed.device)
    query = torch.empty((batch, hv, 128), **f32)
    key = torch.empty((batch, hv, 128), **f32)
    value = torch.empty((batch, hv, head_v_dim), **f32)
    g = torch.empty((batch, hv), **f32)
    beta = torch.empty((batch, hv), **f32)
    args = N.DeltaInputsArgs(
        mixed=mixed.data_ptr(), a=a.data_ptr(), b=b.data_ptr(), A_log=A_log.contiguous().data_ptr(),
        dt_bias=dt_bias.contiguous().data_ptr(), query=query.data_ptr(), key=key.data_ptr(), value=value.data_ptr(),
        g=g.data_ptr(), beta=beta.data_ptr(), ld_mixed=mixed.stride(0), ld_ab=a.stride(0), batch=batch,
        num_k_heads=num_k_heads, num_v_heads=hv, head_k_dim=128, head_v_dim=head_v_dim, eps=eps,
    )
    N.check(N.lib().df_delta_step_inputs(C.byref(args), _stream(mixed)), "delta_step_inputs")
    return query, key, value, g, beta


# ---------------------------------------------------------------------------------------
# Attention decode
# ---------------------------------------------------------------------------------------


def split_kv_decode_attention(query: Tensor, key: Tensor, value: Tensor, scale: float, splits: int,
                              *, out: Tensor | None = None, ws: Tensor | None = None) -> Tensor:
    """Single-token GQA attention over a whole cache with the scan split ``splits`` ways.

    The contract of the reference's ``deltaforge::split_kv_decode_attention``
    (kernels/flash_decode_splitkv.py:177-261), checks in its order: ``query (B, Hq, D)``,
    ``key``/``value`` ``(B, Hkv, L, D)``, output ``(B, Hq, D)`` in the query's dtype. The HIP
    kernel takes bf16 with D = 256 and 4 query heads per KV head.
    """
    if query.dim() != 3:
        raise ValueError(f"expected query (batch, heads_q, head_dim), got {tuple(query.shape)}")
    if key.shape != value.shape:
        raise ValueError(f"key {tuple(key.shape)} and value {tuple(value.shape)} must match")
    batch, heads_q, head_dim = query.shape
    if key.dim() != 4:
        raise ValueError(f"expected key (batch, heads_kv, key_len, head_dim), got {tuple(key.shape)}")
    kv_batch, heads_kv, key_len, kv_dim = key.shape
    if kv_batch != batch or kv_dim != head_dim:
        raise ValueError(f"key {tuple(key.shape)} does not match query {tuple(query.shape)}")
    if heads_kv == 0 or heads_q % heads_kv:
        raise ValueError(f"{heads_q} query heads do not divide into {heads_kv} KV heads")
    if key_len < 1:
        raise ValueError("cannot attend over an empty KV cache")
    if splits < 1 or splits & (splits - 1):
        raise ValueError(f"splits must be a power of two so the merge can index it, got {splits}")
    if splits > 256:
        raise ValueError(f"the HIP merge takes at most 256 splits, got {splits}")
    if query.dtype != BF16 or key.dtype != BF16 or value.dtype != BF16:
        raise ValueError("the HIP split-KV kernel takes bf16 query, key and value")
    if head_dim != 256 or heads_q != 4 * heads_kv:
        raise ValueError(f"written for head_dim 256 and 4 query heads per KV head, got {head_dim}, {heads_q}/{heads_kv}")
    if out is not None and (out.shape != query.shape or out.dtype != BF16 or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous bf16 {tuple(query.shape)}")
    nbytes = int(N.lib().df_attention_decode_workspace_bytes(batch, heads_q, heads_kv, head_dim, splits))
    if ws is not None and ws.numel() < nbytes:
        raise ValueError(f"workspace holds {ws.numel()} bytes, the launch needs {nbytes}")
    require_gpus("split_kv_decode_attention", query, key, value, out, ws)
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if ws is None:
        ws = workspace(query.device, nbytes, "split_kv")
    if out is None:
        out = torch.empty_like(query)
    N.check(N.lib().df_split_kv_decode_attention(query.data_ptr(), key.data_ptr(), value.data_ptr(), batch, heads_q,
                                                 heads_kv, key_len, head_dim, float(scale), splits, out.data_ptr(),
                                                 ws.data_ptr(), ws.numel(), _stream(query)),
            "split_kv_decode_attention")
    return out


def attention_splits(batch: int, num_kv_heads: int, max_keys: int) -> int:
    return int(N.lib().df_attention_decode_splits(batch, num_kv_heads, max_keys))


def attention_decode(
    q: Tensor, k: Tensor, v: Tensor, q_norm_w: Tensor, k_norm_w: Tensor, inv_freq: Tensor,
    k_cache: Tensor, v_cache: Tensor, position: Tensor, *, num_q_heads: int, splits: int | None = None,
    gate: int = 0, eps: float = 1e-6, out: Tensor | None = None, ws: Tensor | None = None,
) -> Tensor:
    """Gated GQA decode for one new token per sequence (see the C header).

    ``q`` ``[B, >= Hq*2D]`` (per head ``[query | gate]``), ``k``/``v`` ``[B, >= Hkv*D]`` sharing
    one row stride, caches ``[B, Hkv, max_len, D]``; ``position`` is a device int32
    scalar (tokens already cached). Returns ``[B, Hq*D]`` bf16.
    """
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.dtype != BF16:
        raise ValueError("k_cache and v_cache must be matching bf16 [B, Hkv, max_len, D]")
    batch, hkv, max_len, d = k_cache.shape
    if d != 256 or num_q_heads != 4 * hkv:
        raise ValueError(f"written for head_dim 256 and 4 query heads per KV head, got D={d} Hq={num_q_heads}")
    for name, t, width in (("q", q, num_q_heads * 2 * d), ("k", k, hkv * d), ("v", v, hkv * d)):
        if t.dim() != 2 or t.shape[0] != batch or t.shape[1] < width or t.stride(1) != 1 or t.dtype != BF16:
            raise ValueError(f"{name} must be bf16 [B, >= {width}], got {t.dtype} {tuple(t.shape)}")
    if k.stride(0) != v.stride(0) or q.stride(0) % 4 or k.stride(0) % 4:
        raise ValueError("k and v must share a row stride; strides must be multiples of 4")
    if position.dtype != torch.int32 or position.numel() != 1:
        raise ValueError("position must be a single int32 device scalar")
    if inv_freq.dtype != torch.float32:
        raise ValueError("inv_freq must be fp32 (the values the model stores)")
    half = inv_freq.numel()
    # each lane finds its rotary partner half/4 lanes away with an xor shuffle, which is the
    # lane + half/4 only when half/4 is a power of two (8, 16, ..., 256 rotary dims)
    if half < 4 or half * 2 > d or half & (half - 1):
        raise ValueError(f"rotary_dim = 2 * inv_freq.numel() must be a power of two in [8, {d}], got {2 * half}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("k_cache and v_cache must be contiguous (the new key is written in place)")
    for name, t in (("q_norm_w", q_norm_w), ("k_norm_w", k_norm_w)):
        if t.dtype != BF16 or t.numel() != d or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous bf16 [{d}], got {t.dtype} {tuple(t.shape)}")
    if out is not None and (out.dtype != BF16 or tuple(out.shape) != (batch, num_q_heads * d) or out.stride(1) != 1
                            or out.stride(0) != num_q_heads * d):
        raise ValueError(f"out must be a contiguous bf16 [{batch}, {num_q_heads * d}]")
    if splits is None:
        splits = attention_splits(batch, hkv, max_len)
    nbytes = int(N.lib().df_attention_decode_workspace_bytes(batch, num_q_heads, hkv, d, splits))
    if ws is not None and ws.numel() < nbytes:
        raise ValueError(f"workspace holds {ws.numel()} bytes, the launch needs {nbytes}")
    require_gpus("attention_decode", q, k, v, q_norm_w, k_norm_w, inv_freq, k_cache, v_cache, position, out, ws)
    if ws is None:
        ws = workspace(q.device, nbytes, "attention")
    if out is None:
        out = torch.empty((batch, num_q_heads * d), dtype=BF16, device=q.device)
    args = N.AttnDecodeArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), q_norm_w=q_norm_w.data_ptr(), k_norm_w=k_norm_w.data_ptr(),
        inv_freq=inv_freq.data_ptr(), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(),
        position=position.data_ptr(), out=out.data_ptr(), batch=batch, ld_q=q.stride(0), ld_kv=k.stride(0),
        num_q_heads=num_q_heads, num_kv_heads=hkv, head_dim=d, rotary_dim=2 * inv_freq.numel(),
        max_len=max_len, splits=splits, gate=gate, eps=eps,
    )
    N.check(N.lib().df_attention_decode(C.byref(args), ws.data_ptr(), ws.numel(), _stream(q)), "attention_decode")
    return out


# ---------------------------------------------------------------------------------------
# Elementwise ops and decode glue
# ---------------------------------------------------------------------------------------


def _rows(x: Tensor, w: Tensor, op: str) -> tuple[int, int]:
    if w.dim() != 1 or x.shape[-1] != w.shape[0]:
        raise ValueError(f"{op}: weight has {w.shape[0]} elements, row is {x.shape[-1]}")
    if x.dtype != BF16 or w.dtype != BF16:
        raise ValueError(f"{op}: expected bf16 activations and weight")
    return x.numel() // x.shape[-1], x.shape[-1]


def rms_norm(x: Tensor, weight: Tensor, eps: float, out: Tensor | None = None) -> Tensor:
    rows, n = _rows(x, weight, "rms_norm")
    require_gpu(x, "rms_norm")
    x = x.contiguous()
    out = torch.empty_like(x) if out is None else out
    N.check(N.lib().df_rms_norm(x.data_ptr(), weight.contiguous().data_ptr(), eps, rows, n, out.data_ptr(),
                                _stream(x)), "rms_norm")
    return out


def add_rms_norm(x: Tensor, residual: Tensor, weight: Tensor, eps: float) -> tuple[Tensor, Tensor]:
    rows, n = _rows(x, weight, "add_rms_norm")
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError(f"residual {tuple(residual.shape)} must match activation {tuple(x.shape)}")
    require_gpu(x, "add_rms_norm")
    x, residual = x.contiguous(), residual.contiguous()
    resid_out, out = torch.empty_like(x), torch.empty_like(x)
    N.check(N.lib().df_add_rms_norm(x.data_ptr(), residual.data_ptr(), weight.contiguous().data_ptr(), eps, rows, n,
                                    resid_out.data_ptr(), out.data_ptr(), _stream(x)), "add_rms_norm")
    return resid_out, out


def silu_mul(gate: Tensor, up: Tensor) -> Tensor:
    if gate.shape != up.shape or gate.dtype != up.dtype or gate.dtype != BF16:
        raise ValueError("gate and up must be bf16 tensors of one shape")
    require_gpu(gate, "silu_mul")
    gate, up = gate.contiguous(), up.contiguous()
    out = torch.empty_like(up)
    N.check(N.lib().df_silu_mul(gate.data_ptr(), up.data_ptr(), out.numel(), out.data_ptr(), _stream(up)),
            "silu_mul")
    return out


def partial_rope(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``x`` ``[B, H, S, D]``, ``cos``/``sin`` ``[B, S, R]`` (reference.py:137-149)."""
    if x.dim() != 4 or cos.dim() != 3 or cos.shape != sin.shape:
        raise ValueError("expected x [B, H, S, D] and cos/sin [B, S, R]")
    batch, heads, seq, d = x.shape
    if cos.shape[0] != batch or cos.shape[1] != seq or cos.shape[2] > d or cos.shape[2] % 2:
        raise ValueError(f"cos {tuple(cos.shape)} does not fit x {tuple(x.shape)}")
    if x.dtype != BF16 or cos.dtype != BF16:
        raise ValueError("partial_rope runs the reference's bf16 op chain; pass bf16")
    require_gpu(x, "partial_rope")
    x, cos, sin = x.contiguous(), cos.contiguous(), sin.contiguous()
    out = torch.empty_like(x)
    N.check(N.lib().df_partial_rope(x.data_ptr(), cos.data_ptr(), sin.data_ptr(), batch, heads, seq, d,
                                    cos.shape[2], out.data_ptr(), _stream(x)), "partial_rope")
    return out


def causal_conv_step(x: Tensor, conv_cache: Tensor, weight: Tensor) -> Tensor:
    """``x`` ``[B, C, 1]``, history ``[B, C, 3]`` advanced in place, weight ``[C, 1, 4]``."""
    if x.dim() != 3 or x.shape[-1] != 1:
        raise ValueError(f"causal_conv_step is the decode step; got x {tuple(x.shape)}")
    batch, channels, _ = x.shape
    if tuple(conv_cache.shape) != (batch, channels, 3):
        raise ValueError(f"expected a (B, C, 3) history, got {tuple(conv_cache.shape)}")
    if weight.numel() != channels * 4:
        raise ValueError("this is the 4-tap case")
    if not conv_cache.is_contiguous():
        raise ValueError("conv history must be contiguous (updated in place)")
    require_gpu(x, "causal_conv_step")
    x = x.contiguous()
    out = torch.empty_like(x)
    N.check(N.lib().df_causal_conv_step(x.data_ptr(), conv_cache.data_ptr(), weight.contiguous().data_ptr(), batch,
                                        channels, out.data_ptr(), _stream(x)), "causal_conv_step")
    return out


def embed_int4(tokens: Tensor, head: Int4Weight, out: Tensor | None = None, *,
               prompt: Tensor | None = None, position: Tensor | None = None) -> Tensor:
    """Tied embedding rows from the int4 head: ``[B, hidden]`` bf16 for ``tokens`` ``[B]`` int64,
    or, with ``prompt`` ``[B, P]`` int64 and a device ``position``, for ``prompt[:, position]``."""
    if tokens.dtype != torch.int64 or tokens.dim() != 1:
        raise ValueError("tokens must be int64 [B]")
    if prompt is not None and (prompt.dtype != torch.int64 or prompt.dim() != 2 or position is None
                               or not prompt.is_contiguous() or prompt.shape[0] != tokens.numel()):
        raise ValueError("prompt must be contiguous int64 [B, P] with a device position")
    require_gpu(tokens, "embed_int4")
    if out is None:
        out = torch.empty((tokens.numel(), head.K), dtype=BF16, device=tokens.device)
    plen = prompt.shape[1] if prompt is not None else 0
    N.check(N.lib().df_embed_int4(tokens.data_ptr(), N.ptr(prompt), plen, N.ptr(position), tokens.numel(),
                                  head.w.data_ptr(), head.s.data_ptr(), head.K, head.N, out.data_ptr(),
                                  _stream(tokens)), "embed_int4")
    return out


def embed_bf16(tokens: Tensor, table: Tensor, out: Tensor | None = None, *,
               prompt: Tensor | None = None, position: Tensor | None = None) -> Tensor:
    """Embedding rows of a bf16 ``[vocab, hidden]`` table (reference.py:804), selected as in
    ``embed_int4``: for checkpoints whose table is not the dequantised int4 head."""
    if tokens.dtype != torch.int64 or tokens.dim() != 1:
        raise ValueError("tokens must be int64 [B]")
    if table.dim() != 2 or table.dtype != BF16 or not table.is_contiguous() or table.shape[1] % 8:
        raise ValueError(f"table must be a contiguous bf16 [vocab, hidden % 8 == 0], got {table.dtype} "
                         f"{tuple(table.shape)}")
    if prompt is not None and (prompt.dtype != torch.int64 or prompt.dim() != 2 or position is None
                               or not prompt.is_contiguous() or prompt.shape[0] != tokens.numel()):
        raise ValueError("prompt must be contiguous int64 [B, P] with a device position")
    vocab, hidden = table.shape
    if out is not None and (out.dtype != BF16 or tuple(out.shape) != (tokens.numel(), hidden)
                            or not out.is_contiguous()):
        raise ValueError(f"out must be a contiguous bf16 [{tokens.numel()}, {hidden}]")
    require_gpus("embed_bf16", tokens, table, prompt, position, out)
    if out is None:
        out = torch.empty((tokens.numel(), hidden), dtype=BF16, device=tokens.device)
    plen = prompt.shape[1] if prompt is not None else 0
    N.check(N.lib().df_embed_bf16(tokens.data_ptr(), N.ptr(prompt), plen, N.ptr(position), tokens.numel(),
                                  table.data_ptr(), hidden, vocab, out.data_ptr(), _stream(tokens)), "embed_bf16")
    return out


def argmax_tokens(logits: Tensor, tokens: Tensor, *, token_log: Tensor | None = None,
                  position: Tensor | None = None, advance: int = 0, step: Tensor | None = None,
                  ws: Tensor | None = None) -> Tensor:
    """First-max argmax of each bf16 row into ``tokens`` (int64), with decode-loop bookkeeping."""
    if logits.dim() != 2 or logits.dtype != BF16 or not logits.is_contiguous():
        raise ValueError("logits must be contiguous bf16 [rows, vocab]")
    rows, n = logits.shape
    require_gpu(logits, "argmax")
    nbytes = int(N.lib().df_argmax_workspace_bytes(rows, n))
    if ws is None:
        ws = workspace(logits.device, nbytes, "argmax")
    N.check(N.lib().df_argmax(logits.data_ptr(), rows, n, tokens.data_ptr(), N.ptr(token_log),
                              token_log.stride(0) if token_log is not None else 0, N.ptr(position), advance,
                              N.ptr(step), ws.data_ptr(), ws.numel(), _stream(logits)), "argmax")
    return tokens
