"""Prompt prefill: the whole prompt through each layer in one pass, into a decoder's caches.

The reference fills its cache by running ``ReferenceModel.forward`` over the prompt
(reference.py:779-817). The projections are ``[P, K] x [K, N]`` products. Gated DeltaNet
convolves the sequence and runs the delta rule as a token-by-token scan
(reference.py:450-458). Attention is causal over the prompt. This module is that forward on
the HIP kernels of ``csrc/prefill.hip``:
- the int4 GEMM on MFMA, with gate/up's SwiGLU fused into its epilogue;
- the causal conv over the sequence;
- the chunked delta rule (64-token chunks, exact in real arithmetic to the scan);
- GatedRMSNorm over rows;
- q/k norm + RoPE, which also writes the KV cache;
- causal GQA attention with the reference's bf16 softmax rounding.

Then RMSNorm, the tied head and the argmax of the last position.

``Prefiller.fill(decoder, prompt)`` leaves a ``PersistentDecoder`` (``fill_engine`` a
``DecodeEngine``, one sequence per row) in the state its own token-by-token prefill would:
the conv rings, recurrent states and KV caches of every layer, the position, the last logits
and the first generated token. Summation order is the only difference. ``Prefiller`` keeps its own copy of the weights, in natural column order (the
persistent kernel's copy is permuted XCD-major).
"""

from __future__ import annotations

import ctypes as C

import torch
from torch import Tensor

from . import _native as N
from . import ops
from .config import FULL_ATTENTION, SIGMOID_GATE, ModelConfig
from .synth import SynthModel, inv_freq

__all__ = [
    "Prefiller",
    "attention_prefill",
    "causal_conv_prefill",
    "delta_rule_prefill",
    "gated_rms_norm_rows",
    "int4_gemm",
    "qk_norm_rope_prefill",
]

BF16 = torch.bfloat16


def _row_view(t: Tensor, what: str) -> int:
    """Row stride of a 2-D tensor whose rows are contiguous."""
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{what} must be a 2-D tensor with contiguous rows, got {tuple(t.shape)} {t.stride()}")
    return t.stride(0)


def int4_gemm(x: Tensor, weight: ops.Int4Weight, *, epilogue: int = N.EPI_STORE, out: Tensor | None = None) -> Tensor:
    """``bf16(x [M, K] @ bf16(dequant(W)))``; with ``EPI_SWIGLU`` the interleaved gate|up
    product becomes ``[M, N/2]`` of ``bf16(bf16(silu(gate)) * up)``."""
    if x.dtype != BF16 or x.dim() != 2 or x.shape[1] != weight.K:
        raise ValueError(f"x must be bf16 [M, {weight.K}], got {x.dtype} {tuple(x.shape)}")
    ldx = _row_view(x, "x")
    if ldx % 8 or x.data_ptr() % 16:
        raise ValueError("x rows must be 16-byte aligned")
    if epilogue not in (N.EPI_STORE, N.EPI_SWIGLU):
        raise ValueError("int4_gemm epilogues: EPI_STORE, EPI_SWIGLU")
    cols = weight.N // 2 if epilogue == N.EPI_SWIGLU else weight.N
    m = x.shape[0]
    if out is None:
        out = torch.empty((m, cols), dtype=BF16, device=x.device)
    elif out.dtype != BF16 or tuple(out.shape) != (m, cols) or out.stride(1) != 1:
        raise ValueError(f"out must be bf16 [{m}, {cols}] with contiguous rows")
    ops.require_gpus("int4_gemm", x, weight.w, weight.s, out)
    args = N.Int4GemmArgs(x=x.data_ptr(), w=weight.w.data_ptr(), s=weight.s.data_ptr(), out=out.data_ptr(),
                          M=m, K=weight.K, N=weight.N, ldx=ldx, ldo=out.stride(0), epilogue=epilogue)
    N.check(N.lib().df_int4_gemm(C.byref(args), ops._stream(x)), "int4_gemm")
    return out


def causal_conv_prefill(x: Tensor, weight: Tensor, ring: Tensor, *, pos0: int = 0, out: Tensor | None = None) -> Tensor:
    """Conv + SiLU over ``x`` ``[P, C]`` (rows may be strided) at positions ``pos0 ..``, history
    from and left in ``ring`` ``[C, 4]`` (slot = position mod 4)."""
    ldx = _row_view(x, "x")
    tokens, channels = x.shape
    weight = weight.reshape(channels, -1)
    if weight.shape[1] != 4 or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [C, 4] (4 taps)")
    if tuple(ring.shape) != (channels, 4) or not ring.is_contiguous():
        raise ValueError(f"ring must be a contiguous [{channels}, 4]")
    for name, t in (("x", x), ("weight", weight), ("ring", ring)):
        ops._check_dtype("causal_conv_prefill", name, t, BF16)
    if out is None:
        out = torch.empty((tokens, channels), dtype=BF16, device=x.device)
    ops.require_gpus("causal_conv_prefill", x, weight, ring, out)
    N.check(N.lib().df_causal_conv_prefill(x.data_ptr(), ldx, tokens, channels, weight.data_ptr(), ring.data_ptr(),
                                           pos0, out.data_ptr(), _row_view(out, "out"), ops._stream(x)),
            "causal_conv_prefill")
    return out


def delta_rule_prefill(mixed: Tensor, a: Tensor, b: Tensor, A_log: Tensor, dt_bias: Tensor, state: Tensor, *,
                       num_k_heads: int, out: Tensor | None = None) -> Tensor:
    """Chunked gated delta rule over ``mixed`` ``[P, q|k|v]`` (the conv output); ``a``, ``b``
    ``[P, >= Hv]`` raw gate projections (strided rows, one stride); ``state`` ``[Hv, 128, 128]``
    fp32 updated in place. Returns the core output ``[P, Hv * 128]`` bf16."""
    if state.dim() != 3 or state.dtype != torch.float32 or not state.is_contiguous() or state.shape[1:] != (128, 128):
        raise ValueError(f"state must be a contiguous fp32 [Hv, 128, 128], got {state.dtype} {tuple(state.shape)}")
    hv = state.shape[0]
    tokens = mixed.shape[0]
    if mixed.shape[1] != (2 * num_k_heads + hv) * 128:
        raise ValueError(f"mixed must be [P, {(2 * num_k_heads + hv) * 128}], got {tuple(mixed.shape)}")
    ld_ab = _row_view(a, "a")
    if _row_view(b, "b") != ld_ab or a.shape[0] != tokens or b.shape[0] != tokens or a.shape[1] < hv or b.shape[1] < hv:
        raise ValueError("a and b must be [P, >= Hv] sharing one row stride")
    op = "delta_rule_prefill"
    for name, t in (("mixed", mixed), ("a", a), ("b", b)):
        ops._check_dtype(op, name, t, BF16)
    ops._check_dtype(op, "A_log", A_log, BF16, hv)
    ops._check_dtype(op, "dt_bias", dt_bias, BF16, hv)
    if out is None:
        out = torch.empty((tokens, hv * 128), dtype=BF16, device=mixed.device)
    ops.require_gpus(op, mixed, a, b, A_log, dt_bias, state, out)
    nbytes = int(N.lib().df_delta_rule_prefill_workspace_bytes(tokens, hv))
    ws = ops.workspace(mixed.device, nbytes, "delta_prefill")
    args = N.DeltaPrefillArgs(mixed=mixed.data_ptr(), a=a.data_ptr(), b=b.data_ptr(), A_log=A_log.data_ptr(),
                              dt_bias=dt_bias.data_ptr(), state=state.data_ptr(), out=out.data_ptr(),
                              ld_mixed=_row_view(mixed, "mixed"), ld_ab=ld_ab, ld_out=_row_view(out, "out"),
                              tokens=tokens, num_k_heads=num_k_heads, num_v_heads=hv)
    N.check(N.lib().df_delta_rule_prefill(C.byref(args), ws.data_ptr(), ws.numel(), ops._stream(mixed)), op)
    return out


def gated_rms_norm_rows(x: Tensor, z: Tensor, weight: Tensor, eps: float, out: Tensor | None = None) -> Tensor:
    """GatedRMSNorm over each 128-wide head of ``x`` ``[P, H*128]`` with gate ``z`` (same shape,
    rows may be strided)."""
    tokens, width = x.shape
    if width % 128 or tuple(z.shape) != (tokens, width) or weight.numel() != 128:
        raise ValueError("x and z must be [P, H*128]; weight [128]")
    for name, t in (("x", x), ("z", z), ("weight", weight)):
        ops._check_dtype("gated_rms_norm_rows", name, t, BF16)
    if out is None:
        out = torch.empty((tokens, width), dtype=BF16, device=x.device)
    ops.require_gpus("gated_rms_norm_rows", x, z, weight, out)
    N.check(N.lib().df_gated_rms_norm_rows(x.data_ptr(), _row_view(x, "x"), z.data_ptr(), _row_view(z, "z"),
                                           weight.contiguous().data_ptr(), eps, tokens, width // 128, out.data_ptr(),
                                           _row_view(out, "out"), ops._stream(x)), "gated_rms_norm_rows")
    return out


def qk_norm_rope_prefill(proj: Tensor, q_norm: Tensor, k_norm: Tensor, inv: Tensor, k_cache: Tensor,
                         v_cache: Tensor, *, num_q_heads: int, k_col: int, v_col: int, pos0: int = 0,
                         eps: float = 1e-6, q_out: Tensor | None = None) -> Tensor:
    """Queries and keys of the attention projection rows normed and roped at positions
    ``pos0 ..``; keys and values written to the caches ``[Hkv, max_len, 256]``. Returns the
    queries ``[P, Hq, 256]``."""
    tokens = proj.shape[0]
    hkv, max_len, d = k_cache.shape
    if d != 256 or v_cache.shape != k_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous [Hkv, max_len, 256] of one shape")
    if pos0 < 0 or pos0 + tokens > max_len:
        raise ValueError(f"positions {pos0} .. {pos0 + tokens - 1} do not fit a cache of {max_len}")
    if inv.dtype != torch.float32:
        raise ValueError("inv_freq must be fp32")
    op = "qk_norm_rope_prefill"
    for name, t in (("proj", proj), ("q_norm", q_norm), ("k_norm", k_norm), ("k_cache", k_cache),
                    ("v_cache", v_cache)):
        ops._check_dtype(op, name, t, BF16)
    if q_out is None:
        q_out = torch.empty((tokens, num_q_heads, d), dtype=BF16, device=proj.device)
    ops.require_gpus(op, proj, q_norm, k_norm, inv, k_cache, v_cache, q_out)
    args = N.QkPrefillArgs(proj=proj.data_ptr(), q_norm=q_norm.data_ptr(), k_norm=k_norm.data_ptr(),
                           inv_freq=inv.data_ptr(), q_out=q_out.data_ptr(), k_cache=k_cache.data_ptr(),
                           v_cache=v_cache.data_ptr(), ld_proj=_row_view(proj, "proj"), k_col=k_col, v_col=v_col,
                           tokens=tokens, pos0=pos0, max_len=max_len, num_q_heads=num_q_heads, num_kv_heads=hkv,
                           rotary_dim=2 * inv.numel(), eps=eps)
    N.check(N.lib().df_qk_norm_rope_prefill(C.byref(args), ops._stream(proj)), op)
    return q_out


def attention_prefill(q: Tensor, k_cache: Tensor, v_cache: Tensor, gate: Tensor, *, gate_head_stride: int,
                      pos0: int = 0, gate_kind: int = 0, scale: float = 256 ** -0.5,
                      out: Tensor | None = None) -> Tensor:
    """Causal GQA attention of ``q`` ``[P, Hq, 256]`` (positions ``pos0 ..``) over the caches,
    times the output gate; ``gate`` ``[P, ...]`` holds head h's gate at column
    ``h * gate_head_stride``. Returns ``[P, Hq * 256]`` bf16."""
    tokens, hq, d = q.shape
    hkv, max_len, _ = k_cache.shape
    if d != 256 or hq != 4 * hkv or not q.is_contiguous():
        raise ValueError("q must be a contiguous [P, 4 Hkv, 256]")
    if v_cache.shape != k_cache.shape or not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous [Hkv, max_len, 256] of one shape")
    if pos0 < 0 or pos0 + tokens > max_len:
        raise ValueError(f"positions {pos0} .. {pos0 + tokens - 1} do not fit a cache of {max_len}")
    op = "attention_prefill"
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("gate", gate)):
        ops._check_dtype(op, name, t, BF16)
    # The kernel sees only pointers and row strides: every extent it reads or writes is
    # checked here, so a short gate or output becomes an error, not an access out of bounds.
    ld_gate = _row_view(gate, "gate")
    gate_cols = (hq - 1) * gate_head_stride + d
    if gate_head_stride < 0 or gate.shape[0] != tokens or gate.shape[1] < gate_cols:
        raise ValueError(f"gate must be [{tokens}, >= {gate_cols}] for {hq} heads at column stride "
                         f"{gate_head_stride}, got {tuple(gate.shape)}")
    if out is None:
        out = torch.empty((tokens, hq * d), dtype=BF16, device=q.device)
    ops._check_dtype(op, "out", out, BF16)
    ld_out = _row_view(out, "out")
    if out.shape[0] != tokens or out.shape[1] < hq * d:
        raise ValueError(f"out must be [{tokens}, >= {hq * d}], got {tuple(out.shape)}")
    ops.require_gpus(op, q, k_cache, v_cache, gate, out)
    args = N.AttnPrefillArgs(q=q.data_ptr(), k_cache=k_cache.data_ptr(), v_cache=v_cache.data_ptr(),
                             gate=gate.data_ptr(), out=out.data_ptr(), ld_gate=ld_gate,
                             gate_head_stride=gate_head_stride, ld_out=ld_out, tokens=tokens,
                             pos0=pos0, max_len=max_len, num_q_heads=hq, num_kv_heads=hkv, gate_kind=gate_kind,
                             scale=scale)
    N.check(N.lib().df_attention_prefill(C.byref(args), ops._stream(q)), op)
    return out


def unsupported_geometry(c: ModelConfig) -> str | None:
    """Why the prefill kernels cannot run model ``c``, or ``None`` when they can: 256-wide
    attention heads, four query heads per KV head, 128-wide Gated DeltaNet heads with a 4-tap
    conv, every projection's K a multiple of 256 and N of 16, a power-of-two rotary half."""
    half = c.rotary_dim // 2
    if c.head_dim != 256 or c.num_attention_heads != 4 * c.num_key_value_heads:
        return "attention needs head_dim 256 and four query heads per KV head"
    if c.linear_key_head_dim != 128 or c.linear_value_head_dim != 128 or c.linear_conv_kernel_dim != 4:
        return "Gated DeltaNet needs 128-wide heads and a 4-tap conv"
    if c.linear_num_value_heads % c.linear_num_key_heads:
        return "value heads must be a multiple of key heads"
    if half < 4 or half & (half - 1) or c.rotary_dim > c.head_dim:
        return f"rotary dim {c.rotary_dim} is not twice a power of two of at least 4"
    for k in (c.hidden_size, c.intermediate_size, c.linear_value_dim, c.num_attention_heads * c.head_dim):
        if k % 256:
            return f"a projection has K = {k}, not a multiple of 256"
    if c.vocab_size % 16 or c.intermediate_size % 16:
        return "a projection's N is not a multiple of 16"
    return None


class Prefiller:
    """The model's weights in natural column order, and the forward over a prompt."""

    def __init__(self, model: SynthModel, device: str | torch.device = "cuda") -> None:
        c: ModelConfig = model.config
        self.config = c
        self.device = dev = torch.device(device)
        ops.require_gpu(torch.empty(0, device=dev), "prefill")
        p = {k: v.to(dev) for k, v in model.params.items()}
        lin = model.linears

        def repack(names: list[str]) -> ops.Int4Weight:
            packed = torch.cat([lin[n].packed for n in names], 1).to(dev)
            scale = torch.cat([lin[n].scale for n in names], 1).to(dev)
            return ops.int4_repack(packed, scale)

        self.layers: list[dict] = []
        for i, kind in enumerate(c.layer_types):
            pre = f"layers.{i}."
            gp, gs = ops.interleave_gate_up(lin[pre + "mlp.gate_proj.weight"].packed, lin[pre + "mlp.gate_proj.weight"].scale,
                                            lin[pre + "mlp.up_proj.weight"].packed, lin[pre + "mlp.up_proj.weight"].scale)
            layer = {"kind": kind, "in_norm": p[pre + "input_layernorm.weight"],
                     "post_norm": p[pre + "post_attention_layernorm.weight"],
                     "gate_up": ops.int4_repack(gp.to(dev), gs.to(dev)),
                     "down": repack([pre + "mlp.down_proj.weight"])}
            if kind == FULL_ATTENTION:
                a = pre + "self_attn."
                layer["proj"] = repack([a + "q_proj.weight", a + "k_proj.weight", a + "v_proj.weight"])
                layer["out"] = repack([a + "o_proj.weight"])
                layer["q_norm"], layer["k_norm"] = p[a + "q_norm.weight"], p[a + "k_norm.weight"]
            else:
                a = pre + "linear_attn."
                layer["proj"] = repack([a + "in_proj_qkv.weight", a + "in_proj_z.weight", a + "in_proj_a.weight",
                                        a + "in_proj_b.weight"])
                layer["out"] = repack([a + "out_proj.weight"])
                layer["conv_w"] = p[a + "conv1d.weight"].reshape(c.linear_conv_dim, -1).contiguous()
                layer["A_log"], layer["dt_bias"] = p[a + "A_log"], p[a + "dt_bias"]
                layer["gnorm_w"] = p[a + "norm.weight"]
            self.layers.append(layer)
        self.head = ops.int4_repack(lin["lm_head"].packed.to(dev), lin["lm_head"].scale.to(dev))
        self.final_norm = p["norm.weight"]
        self.embed_table = p.get("embed_tokens.weight")
        self.inv_freq = inv_freq(c).to(dev)

    def forward(self, prompt: Tensor, caches: list[dict], *, pos0: int = 0) -> Tensor:
        """Run ``prompt`` ``[P]`` (int64, on the device) through every layer from position
        ``pos0``, updating ``caches`` (per layer: ``conv_ring`` ``[C, 4]`` and ``state``
        ``[Hv, 128, 128]``, or ``k_cache``/``v_cache`` ``[Hkv, max_len, 256]``). Returns the
        last position's logits ``[1, vocab]`` bf16."""
        c = self.config
        if prompt.dim() != 1 or prompt.dtype != torch.int64 or prompt.numel() < 1:
            raise ValueError("prompt must be a non-empty int64 [P]")
        eps = c.rms_norm_eps
        if self.embed_table is not None:
            h = ops.embed_bf16(prompt, self.embed_table)
        else:
            h = ops.embed_int4(prompt, self.head)
        x = ops.rms_norm(h, self.layers[0]["in_norm"], eps)
        conv_c, vd, hv = c.linear_conv_dim, c.linear_value_dim, c.linear_num_value_heads
        qd, kvd = 2 * c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
        gate_kind = 0 if c.output_gate_type == SIGMOID_GATE else 1
        for i, (layer, cache) in enumerate(zip(self.layers, caches)):
            proj = int4_gemm(x, layer["proj"])
            if layer["kind"] == FULL_ATTENTION:
                q = qk_norm_rope_prefill(proj, layer["q_norm"], layer["k_norm"], self.inv_freq, cache["k_cache"],
                                         cache["v_cache"], num_q_heads=c.num_attention_heads, k_col=qd,
                                         v_col=qd + kvd, pos0=pos0, eps=eps)
                attn = attention_prefill(q, cache["k_cache"], cache["v_cache"], proj[:, c.head_dim:],
                                         gate_head_stride=2 * c.head_dim, pos0=pos0, gate_kind=gate_kind,
                                         scale=c.head_dim ** -0.5)
                o = int4_gemm(attn, layer["out"])
            else:
                mixed = causal_conv_prefill(proj[:, :conv_c], layer["conv_w"], cache["conv_ring"], pos0=pos0)
                core = delta_rule_prefill(mixed, proj[:, conv_c + vd:], proj[:, conv_c + vd + hv:], layer["A_log"],
                                          layer["dt_bias"], cache["state"], num_k_heads=c.linear_num_key_heads)
                y = gated_rms_norm_rows(core, proj[:, conv_c:conv_c + vd], layer["gnorm_w"], eps)
                o = int4_gemm(y, layer["out"])
            h, x = ops.add_rms_norm(o, h, layer["post_norm"], eps)
            act = int4_gemm(x, layer["gate_up"], epilogue=N.EPI_SWIGLU)
            d = int4_gemm(act, layer["down"])
            nxt = self.layers[i + 1]["in_norm"] if i + 1 < len(self.layers) else self.final_norm
            h, x = ops.add_rms_norm(d, h, nxt, eps)
        return ops.int4_gemv(x[-1:], self.head)

    def fill(self, decoder, prompt: Tensor, *, chunk: int = 16384) -> None:
        """Prefill a ``PersistentDecoder`` (fresh or reset) with ``prompt`` ``[1, P]``: its caches,
        position, last logits and first generated token, as its own ``prefill`` leaves them.

        The prompt runs through ``forward`` ``chunk`` tokens at a time (positions continue from
        the caches), which bounds the activations and the conv kernel's grid (at most 65 535
        rows). ``chunk`` is a multiple of the delta rule's 64-token chunk, so the chunks are the
        ones a single pass would form and the result is the same."""
        plen = self._check_prompt(decoder, prompt, chunk, rows=1)
        decoder.reset()
        ids = prompt[0].to(self.device, torch.int64).contiguous()
        decoder.prompt[:plen].copy_(ids)
        decoder.prompt_len = plen
        decoder.logits.copy_(self._run(ids, decoder.layer_state, chunk))
        ops.argmax_tokens(decoder.logits, decoder.tokens)
        decoder.position.fill_(plen)
        decoder.step_index.zero_()

    def fill_engine(self, engine, prompt: Tensor, *, chunk: int = 16384) -> None:
        """Prefill a ``DecodeEngine`` with ``prompt`` ``[B, P]``, one sequence per engine row:
        every layer's caches, the position, the last logits and the first generated token, as
        the engine's teacher-forced ``prefill`` leaves them (summation order aside)."""
        plen = self._check_prompt(engine, prompt, chunk, rows=engine.batch)
        engine.reset()
        engine.set_prompt(prompt)
        for row in range(engine.batch):
            ids = engine.prompt[row].contiguous()
            engine.logits[row:row + 1].copy_(self._run(ids, engine.row_caches(row), chunk))
        engine.finish_fill(plen)
        ops.argmax_tokens(engine.logits, engine.tokens)

    def _check_prompt(self, decoder, prompt: Tensor, chunk: int, *, rows: int) -> int:
        if prompt.dim() != 2 or prompt.shape[0] != rows:
            raise ValueError(f"prompt must be [{rows}, P], got {tuple(prompt.shape)}")
        if chunk < 64 or chunk % 64 or chunk > 65535:
            raise ValueError("chunk must be a multiple of 64 below 65536")
        plen = prompt.shape[1]
        if plen < 1:
            raise ValueError("prompt must hold at least one token")
        if plen + decoder.max_new_tokens > decoder.max_seq_len:
            raise ValueError("prompt + max_new_tokens exceeds the cache")
        # The embedding kernels skip an id outside the table and leave its row unwritten, so
        # the ids are checked here, once, before anything runs (an index error, as the
        # reference's embedding lookup raises).
        lo, hi = int(prompt.min()), int(prompt.max())
        if lo < 0 or hi >= self.config.vocab_size:
            raise ValueError(f"token ids must lie in [0, {self.config.vocab_size}), got {lo} .. {hi}")
        return plen

    def _run(self, ids: Tensor, caches: list[dict], chunk: int) -> Tensor:
        """``ids`` through ``forward`` ``chunk`` tokens at a time; the last position's logits."""
        for s in range(0, ids.numel(), chunk):
            logits = self.forward(ids[s:s + chunk], caches, pos0=s)
        return logits
