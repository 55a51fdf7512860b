"""Functional CPU restatement of the reference decode model. TEST ONLY.

Each function follows ``/root/reference/src/deltaforge/reference.py`` operation for
operation (same dtypes, same rounding points, same op order), so that on the CPU it is
bit-identical to the reference on the same inputs; ``tests/golden`` holds vectors written
by the reference itself that pin this. Parameters live in a flat dict keyed by the
reference's ``state_dict`` names. A linear whose name is in ``OracleModel.int4`` runs the
int4 champion expression (``oracle.int4.dequant_gemv``) instead of ``F.linear``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

from deltaforge_amd.config import FULL_ATTENTION, LINEAR_ATTENTION, SIGMOID_GATE, ModelConfig

from .int4 import dequant_gemv

__all__ = [
    "OracleCache",
    "OracleModel",
    "apply_partial_rope",
    "causal_conv",
    "delta_rule_step",
    "gated_delta_rule",
    "gated_rms_norm",
    "l2norm",
    "output_gate",
    "rms_norm",
    "rope_cos_sin",
    "rotate_half",
]


# -- elementwise / normalisation ----------------------------------------------------------


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm with the zero-centred ``(1 + weight)`` scale (reference.py:92-96)."""
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    h = h * (1.0 + weight.float())
    return h.type_as(x)


def gated_rms_norm(x: torch.Tensor, gate: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """Norm first, then ``weight`` (plain), then the SiLU gate (reference.py:115-121)."""
    dtype = x.dtype
    h = x.float()
    h = h * torch.rsqrt(h.pow(2).mean(-1, keepdim=True) + eps)
    h = weight * h.to(dtype)
    h = h * F.silu(gate.float())
    return h.to(dtype)


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """``[-x2, x1]`` over the last axis (reference.py:132-134)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_partial_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate the leading ``cos.shape[-1]`` dims of ``(B, H, S, D)`` (reference.py:137-149)."""
    cos = cos.unsqueeze(1)
    sin = sin.unsqueeze(1)
    width = cos.shape[-1]
    rot, tail = x[..., :width], x[..., width:]
    return torch.cat((rot * cos + rotate_half(rot) * sin, tail), dim=-1)


def rope_cos_sin(
    position_ids: torch.Tensor, config: ModelConfig, dtype: torch.dtype,
    inv_freq_dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Text-only mRoPE, which is standard RoPE at the token position (reference.py:165-200).

    With the three mRoPE rows equal, the interleave picks every band from identical rows, so
    the result is ``freqs[0]``; the golden vectors pin this against the reference's own
    interleaving code.

    ``inv_freq_dtype``: ``inv_freq`` is a module buffer, so the reference's
    ``ReferenceModel(...).to(dtype=bfloat16)`` (model.py:83-105) stores it rounded to bf16;
    the angles are then ``position * bf16(inv_freq)`` in fp32. The decode model passes its
    parameter dtype here to reproduce that.
    """
    rotary = config.rotary_dim
    inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, rotary, 2, dtype=torch.float32) / rotary))
    inv_freq = inv_freq.to(inv_freq_dtype)
    freqs = position_ids.float().unsqueeze(-1) * inv_freq.to(position_ids.device)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def output_gate(gate: torch.Tensor, kind: str) -> torch.Tensor:
    """Attention output gate nonlinearity in fp32, cast back (reference.py:558-568)."""
    if kind == SIGMOID_GATE:
        return torch.sigmoid(gate.float()).to(gate.dtype)
    return F.silu(gate.float()).to(gate.dtype)


def l2norm(x: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """reference.py:403-404."""
    return x * torch.rsqrt((x * x).sum(dim=-1, keepdim=True) + eps)


# -- Gated DeltaNet -------------------------------------------------------------------------


def gated_delta_rule(query, key, value, g, beta, initial_state=None):
    """The sequential delta rule, token by token, fp32 (reference.py:407-461).

    ``query``/``key`` ``(B, S, H, Dk)`` already expanded to value heads, ``value``
    ``(B, S, H, Dv)``, ``g``/``beta`` ``(B, S, H)``. Returns ``(out (B, S, H, Dv), state)``.
    """
    in_dtype = query.dtype
    q, k, v, b, gg = (t.transpose(1, 2).to(torch.float32).contiguous() for t in (query, key, value, beta, g))
    q = l2norm(q)
    k = l2norm(k)
    q = q / math.sqrt(q.shape[-1])
    batch, heads, steps, dk = k.shape
    dv = v.shape[-1]
    if initial_state is None:
        state = torch.zeros((batch, heads, dk, dv), dtype=torch.float32)
    else:
        state = initial_state.to(torch.float32)
    out = torch.zeros_like(v)
    for t in range(steps):
        out[:, :, t], state = delta_rule_step(state, q[:, :, t], k[:, :, t], v[:, :, t], gg[:, :, t], b[:, :, t])
    return out.transpose(1, 2).contiguous().to(in_dtype), state


def delta_rule_step(state, q, k, v, g, beta):
    """One token of the rule on normalised fp32 inputs (the loop body of reference.py:450-458;
    the contract of deltaforge::delta_rule_step, kernels/gated_delta_step.py:109-186):
    ``state (B, H, Dk, Dv)``, ``q``/``k`` ``(B, H, Dk)``, ``v (B, H, Dv)``, ``g``/``beta``
    ``(B, H)``. Returns ``(out (B, H, Dv), new_state)``."""
    state = state * g.exp()[..., None, None]
    recalled = (state * k.unsqueeze(-1)).sum(dim=-2)
    delta = (v - recalled) * beta.unsqueeze(-1)
    state = state + k.unsqueeze(-1) * delta.unsqueeze(-2)
    return (state * q.unsqueeze(-1)).sum(dim=-2), state


def causal_conv(x: torch.Tensor, history: torch.Tensor | None, weight: torch.Tensor):
    """Depthwise causal conv over ``(B, C, S)`` with a ``(B, C, taps-1)`` history.

    Reference.py:496-510: prepend the history, ``F.conv1d`` (grouped), SiLU. Returns
    ``(silu(conv), new_history)``.
    """
    taps = weight.shape[-1]
    keep = taps - 1
    prefix = history if history is not None else x.new_zeros((x.shape[0], x.shape[1], keep))
    full = torch.cat((prefix.to(x.dtype), x), dim=-1)
    out = F.conv1d(full, weight, groups=x.shape[1])
    return F.silu(out), full[..., -keep:]


# -- cache ----------------------------------------------------------------------------------


@dataclass
class OracleCache:
    """KV for attention layers, conv history + fp32 state for linear layers (reference.py:241-395)."""

    config: ModelConfig
    batch: int
    max_seq_len: int
    dtype: torch.dtype = torch.bfloat16
    seq_len: int = 0
    layers: list = field(default_factory=list)

    def __post_init__(self) -> None:
        c = self.config
        for kind in c.layer_types:
            if kind == FULL_ATTENTION:
                shape = (self.batch, c.num_key_value_heads, self.max_seq_len, c.head_dim)
                self.layers.append({"keys": torch.zeros(shape, dtype=self.dtype),
                                    "values": torch.zeros(shape, dtype=self.dtype)})
            else:
                self.layers.append({
                    "conv": torch.zeros((self.batch, c.linear_conv_dim, c.linear_conv_kernel_dim - 1),
                                        dtype=self.dtype),
                    "recurrent": torch.zeros((self.batch, c.linear_num_value_heads, c.linear_key_head_dim,
                                              c.linear_value_head_dim), dtype=torch.float32),
                })

    def ensure_capacity(self, n: int) -> None:
        if self.seq_len + n > self.max_seq_len:
            raise ValueError(f"cache overflow: {self.seq_len} + {n} > {self.max_seq_len}")


# -- model ----------------------------------------------------------------------------------


class OracleModel:
    """The reference decoder as functions over a parameter dict (reference.py:701-817).

    ``params`` maps reference ``state_dict`` names to tensors. ``int4`` maps a linear's
    weight name to ``(packed, scale, group)``; those linears (and ``"lm_head"`` for the tied
    head) run the int4 champion expression.
    """

    def __init__(self, config: ModelConfig, params: dict, int4: dict | None = None, gemv=None) -> None:
        self.config = config
        self.params = params
        self.int4 = int4 or {}
        # the int4 linear's expression: the reference's unless a sensitivity probe swaps it
        self.gemv = gemv or dequant_gemv

    def new_cache(self, batch: int, max_seq_len: int) -> OracleCache:
        return OracleCache(self.config, batch, max_seq_len, dtype=self.params["embed_tokens.weight"].dtype)

    def linear(self, x: torch.Tensor, name: str) -> torch.Tensor:
        if name in self.int4:
            packed, scale, group = self.int4[name]
            return self.gemv(x, packed, scale, group)
        return F.linear(x, self.params[name])

    def project_logits(self, h: torch.Tensor) -> torch.Tensor:
        """reference.py:764-777 (tied head); the int4 head when quantised."""
        if "lm_head" in self.int4:
            packed, scale, group = self.int4["lm_head"]
            return self.gemv(h, packed, scale, group)
        return F.linear(h, self.params["embed_tokens.weight"].to(h.dtype))

    def _delta_net(self, i: int, h: torch.Tensor, cache: dict | None) -> torch.Tensor:
        c = self.config
        p = f"layers.{i}.linear_attn."
        batch, steps, _ = h.shape
        qkv = self.linear(h, p + "in_proj_qkv.weight").transpose(1, 2)
        mixed, new_hist = causal_conv(qkv, cache["conv"] if cache is not None else None,
                                      self.params[p + "conv1d.weight"])
        if cache is not None:
            cache["conv"].copy_(new_hist.to(cache["conv"].dtype))
        mixed = mixed.transpose(1, 2)
        q, k, v = torch.split(mixed, [c.linear_key_dim, c.linear_key_dim, c.linear_value_dim], dim=-1)
        q = q.reshape(batch, steps, c.linear_num_key_heads, c.linear_key_head_dim)
        k = k.reshape(batch, steps, c.linear_num_key_heads, c.linear_key_head_dim)
        v = v.reshape(batch, steps, c.linear_num_value_heads, c.linear_value_head_dim)
        z = self.linear(h, p + "in_proj_z.weight").reshape(
            batch, steps, c.linear_num_value_heads, c.linear_value_head_dim)
        beta = self.linear(h, p + "in_proj_b.weight").sigmoid()
        g = -self.params[p + "A_log"].float().exp() * F.softplus(
            self.linear(h, p + "in_proj_a.weight").float() + self.params[p + "dt_bias"].float())
        if c.linear_value_groups > 1:
            q = q.repeat_interleave(c.linear_value_groups, dim=2)
            k = k.repeat_interleave(c.linear_value_groups, dim=2)
        core, state = gated_delta_rule(q, k, v, g, beta, cache["recurrent"] if cache is not None else None)
        if cache is not None:
            cache["recurrent"].copy_(state)
        core = gated_rms_norm(core.reshape(-1, c.linear_value_head_dim),
                              z.reshape(-1, c.linear_value_head_dim),
                              self.params[p + "norm.weight"], c.rms_norm_eps)
        return self.linear(core.reshape(batch, steps, c.linear_value_dim), p + "out_proj.weight")

    def _attention(self, i, h, cos, sin, cache, offset):
        c = self.config
        p = f"layers.{i}.self_attn."
        batch, steps, _ = h.shape
        d = c.head_dim
        proj = self.linear(h, p + "q_proj.weight").view(batch, steps, c.num_attention_heads, 2 * d)
        query, gate = torch.chunk(proj, 2, dim=-1)
        gate = gate.reshape(batch, steps, -1)
        query = rms_norm(query, self.params[p + "q_norm.weight"], c.rms_norm_eps).transpose(1, 2)
        key = rms_norm(self.linear(h, p + "k_proj.weight").view(batch, steps, c.num_key_value_heads, d),
                       self.params[p + "k_norm.weight"], c.rms_norm_eps).transpose(1, 2)
        value = self.linear(h, p + "v_proj.weight").view(batch, steps, c.num_key_value_heads, d).transpose(1, 2)
        query = apply_partial_rope(query, cos, sin)
        key = apply_partial_rope(key, cos, sin)
        if cache is not None:
            end = offset + steps
            cache["keys"][:, :, offset:end] = key.to(cache["keys"].dtype)
            cache["values"][:, :, offset:end] = value.to(cache["values"].dtype)
            key = cache["keys"][:, :, :end]
            value = cache["values"][:, :, :end]
        groups = c.num_key_value_groups
        if groups > 1:
            key = key.repeat_interleave(groups, dim=1)
            value = value.repeat_interleave(groups, dim=1)
        scores = torch.matmul(query, key.transpose(2, 3)) * (d ** -0.5)
        if steps > 1:
            qpos = torch.arange(steps) + offset
            kpos = torch.arange(key.shape[2])
            scores = scores.masked_fill(kpos.unsqueeze(0) > qpos.unsqueeze(1), torch.finfo(scores.dtype).min)
        weights = F.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
        attn = torch.matmul(weights, value).transpose(1, 2).reshape(batch, steps, -1)
        attn = attn * output_gate(gate, c.output_gate_type)
        return self.linear(attn, p + "o_proj.weight")

    def _mlp(self, i, x):
        p = f"layers.{i}.mlp."
        return self.linear(F.silu(self.linear(x, p + "gate_proj.weight")) * self.linear(x, p + "up_proj.weight"),
                           p + "down_proj.weight")

    def forward(self, input_ids: torch.Tensor, cache: OracleCache | None = None,
                num_logits_to_keep: int = 0) -> torch.Tensor:
        """reference.py:779-817: returns logits; advances ``cache``."""
        c = self.config
        batch, steps = input_ids.shape
        offset = 0
        if cache is not None:
            cache.ensure_capacity(steps)
            offset = cache.seq_len
        positions = (torch.arange(steps) + offset).unsqueeze(0).expand(batch, -1)
        h = F.embedding(input_ids, self.params["embed_tokens.weight"])
        cos, sin = rope_cos_sin(positions, c, h.dtype, inv_freq_dtype=h.dtype)
        for i, kind in enumerate(c.layer_types):
            layer_cache = cache.layers[i] if cache is not None else None
            residual = h
            x = rms_norm(h, self.params[f"layers.{i}.input_layernorm.weight"], c.rms_norm_eps)
            if kind == LINEAR_ATTENTION:
                x = self._delta_net(i, x, layer_cache)
            else:
                x = self._attention(i, x, cos, sin, layer_cache, offset)
            h = residual + x
            residual = h
            x = rms_norm(h, self.params[f"layers.{i}.post_attention_layernorm.weight"], c.rms_norm_eps)
            h = residual + self._mlp(i, x)
        h = rms_norm(h, self.params["norm.weight"], c.rms_norm_eps)
        if num_logits_to_keep:
            h = h[:, -num_logits_to_keep:]
        logits = self.project_logits(h)
        if cache is not None:
            cache.seq_len += steps
        return logits

    @torch.no_grad()
    def greedy(self, prompt: torch.Tensor, new_tokens: int, cache: OracleCache | None = None):
        """``greedy_decode`` (reference model.py:108-148): returns ``(tokens, per-step logits)``."""
        if cache is None:
            cache = self.new_cache(prompt.shape[0], prompt.shape[1] + new_tokens)
        logits = self.forward(prompt, cache, num_logits_to_keep=1)
        token = logits[:, -1].argmax(dim=-1, keepdim=True)
        tokens, all_logits = [token], [logits[:, -1]]
        for _ in range(new_tokens - 1):
            logits = self.forward(token, cache, num_logits_to_keep=1)
            token = logits[:, -1].argmax(dim=-1, keepdim=True)
            tokens.append(token)
            all_logits.append(logits[:, -1])
        return torch.cat(tokens, dim=1), torch.stack(all_logits, dim=1)
