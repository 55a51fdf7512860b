"""Per-config CPU oracles (configs 1-4 of the benchmark), composed from ``oracle.model``. TEST ONLY.

Each function is the reference's own composition for that slice of the decode step, with
the reference's rounding points (pinned through ``oracle.model`` by the golden vectors):

* ``head``       reference.py:730-735 (residual add), 810 (final RMSNorm), 764-777 (head)
                 with the int4 champion expression (kernels/visible_int4_head.py:187-199).
* ``mlp_block``  reference.py:732-735 and 692-693 with int4 linears.
* ``delta_step`` reference.py:496-545 at seq_len 1 (conv, split, gates, repeat_interleave,
                 delta rule) -- the part between the projections and the GatedRMSNorm.
* ``attention_decode`` reference.py:621-676 at seq_len 1 between the projections and
                 o_proj (q/gate split, q/k norm, partial RoPE, cache write, GQA
                 expansion, bf16 scores, fp32 softmax, bf16 PV, output gate).
* ``decode_attention`` the attention core of the same lines (gqa_decode.py:322-335), the
                 contract of deltaforge::split_kv_decode_attention.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from deltaforge_amd.config import ModelConfig

from .int4 import dequant_gemv
from .model import apply_partial_rope, causal_conv, gated_delta_rule, output_gate, rms_norm, rope_cos_sin

__all__ = ["attention_decode", "decode_attention", "delta_step", "head", "mlp_block"]


def head(x, residual, norm_w, packed, scale, group=128, eps=1e-6):
    h = residual + x
    return dequant_gemv(rms_norm(h, norm_w, eps), packed, scale, group)


def mlp_block(x, norm_w, gate, up, down, eps=1e-6):
    """``x + down(silu(gate(n)) * up(n))`` with ``n = rms_norm(x)``; weights are (packed, scale)."""
    n = rms_norm(x, norm_w, eps)
    g = dequant_gemv(n, *gate, 128)
    u = dequant_gemv(n, *up, 128)
    return x + dequant_gemv(F.silu(g) * u, *down, 128)


def delta_step(qkv, conv_state, conv_w, a, b, A_log, dt_bias, state, num_k_heads, head_dim=128):
    """Returns ``(out [B, Hv, Dv] bf16, new_state fp32, new_conv_state [B, C, 3])``."""
    batch, channels = qkv.shape
    hv = a.shape[1]
    key_dim = num_k_heads * head_dim
    mixed, new_hist = causal_conv(qkv.unsqueeze(-1), conv_state, conv_w)
    mixed = mixed.transpose(1, 2)  # [B, 1, C]
    q, k, v = torch.split(mixed, [key_dim, key_dim, hv * head_dim], dim=-1)
    q = q.reshape(batch, 1, num_k_heads, head_dim)
    k = k.reshape(batch, 1, num_k_heads, head_dim)
    v = v.reshape(batch, 1, hv, head_dim)
    beta = b.unsqueeze(1).sigmoid()
    g = -A_log.float().exp() * F.softplus(a.unsqueeze(1).float() + dt_bias.float())
    groups = hv // num_k_heads
    if groups > 1:
        q = q.repeat_interleave(groups, dim=2)
        k = k.repeat_interleave(groups, dim=2)
    out, new_state = gated_delta_rule(q, k, v, g, beta, state)
    return out[:, 0], new_state, new_hist


def attention_decode(q_proj, k_raw, v_raw, q_norm_w, k_norm_w, k_cache, v_cache, position: int,
                     config: ModelConfig):
    """One new token per sequence at ``position``; caches updated in place. Returns ``[B, Hq*D]``."""
    c = config
    batch = q_proj.shape[0]
    d = c.head_dim
    proj = q_proj.reshape(batch, 1, c.num_attention_heads, 2 * d)
    query, gate = torch.chunk(proj, 2, dim=-1)
    gate = gate.reshape(batch, 1, -1)
    query = rms_norm(query, q_norm_w, c.rms_norm_eps).transpose(1, 2)
    key = rms_norm(k_raw.reshape(batch, 1, c.num_key_value_heads, d), k_norm_w, c.rms_norm_eps).transpose(1, 2)
    value = v_raw.reshape(batch, 1, c.num_key_value_heads, d).transpose(1, 2)
    positions = torch.full((batch, 1), position, dtype=torch.long)
    cos, sin = rope_cos_sin(positions, c, q_proj.dtype, inv_freq_dtype=q_proj.dtype)
    query = apply_partial_rope(query, cos, sin)
    key = apply_partial_rope(key, cos, sin)
    end = position + 1
    k_cache[:, :, position:end] = key
    v_cache[:, :, position:end] = value
    attn = decode_attention(query[:, :, 0], k_cache[:, :, :end], v_cache[:, :, :end], d ** -0.5)
    attn = attn.unsqueeze(1).reshape(batch, 1, -1)
    return (attn * output_gate(gate, c.output_gate_type)).reshape(batch, -1)


def decode_attention(query, key, value, scale):
    """Single-token GQA attention as the reference's layer computes it, expansion and all
    (reference.py:652-672; restated as gqa_decode.py:322-335 for the split-KV op's check):
    ``query (B, Hq, D)``, ``key``/``value`` ``(B, Hkv, L, D)``: bf16 scores, fp32 softmax
    rounded to the query dtype, bf16 PV. Returns ``(B, Hq, D)``."""
    groups = query.shape[1] // key.shape[1]
    outs = []
    for bi in range(query.shape[0]):  # one sequence at a time keeps the GQA expansion small
        kk = key[bi:bi + 1].repeat_interleave(groups, dim=1)
        vv = value[bi:bi + 1].repeat_interleave(groups, dim=1)
        scores = torch.matmul(query[bi:bi + 1].unsqueeze(2), kk.transpose(2, 3)) * scale
        weights = F.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype)
        outs.append(torch.matmul(weights, vv).squeeze(2))
    return torch.cat(outs, dim=0)
