"""Seeded parameter sets for the golden vectors, keyed by the reference's state_dict names.

Frozen on purpose: ``make_golden.py`` loaded exactly these tensors into the reference's
``ReferenceModel`` (``load_state_dict(strict=True)``, which also proves the names and shapes
match the reference's) to write the vectors, and the tests regenerate them from the same
seed. Changing a draw here invalidates every stored vector; ``PARAM_CHECKSUMS`` in the
fixture guards against that silently happening.
"""

from __future__ import annotations

import math

import torch

from deltaforge_amd.config import FULL_ATTENTION, ModelConfig


def param_shapes(c: ModelConfig) -> list[tuple[str, tuple[int, ...], str]]:
    """``(name, shape, kind)`` in a fixed order. ``kind`` selects the draw."""
    out = [("embed_tokens.weight", (c.vocab_size, c.hidden_size), "embed")]
    for i, kind in enumerate(c.layer_types):
        p = f"layers.{i}."
        out.append((p + "input_layernorm.weight", (c.hidden_size,), "norm"))
        out.append((p + "post_attention_layernorm.weight", (c.hidden_size,), "norm"))
        if kind == FULL_ATTENTION:
            a = p + "self_attn."
            out += [
                (a + "q_proj.weight", (2 * c.num_attention_heads * c.head_dim, c.hidden_size), "linear"),
                (a + "k_proj.weight", (c.num_key_value_heads * c.head_dim, c.hidden_size), "linear"),
                (a + "v_proj.weight", (c.num_key_value_heads * c.head_dim, c.hidden_size), "linear"),
                (a + "o_proj.weight", (c.hidden_size, c.num_attention_heads * c.head_dim), "linear"),
                (a + "q_norm.weight", (c.head_dim,), "norm"),
                (a + "k_norm.weight", (c.head_dim,), "norm"),
            ]
        else:
            a = p + "linear_attn."
            out += [
                (a + "in_proj_qkv.weight", (c.linear_conv_dim, c.hidden_size), "linear"),
                (a + "in_proj_z.weight", (c.linear_value_dim, c.hidden_size), "linear"),
                (a + "in_proj_b.weight", (c.linear_num_value_heads, c.hidden_size), "linear"),
                (a + "in_proj_a.weight", (c.linear_num_value_heads, c.hidden_size), "linear"),
                (a + "conv1d.weight", (c.linear_conv_dim, 1, c.linear_conv_kernel_dim), "conv"),
                (a + "dt_bias", (c.linear_num_value_heads,), "gate_bias"),
                (a + "A_log", (c.linear_num_value_heads,), "gate_bias"),
                (a + "norm.weight", (c.linear_value_head_dim,), "gated_norm"),
                (a + "out_proj.weight", (c.hidden_size, c.linear_value_dim), "linear"),
            ]
        m = p + "mlp."
        out += [
            (m + "gate_proj.weight", (c.intermediate_size, c.hidden_size), "linear"),
            (m + "up_proj.weight", (c.intermediate_size, c.hidden_size), "linear"),
            (m + "down_proj.weight", (c.hidden_size, c.intermediate_size), "linear"),
        ]
    out.append(("norm.weight", (c.hidden_size,), "norm"))
    return out


def make_params(c: ModelConfig, seed: int) -> dict[str, torch.Tensor]:
    """bf16 parameters drawn in a fixed order from one CPU generator."""
    gen = torch.Generator().manual_seed(seed)
    params = {}
    for name, shape, kind in param_shapes(c):
        x = torch.randn(shape, generator=gen, dtype=torch.float32)
        if kind == "linear":
            x = x / math.sqrt(shape[1])
        elif kind == "norm":
            x = x * 0.1
        elif kind == "gated_norm":
            x = 1.0 + 0.1 * x
        elif kind == "conv":
            x = x * 0.3
        elif kind == "gate_bias":
            x = x * 0.5
        params[name] = x.to(torch.bfloat16)
    return params


def checksum(params: dict[str, torch.Tensor]) -> torch.Tensor:
    """float64 sum and sum of squares per tensor, in ``param_shapes`` order."""
    return torch.tensor([[float(t.double().sum()), float(t.double().pow(2).sum())] for t in params.values()],
                        dtype=torch.float64)
