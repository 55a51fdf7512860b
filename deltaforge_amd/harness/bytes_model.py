"""Algorithmic bytes per call: the numerator of every GB/s and roofline figure.

Counts what the computation must move at least once (weights and scales read, recurrent
state read and written, KV read and the new KV written, inputs and outputs), following the
reference's byte model (harness/bytes_model.py:97-147) restated for the int4 format:
an int4 group-128 ``[K, N]`` weight is ``K*N/2`` bytes of nibbles plus ``(K/128)*N`` bf16
scales.
"""

from __future__ import annotations

from ..config import FULL_ATTENTION, LINEAR_ATTENTION, ModelConfig, qwen3_5_4b_config

__all__ = [
    "HBM_PEAK_BYTES_PER_S",
    "attention_bytes",
    "decode_bytes_per_token",
    "delta_bytes",
    "head_bytes",
    "int4_bytes",
    "linear_weight_bytes",
    "mean_decode_bytes",
    "mlp_bytes",
]

HBM_PEAK_BYTES_PER_S = 8.0e12  # MI355X HBM3E


def int4_bytes(k: int, n: int) -> int:
    return k * n // 2 + (k // 128) * n * 2


def head_bytes(hidden: int = 2560, vocab: int = 248320, rows: int = 1) -> int:
    """Config 1: nibbles + scales + x, residual, norm weight + logits (328,294,400 at bs=1)."""
    return int4_bytes(hidden, vocab) + rows * 2 * hidden * 2 + hidden * 2 + rows * vocab * 2


def delta_bytes(batch: int = 1, num_k_heads: int = 16, num_v_heads: int = 32, dk: int = 128) -> int:
    """Config 2: per batch row state r/w, qkv in, conv history r/w, out, a/b; plus conv weights."""
    channels = 2 * num_k_heads * dk + num_v_heads * dk
    per_row = (num_v_heads * dk * dk * 4 * 2 + channels * 2 + channels * 3 * 2 * 2 + num_v_heads * dk * 2
               + num_v_heads * 2 * 2)
    return batch * per_row + channels * 4 * 2


def attention_bytes(batch: int = 1, context: int = 4096, num_q_heads: int = 16, num_kv_heads: int = 4,
                    head_dim: int = 256) -> int:
    """Config 3: KV read for context+1 keys, new K/V written, q|gate + k + v in, out, norm weights."""
    kv_per_key = num_kv_heads * head_dim * 2 * 2
    inputs = (2 * num_q_heads + 2 * num_kv_heads) * head_dim * 2
    return batch * (kv_per_key * (context + 1) + kv_per_key + inputs + num_q_heads * head_dim * 2) + 2 * head_dim * 2


def mlp_bytes(rows: int = 1, hidden: int = 2560, inter: int = 9216) -> int:
    """Config 4: gate+up+down nibbles and scales, norm weight, x in and out."""
    return 2 * int4_bytes(hidden, inter) + int4_bytes(inter, hidden) + hidden * 2 + rows * hidden * 2 * 2


def linear_weight_bytes(c: ModelConfig) -> int:
    total = 0
    for kind in c.layer_types:
        if kind == FULL_ATTENTION:
            total += int4_bytes(c.hidden_size, 2 * c.num_attention_heads * c.head_dim)
            total += 2 * int4_bytes(c.hidden_size, c.num_key_value_heads * c.head_dim)
            total += int4_bytes(c.num_attention_heads * c.head_dim, c.hidden_size)
        else:
            total += int4_bytes(c.hidden_size, c.linear_conv_dim) + int4_bytes(c.hidden_size, c.linear_value_dim)
            total += 2 * int4_bytes(c.hidden_size, c.linear_num_value_heads)
            total += int4_bytes(c.linear_value_dim, c.hidden_size)
        total += 2 * int4_bytes(c.hidden_size, c.intermediate_size) + int4_bytes(c.intermediate_size, c.hidden_size)
    return total


def decode_bytes_per_token(c: ModelConfig | None = None, position: int = 4096, batch: int = 1) -> dict[str, int]:
    """Config 5 bytes for the token at ``position`` (it attends ``position + 1`` keys)."""
    c = c or qwen3_5_4b_config()
    n_lin = len(c.layer_indices(LINEAR_ATTENTION))
    n_full = len(c.layer_indices(FULL_ATTENTION))
    small = (c.num_hidden_layers * 2 * c.hidden_size * 2 + c.hidden_size * 2
             + n_lin * (c.linear_conv_dim * c.linear_conv_kernel_dim * 2 + c.linear_num_value_heads * 2 * 2
                        + c.linear_value_head_dim * 2)
             + n_full * 2 * c.head_dim * 2)
    kv_per_key = n_full * c.num_key_value_heads * c.head_dim * 2 * 2
    parts = {
        "linears": linear_weight_bytes(c),
        "head": int4_bytes(c.hidden_size, c.vocab_size),
        "norms_conv_gates": small,
        "embed_row": batch * c.hidden_size * 2,
        "recurrent_state": batch * n_lin * c.linear_num_value_heads * c.linear_key_head_dim
        * c.linear_value_head_dim * 4 * 2,
        "conv_state": batch * n_lin * c.linear_conv_dim * (c.linear_conv_kernel_dim - 1) * 2 * 2,
        "kv_read": batch * kv_per_key * (position + 1),
        "kv_write": batch * kv_per_key,
    }
    parts["total"] = sum(parts.values())
    return parts


def mean_decode_bytes(c: ModelConfig | None = None, start: int = 4096, steps: int = 256, batch: int = 1) -> float:
    """Mean bytes per token over ``steps`` greedy tokens starting at ``start``."""
    return sum(decode_bytes_per_token(c, start + i, batch)["total"] for i in range(steps)) / steps
