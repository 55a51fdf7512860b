"""Seeded synthetic inputs for the five benchmark configurations (all drawn on the CPU).

Draw order is fixed per config so a seed names exactly one input set. Int4 weights are
drawn directly in the canonical K-major interchange format (reference
kernels/tiled_gemv.py:242-278): nibbles uniform over 0..15 (zero point 8, so -8 occurs),
bf16 scales |N(0,1)| * 0.02 per 128-group. RMSNorm weights are stored zero-centred
(w ~ N(0, 0.02), effective scale 1 + w), which is how the reference applies them
(reference.py:79-96).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .config import FULL_ATTENTION, ModelConfig, qwen3_5_4b_config

BF16 = torch.bfloat16

__all__ = [
    "CanonicalInt4",
    "SynthModel",
    "attention_inputs",
    "delta_inputs",
    "head_inputs",
    "inv_freq",
    "mlp_inputs",
    "synth_model",
]


@dataclass
class CanonicalInt4:
    """K-major packed nibbles ``[K/2, N]`` uint8 and bf16 scales ``[K/128, N]``."""

    packed: torch.Tensor
    scale: torch.Tensor

    @property
    def K(self) -> int:
        return self.packed.shape[0] * 2

    @property
    def N(self) -> int:
        return self.packed.shape[1]

    @property
    def group(self) -> int:
        return self.K // self.scale.shape[0]


def draw_int4(gen: torch.Generator, k: int, n: int, scale_std: float = 0.02, symmetric: bool = False) -> CanonicalInt4:
    """Uniform bytes (two uniform nibbles each), drawn as 32-bit words for speed.

    ``symmetric`` maps nibble 0 to 8, so ``n - 8`` lies in -7..7 with mean 0, the range of the
    reference's symmetric quantiser (kernels/tiled_gemv.py:242-278). The default keeps
    BASELINE's uniform 0..15, whose ``n - 8`` has mean -1/2."""
    nbytes = (k // 2) * n
    words = torch.randint(-(2**31), 2**31 - 1, ((nbytes + 3) // 4,), generator=gen, dtype=torch.int32)
    packed = words.view(torch.uint8)[:nbytes].reshape(k // 2, n)
    if symmetric:
        lo, hi = packed & 0x0F, packed >> 4
        lo = torch.where(lo == 0, 8, lo)
        hi = torch.where(hi == 0, 8, hi)
        packed = (lo | (hi << 4)).to(torch.uint8)
    scale = (torch.randn((k // 128, n), generator=gen).abs() * scale_std).to(BF16)
    return CanonicalInt4(packed, scale)


def _normal(gen, shape, std=1.0, mean=0.0, dtype=BF16):
    return (torch.randn(shape, generator=gen) * std + mean).to(dtype)


def inv_freq(config: ModelConfig, dtype: torch.dtype = BF16) -> torch.Tensor:
    """RoPE inverse frequencies as the bf16 model stores them, returned as fp32.

    Same expression as the reference (reference.py:170-173); the module buffer is cast
    with the model (``.to(dtype=bf16)``, model.py:83-105), so its values are bf16-rounded.
    """
    r = config.rotary_dim
    f = 1.0 / (config.rope_theta ** (torch.arange(0, r, 2, dtype=torch.float32) / r))
    return f.to(dtype).float()


# -- config 1: tied int4 head with final residual + RMSNorm ----------------------------------


def head_inputs(seed: int = 0, hidden: int = 2560, vocab: int = 248320, rows: int = 1):
    gen = torch.Generator().manual_seed(seed)
    weight = draw_int4(gen, hidden, vocab)
    x = _normal(gen, (rows, hidden))
    residual = _normal(gen, (rows, hidden))
    norm_w = _normal(gen, (hidden,), 0.02)
    return {"weight": weight, "x": x, "residual": residual, "norm_w": norm_w, "eps": 1e-6}


# -- config 2: gated-delta decode step ---------------------------------------------------------


def delta_inputs(seed: int = 0, batch: int = 1, num_k_heads: int = 16, num_v_heads: int = 32, dk: int = 128):
    gen = torch.Generator().manual_seed(seed)
    channels = 2 * num_k_heads * dk + num_v_heads * dk
    return {
        "state": _normal(gen, (batch, num_v_heads, dk, dk), 0.1, dtype=torch.float32),
        "qkv": _normal(gen, (batch, channels)),
        "conv_state": _normal(gen, (batch, channels, 3)),
        "conv_w": _normal(gen, (channels, 1, 4), 0.3),
        "a": _normal(gen, (batch, num_v_heads)),
        "b": _normal(gen, (batch, num_v_heads)),
        "A_log": torch.zeros(num_v_heads, dtype=BF16),
        "dt_bias": torch.zeros(num_v_heads, dtype=BF16),
        "num_k_heads": num_k_heads,
    }


# -- config 3: split-KV GQA decode ------------------------------------------------------------


def attention_inputs(seed: int = 0, batch: int = 1, context: int = 4096, num_q_heads: int = 16,
                     num_kv_heads: int = 4, head_dim: int = 256, slack: int = 64):
    """``context`` keys already cached; the new token sits at position ``context``."""
    gen = torch.Generator().manual_seed(seed)
    max_len = context + slack
    k_cache = torch.zeros((batch, num_kv_heads, max_len, head_dim), dtype=BF16)
    v_cache = torch.zeros_like(k_cache)
    k_cache[:, :, :context] = _normal(gen, (batch, num_kv_heads, context, head_dim))
    v_cache[:, :, :context] = _normal(gen, (batch, num_kv_heads, context, head_dim))
    return {
        "q": _normal(gen, (batch, num_q_heads * 2 * head_dim)),  # per head [query | gate]
        "k": _normal(gen, (batch, num_kv_heads * head_dim)),
        "v": _normal(gen, (batch, num_kv_heads * head_dim)),
        "q_norm_w": _normal(gen, (head_dim,), 0.02),
        "k_norm_w": _normal(gen, (head_dim,), 0.02),
        "k_cache": k_cache,
        "v_cache": v_cache,
        "position": context,
    }


# -- config 4: int4 MLP block -----------------------------------------------------------------


def mlp_inputs(seed: int = 0, rows: int = 1, hidden: int = 2560, inter: int = 9216):
    gen = torch.Generator().manual_seed(seed)
    return {
        "gate": draw_int4(gen, hidden, inter),
        "up": draw_int4(gen, hidden, inter),
        "down": draw_int4(gen, inter, hidden),
        "norm_w": _normal(gen, (hidden,), 0.02),
        "x": _normal(gen, (rows, hidden)),
        "eps": 1e-6,
    }


# -- config 5: the whole hybrid model ---------------------------------------------------------


@dataclass
class SynthModel:
    """A random-init int4 model: canonical int4 linears plus bf16 small parameters.

    ``linears`` maps reference weight names (``layers.{i}.mlp.gate_proj.weight`` ...) and
    ``"lm_head"`` to ``CanonicalInt4`` ``[K = in_features, N = out_features]``. ``params``
    holds the bf16 norms, conv weights, A_log and dt_bias under reference names. The
    embedding is tied to the head: its bf16 table is the dequantised head.
    """

    config: ModelConfig
    linears: dict = field(default_factory=dict)
    params: dict = field(default_factory=dict)

    def nbytes(self) -> int:
        total = sum(w.packed.numel() + 2 * w.scale.numel() for w in self.linears.values())
        return total + sum(p.numel() * p.element_size() for p in self.params.values())


def linear_shapes(c: ModelConfig) -> list[tuple[str, int, int]]:
    """``(name, K, N)`` of every linear, in a fixed order (reference.py:477-494, 591-605, 688-690)."""
    out = []
    for i, kind in enumerate(c.layer_types):
        p = f"layers.{i}."
        if kind == FULL_ATTENTION:
            a = p + "self_attn."
            out += [(a + "q_proj.weight", c.hidden_size, 2 * c.num_attention_heads * c.head_dim),
                    (a + "k_proj.weight", c.hidden_size, c.num_key_value_heads * c.head_dim),
                    (a + "v_proj.weight", c.hidden_size, c.num_key_value_heads * c.head_dim),
                    (a + "o_proj.weight", c.num_attention_heads * c.head_dim, c.hidden_size)]
        else:
            a = p + "linear_attn."
            out += [(a + "in_proj_qkv.weight", c.hidden_size, c.linear_conv_dim),
                    (a + "in_proj_z.weight", c.hidden_size, c.linear_value_dim),
                    (a + "in_proj_b.weight", c.hidden_size, c.linear_num_value_heads),
                    (a + "in_proj_a.weight", c.hidden_size, c.linear_num_value_heads),
                    (a + "out_proj.weight", c.linear_value_dim, c.hidden_size)]
        m = p + "mlp."
        out += [(m + "gate_proj.weight", c.hidden_size, c.intermediate_size),
                (m + "up_proj.weight", c.hidden_size, c.intermediate_size),
                (m + "down_proj.weight", c.intermediate_size, c.hidden_size)]
    out.append(("lm_head", c.hidden_size, c.vocab_size))
    return out


def synth_model(config: ModelConfig | None = None, seed: int = 0, symmetric: bool = False) -> SynthModel:
    """The seeded random-init model; the benchmark uses the defaults (BASELINE's draws).

    BASELINE's nibbles (uniform 0..15, zero point 8) give every int4 output a bias of
    -s/2 * sum(x), which 32 residual layers grow into a constant vector that fixes the argmax
    whatever the input. ``symmetric=True`` draws the reference quantiser's -7..7 instead, whose
    logits follow the input (std ~4, top logits ~25, where a bf16 ulp is 0.125)."""
    c = config or qwen3_5_4b_config()
    gen = torch.Generator().manual_seed(seed)
    model = SynthModel(c)
    for name, k, n in linear_shapes(c):
        model.linears[name] = draw_int4(gen, k, n, symmetric=symmetric)
    for i, kind in enumerate(c.layer_types):
        p = f"layers.{i}."
        model.params[p + "input_layernorm.weight"] = _normal(gen, (c.hidden_size,), 0.02)
        model.params[p + "post_attention_layernorm.weight"] = _normal(gen, (c.hidden_size,), 0.02)
        if kind == FULL_ATTENTION:
            model.params[p + "self_attn.q_norm.weight"] = _normal(gen, (c.head_dim,), 0.02)
            model.params[p + "self_attn.k_norm.weight"] = _normal(gen, (c.head_dim,), 0.02)
        else:
            a = p + "linear_attn."
            model.params[a + "conv1d.weight"] = _normal(gen, (c.linear_conv_dim, 1, c.linear_conv_kernel_dim), 0.3)
            model.params[a + "A_log"] = _normal(gen, (c.linear_num_value_heads,), 0.1)
            model.params[a + "dt_bias"] = _normal(gen, (c.linear_num_value_heads,), 0.1)
            model.params[a + "norm.weight"] = _normal(gen, (c.linear_value_head_dim,), 0.02, mean=1.0)
    model.params["norm.weight"] = _normal(gen, (c.hidden_size,), 0.02)
    return model


def prompt_ids(vocab: int, length: int, seed: int = 1, batch: int = 1) -> torch.Tensor:
    """Random prompt token ids (config 5: 4096 ids, seed 1)."""
    return torch.randint(0, vocab, (batch, length), generator=torch.Generator().manual_seed(seed))


def expected_logit_scale(hidden: int, scale_std: float = 0.02) -> float:
    """rms of a logit for unit-rms inputs: sqrt(K * E[(q-8)^2] * E[s^2])."""
    return math.sqrt(hidden * 21.5 * scale_std**2)
