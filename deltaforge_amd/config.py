"""Decode-path configuration for the Qwen3.5 hybrid family (Gated DeltaNet + gated GQA).

Field names follow the checkpoint's ``text_config`` keys, which is the interchange format
the reference reads (reference: ``src/deltaforge/config.py:39-152``). Only the text decode
path is modelled; the vision tower and MTP head are outside it.

The layer schedule is "every fourth layer is full attention" (config.py:155-159): with 32
layers that is 24 Gated DeltaNet layers and 8 gated-attention layers.
"""

from __future__ import annotations

from dataclasses import dataclass

LINEAR_ATTENTION = "linear_attention"
FULL_ATTENTION = "full_attention"
SIGMOID_GATE = "sigmoid"
SWISH_GATE = "swish"

__all__ = [
    "FULL_ATTENTION",
    "LINEAR_ATTENTION",
    "ModelConfig",
    "SIGMOID_GATE",
    "SWISH_GATE",
    "hybrid_layer_types",
    "mid_config",
    "qwen3_5_4b_config",
    "tiny_config",
]


def hybrid_layer_types(num_layers: int, full_every: int = 4) -> tuple[str, ...]:
    """``3 x linear`` then ``1 x full``, repeated (reference config.py:155-159)."""
    return tuple(
        FULL_ATTENTION if (index + 1) % full_every == 0 else LINEAR_ATTENTION for index in range(num_layers)
    )


@dataclass(frozen=True)
class ModelConfig:
    """Shapes of the text decoder. Defaults are Qwen3.5-4B's per-layer values."""

    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    vocab_size: int
    layer_types: tuple[str, ...]
    rms_norm_eps: float = 1e-6
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    head_dim: int = 256
    attn_output_gate: bool = True
    output_gate_type: str = SIGMOID_GATE
    linear_num_key_heads: int = 16
    linear_num_value_heads: int = 32
    linear_key_head_dim: int = 128
    linear_value_head_dim: int = 128
    linear_conv_kernel_dim: int = 4
    rope_theta: float = 1e7
    partial_rotary_factor: float = 0.25
    mrope_section: tuple[int, ...] = (11, 11, 10)
    max_position_embeddings: int = 262144
    tie_word_embeddings: bool = True
    name: str = "qwen3.5-4b"

    def __post_init__(self) -> None:
        if len(self.layer_types) != self.num_hidden_layers:
            raise ValueError(
                f"{len(self.layer_types)} layer types for {self.num_hidden_layers} layers"
            )
        bad = set(self.layer_types) - {LINEAR_ATTENTION, FULL_ATTENTION}
        if bad:
            raise ValueError(f"unknown layer types {sorted(bad)}")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("query heads must be a multiple of KV heads")
        if self.linear_num_value_heads % self.linear_num_key_heads:
            raise ValueError("linear value heads must be a multiple of linear key heads")
        if self.rotary_dim % 2:
            raise ValueError(f"rotary_dim {self.rotary_dim} is odd")
        if sum(self.mrope_section) != self.rotary_dim // 2:
            raise ValueError("mrope_section must sum to rotary_dim // 2")
        if self.output_gate_type not in (SIGMOID_GATE, SWISH_GATE):
            raise ValueError(f"unknown output gate {self.output_gate_type!r}")

    # Derived dimensions (reference config.py:120-152).
    @property
    def rotary_dim(self) -> int:
        return int(self.head_dim * self.partial_rotary_factor)

    @property
    def num_key_value_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    @property
    def linear_key_dim(self) -> int:
        return self.linear_num_key_heads * self.linear_key_head_dim

    @property
    def linear_value_dim(self) -> int:
        return self.linear_num_value_heads * self.linear_value_head_dim

    @property
    def linear_conv_dim(self) -> int:
        return 2 * self.linear_key_dim + self.linear_value_dim

    @property
    def linear_value_groups(self) -> int:
        return self.linear_num_value_heads // self.linear_num_key_heads

    def layer_indices(self, layer_type: str) -> tuple[int, ...]:
        return tuple(i for i, kind in enumerate(self.layer_types) if kind == layer_type)


def qwen3_5_4b_config() -> ModelConfig:
    """Qwen3.5-4B text decoder (reference config.py:200-230)."""
    return ModelConfig(
        hidden_size=2560,
        intermediate_size=9216,
        num_hidden_layers=32,
        vocab_size=248320,
        layer_types=hybrid_layer_types(32),
    )


def tiny_config() -> ModelConfig:
    """Two-layer (1 linear + 1 full) CPU fixture shape (reference config.py:233-266)."""
    return ModelConfig(
        hidden_size=128,
        intermediate_size=256,
        num_hidden_layers=2,
        vocab_size=512,
        layer_types=(LINEAR_ATTENTION, FULL_ATTENTION),
        num_attention_heads=2,
        num_key_value_heads=1,
        head_dim=32,
        linear_num_key_heads=2,
        linear_num_value_heads=4,
        linear_key_head_dim=16,
        linear_value_head_dim=16,
        rope_theta=1e4,
        mrope_section=(2, 1, 1),
        max_position_embeddings=4096,
        name="tiny",
    )


def mid_config(num_layers: int = 4) -> ModelConfig:
    """Qwen3.5-4B's per-head shapes on a narrow, short stack.

    Head dims (128 for Gated DeltaNet, 256 for attention), head counts, the GQA ratios and
    RoPE are the real model's, so every HIP kernel runs at its production head geometry;
    only ``hidden_size``, ``intermediate_size``, depth and vocabulary shrink so a CPU oracle
    finishes in seconds. All K dimensions stay multiples of 256 (group-128 int4 with the
    two halves of K each group-aligned).
    """
    return ModelConfig(
        hidden_size=512,
        intermediate_size=1024,
        num_hidden_layers=num_layers,
        vocab_size=4096,
        layer_types=hybrid_layer_types(num_layers),
        name=f"mid-{num_layers}",
    )
