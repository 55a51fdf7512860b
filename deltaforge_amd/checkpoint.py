"""Real-checkpoint path: the safetensors name map, the shape proof, and install-time int4.

The published Qwen3.5 checkpoint stores the text decoder under ``model.language_model.``,
plus a vision tower (``model.visual.``) and a multi-token-prediction head (``mtp.``). Decode
uses neither, so both are skipped by prefix and counted in the report. Every other name maps
explicitly. A text-decoder tensor with no mapping is an error, never a silent skip. This is the
reference's loader contract (weights.py:130-270), restated for this build's model format.

Model format (``synth.SynthModel``):
- ``linears`` holds each projection as canonical K-major int4 (``CanonicalInt4``, bf16
  group scales), quantised once at load.
- ``params`` holds the small tensors (norms, conv taps, ``A_log``, ``dt_bias``) in bf16. The
  reference casts the whole model to bf16 (model.py:83-105), fp32 ``A_log`` and the fp32
  gated-norm weight included.
- ``lm_head`` is the tied embedding, quantised like every other linear.
- When a checkpoint is loaded, its bf16 embedding table is also kept, as
  ``params["embed_tokens.weight"]``.

The quantiser is the reference's symmetric int4 (kernels/tiled_gemv.py:242-278):
- per group, ``scale = amax / 7`` (1 for an all-zero group);
- ``q = clamp(round(w / scale), -7, 7)``, stored as ``q + 8``.

One change: the scale is rounded to bf16 (this build's interchange format stores bf16
scales) *before* ``q`` is computed, so the stored (q, scale) pair is self-consistent. The
reference keeps fp32 scales. A dequantised weight can therefore differ from the reference's
by the bf16 rounding of its group's scale.
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass, field
from pathlib import Path

import torch

from .config import FULL_ATTENTION, ModelConfig
from .synth import CanonicalInt4, SynthModel, linear_shapes

__all__ = [
    "LoadReport",
    "MTP_PREFIX",
    "TEXT_PREFIX",
    "VISION_PREFIX",
    "WeightMappingError",
    "checkpoint_shapes",
    "group_size_for",
    "load_checkpoint",
    "map_checkpoint_name",
    "quantise_int4_k_major",
]

TEXT_PREFIX = "model.language_model."
VISION_PREFIX = "model.visual."
MTP_PREFIX = "mtp."

# Suffixes below ``model.language_model.layers.<i>.`` that the decoder owns. The names on
# both sides are the module paths of the reference model, so the map is the identity on this
# set. What the set fixes is *which* suffixes exist: anything else under a layer fails.
_LAYER_SUFFIXES = frozenset({
    "input_layernorm.weight", "post_attention_layernorm.weight",
    "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight",
    "self_attn.q_norm.weight", "self_attn.k_norm.weight",
    "linear_attn.in_proj_qkv.weight", "linear_attn.in_proj_z.weight", "linear_attn.in_proj_b.weight",
    "linear_attn.in_proj_a.weight", "linear_attn.conv1d.weight", "linear_attn.A_log", "linear_attn.dt_bias",
    "linear_attn.norm.weight", "linear_attn.out_proj.weight",
})
_TOP_LEVEL = {
    TEXT_PREFIX + "embed_tokens.weight": "embed_tokens.weight",
    TEXT_PREFIX + "norm.weight": "norm.weight",
    "lm_head.weight": "lm_head.weight",  # only in untied checkpoints
}
_LAYER_NAME = re.compile(re.escape(TEXT_PREFIX) + r"layers\.(\d+)\.(.+)$")


class WeightMappingError(RuntimeError):
    """The checkpoint and the model do not line up (unknown, missing or misshapen tensors)."""


def map_checkpoint_name(name: str) -> str | None:
    """Checkpoint tensor name -> model parameter name; ``None`` for the vision tower and the
    MTP head; ``WeightMappingError`` for any other name the decoder does not own."""
    if name.startswith((VISION_PREFIX, MTP_PREFIX)):
        return None
    if name in _TOP_LEVEL:
        return _TOP_LEVEL[name]
    m = _LAYER_NAME.match(name)
    if m is None:
        raise WeightMappingError(f"unrecognised checkpoint tensor: {name!r}")
    if m.group(2) not in _LAYER_SUFFIXES:
        raise WeightMappingError(f"unrecognised tensor {name!r}: no mapping for layer suffix {m.group(2)!r}")
    return f"layers.{int(m.group(1))}.{m.group(2)}"


def checkpoint_shapes(config: ModelConfig) -> dict[str, tuple[int, ...]]:
    """Model parameter name -> the shape its checkpoint tensor must have.

    Linears are stored as ``nn.Linear`` weights, ``[out_features, in_features]``. The
    embedding is ``[vocab, hidden]``. There is no ``lm_head.weight`` when embeddings are tied.
    """
    c = config
    shapes: dict[str, tuple[int, ...]] = {}
    for name, k, n in linear_shapes(c):
        if name != "lm_head":
            shapes[name] = (n, k)
    for i, kind in enumerate(c.layer_types):
        p = f"layers.{i}."
        shapes[p + "input_layernorm.weight"] = (c.hidden_size,)
        shapes[p + "post_attention_layernorm.weight"] = (c.hidden_size,)
        if kind == FULL_ATTENTION:
            shapes[p + "self_attn.q_norm.weight"] = (c.head_dim,)
            shapes[p + "self_attn.k_norm.weight"] = (c.head_dim,)
        else:
            a = p + "linear_attn."
            shapes[a + "conv1d.weight"] = (c.linear_conv_dim, 1, c.linear_conv_kernel_dim)
            shapes[a + "A_log"] = (c.linear_num_value_heads,)
            shapes[a + "dt_bias"] = (c.linear_num_value_heads,)
            shapes[a + "norm.weight"] = (c.linear_value_head_dim,)
    shapes["norm.weight"] = (c.hidden_size,)
    shapes["embed_tokens.weight"] = (c.vocab_size, c.hidden_size)
    if not c.tie_word_embeddings:
        shapes["lm_head.weight"] = (c.vocab_size, c.hidden_size)
    return shapes


def group_size_for(k: int) -> int:
    """128 when ``K % 256 == 0``, else ``K / 2`` (reference kernels/quantised_linear.py:193-207)."""
    if k % 2:
        raise ValueError(f"int4 packing needs an even K, got {k}")
    group = 128 if k % 256 == 0 else k // 2
    if group & (group - 1):
        raise ValueError(f"group {group} for K={k} is not a power of two")
    return group


def quantise_int4_k_major(weight: torch.Tensor, rows_per_chunk: int = 8192) -> CanonicalInt4:
    """``[N, K]`` weight -> K-major int4 with bf16 group scales (see the module docstring).

    Byte ``[j, n]`` holds ``k = j`` in its low nibble and ``k = j + K/2`` in its high
    nibble. The work runs on the weight's device, in row chunks that bound the fp32
    temporaries.
    """
    if weight.dim() != 2:
        raise ValueError(f"expected a 2-D [N, K] weight, got {tuple(weight.shape)}")
    n, k = weight.shape
    group = group_size_for(k)
    half = k // 2
    packed = torch.empty((half, n), dtype=torch.uint8, device=weight.device)
    scale = torch.empty((k // group, n), dtype=torch.bfloat16, device=weight.device)
    for r0 in range(0, n, rows_per_chunk):
        blk = weight[r0:r0 + rows_per_chunk].detach().float().reshape(-1, k // group, group)
        s = blk.abs().amax(dim=2) / 7.0
        s = torch.where(s > 0, s, torch.ones_like(s)).to(torch.bfloat16)
        q = torch.round(blk / s.float().unsqueeze(2)).clamp_(-7, 7).to(torch.int16).reshape(-1, k)
        nib = (q + 8).to(torch.uint8)
        packed[:, r0:r0 + rows_per_chunk] = (nib[:, :half] | (nib[:, half:] << 4)).t()
        scale[:, r0:r0 + rows_per_chunk] = s.t()
    return CanonicalInt4(packed, scale)


@dataclass(frozen=True)
class LoadReport:
    """Counts and names of what a load did. It is ``ok`` when nothing is missing, unmapped
    or misshapen."""

    loaded: tuple[str, ...] = ()
    skipped_vision: tuple[str, ...] = ()
    skipped_mtp: tuple[str, ...] = ()
    missing: tuple[str, ...] = ()
    unmapped: tuple[str, ...] = ()
    mismatched: tuple[str, ...] = field(default=())

    @property
    def ok(self) -> bool:
        return not (self.missing or self.unmapped or self.mismatched)

    def summary(self) -> str:
        lines = [f"loaded {len(self.loaded)} tensors",
                 f"skipped {len(self.skipped_vision)} vision-tower tensors (not on the decode path)",
                 f"skipped {len(self.skipped_mtp)} MTP-head tensors (not on the decode path)"]
        for label, names in (("missing from checkpoint", self.missing), ("unmapped in checkpoint", self.unmapped),
                             ("shape mismatch", self.mismatched)):
            if names:
                more = f" (+{len(names) - 8} more)" if len(names) > 8 else ""
                lines.append(f"{len(names)} {label}: {', '.join(names[:8])}{more}")
        return "\n".join(lines)


def _shards(path: Path) -> list[Path]:
    if path.is_file():
        return [path]
    index = path / "model.safetensors.index.json"
    if index.exists():
        weight_map = json.loads(index.read_text())["weight_map"]
        return [path / shard for shard in sorted(set(weight_map.values()))]
    shards = sorted(path.glob("*.safetensors"))
    if not shards:
        raise FileNotFoundError(f"no .safetensors files under {path}")
    return shards


def load_checkpoint(path: str | Path, config: ModelConfig, *, strict: bool = True,
                    device: str | torch.device = "cpu") -> tuple[SynthModel, LoadReport]:
    """Read a safetensors checkpoint (a file, a directory of shards, or a sharded index).

    Returns the model in this build's format and the load report. Linears are quantised on
    ``device``; a GPU makes the 4B model's 248 matrices take seconds rather than minutes.
    ``strict`` raises ``WeightMappingError`` unless the report is ``ok``.
    """
    from safetensors import safe_open

    expected = checkpoint_shapes(config)
    linear_names = {name for name, _, _ in linear_shapes(config) if name != "lm_head"}
    model = SynthModel(config)
    loaded, vision, mtp, unmapped, mismatched = [], [], [], [], []
    seen: set[str] = set()
    for shard in _shards(Path(path)):
        with safe_open(str(shard), framework="pt") as handle:
            for name in handle.keys():  # noqa: SIM118 - safe_open has no __contains__
                if name.startswith(VISION_PREFIX):
                    vision.append(name)
                    continue
                if name.startswith(MTP_PREFIX):
                    mtp.append(name)
                    continue
                try:
                    target = map_checkpoint_name(name)
                except WeightMappingError:
                    unmapped.append(name)
                    continue
                if target not in expected:  # e.g. lm_head.weight of a tied model
                    unmapped.append(name)
                    continue
                t = handle.get_tensor(name)
                if tuple(t.shape) != expected[target]:
                    mismatched.append(f"{name}: checkpoint {tuple(t.shape)} != model {expected[target]}")
                    continue
                if target in linear_names:
                    q = quantise_int4_k_major(t.to(device))
                    model.linears[target] = CanonicalInt4(q.packed.cpu(), q.scale.cpu())
                elif target == "embed_tokens.weight":
                    table = t.to(torch.bfloat16)
                    model.params[target] = table
                    if config.tie_word_embeddings:
                        q = quantise_int4_k_major(table.to(device))
                        model.linears["lm_head"] = CanonicalInt4(q.packed.cpu(), q.scale.cpu())
                elif target == "lm_head.weight":
                    q = quantise_int4_k_major(t.to(device))
                    model.linears["lm_head"] = CanonicalInt4(q.packed.cpu(), q.scale.cpu())
                else:
                    model.params[target] = t.to(torch.bfloat16)
                loaded.append(name)
                seen.add(target)
    report = LoadReport(loaded=tuple(sorted(loaded)), skipped_vision=tuple(sorted(vision)),
                        skipped_mtp=tuple(sorted(mtp)), missing=tuple(sorted(set(expected) - seen)),
                        unmapped=tuple(sorted(unmapped)), mismatched=tuple(sorted(mismatched)))
    if strict and not report.ok:
        raise WeightMappingError("checkpoint did not map cleanly onto the model:\n" + report.summary())
    return model, report
