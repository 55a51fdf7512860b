"""Real-checkpoint path: the safetensors name map, the shape proof, and install-time int4.

The published Qwen3.5 checkpoint stores the text decoder under ``model.language_model.``,
plus a vision tower (``model.visual.``) and a multi-token-prediction head (``mtp.``). Decode
uses neither, so both are skipped by prefix and counted in the report. Every other name maps
explicitly. A text-decoder tensor with no mapping is an error, never a silent skip. That is the
reference's loader contract (weights.py:130-270); the loader here is built differently:

1. a catalogue of every tensor (name -> shard, dtype, shape) is read from the safetensors
   headers alone, so the whole name map and shape proof are settled before any weight byte
   is read;
2. each entry is routed (skipped by prefix, mapped to a parameter, or refused), and the
   mapped ones are checked against ``checkpoint_shapes``;
3. only when the plan is whole (or ``strict=False``) are the tensors read, shard by shard,
   each handed to the converter of its parameter kind.

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
import struct
from collections import defaultdict
from dataclasses import dataclass, field
from pathlib import Path
from typing import NamedTuple

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


# -- routing -----------------------------------------------------------------------------------


class _Route(NamedTuple):
    """Where one checkpoint tensor goes: ``kind`` is ``"vision"`` or ``"mtp"`` (skipped by
    design), ``"param"`` (``target`` names the model parameter) or ``"foreign"`` (``why`` says
    which rule refused it)."""

    kind: str
    target: str | None = None
    why: str = ""


def _route(name: str) -> _Route:
    if name.startswith(VISION_PREFIX):
        return _Route("vision")
    if name.startswith(MTP_PREFIX):
        return _Route("mtp")
    top = _TOP_LEVEL.get(name)
    if top is not None:
        return _Route("param", top)
    m = _LAYER_NAME.match(name)
    if m is None:
        return _Route("foreign", why="outside the text decoder, the vision tower and the MTP head")
    layer, suffix = int(m.group(1)), m.group(2)
    if suffix not in _LAYER_SUFFIXES:
        return _Route("foreign", why=f"layer {layer} has no parameter {suffix!r}")
    return _Route("param", f"layers.{layer}.{suffix}")


def map_checkpoint_name(name: str) -> str | None:
    """Checkpoint tensor name -> model parameter name; ``None`` for the vision tower and the
    MTP head; ``WeightMappingError`` for any other name the decoder does not own."""
    r = _route(name)
    if r.kind == "foreign":
        raise WeightMappingError(f"checkpoint tensor {name!r} has no place in the decoder: {r.why}")
    return r.target


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


# -- int4 --------------------------------------------------------------------------------------


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


# -- report ------------------------------------------------------------------------------------


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
        return not any(self.problems().values())

    def problems(self) -> dict[str, tuple[str, ...]]:
        """Each way the checkpoint can fail to fit the model, with the names concerned."""
        return {"missing (model parameters with no checkpoint tensor)": self.missing,
                "unmapped (checkpoint tensors the decoder has no place for)": self.unmapped,
                "shape mismatch": self.mismatched}

    def summary(self, show: int = 6) -> str:
        out = [f"{len(self.loaded)} decoder tensors loaded; skipped by design: {len(self.skipped_vision)} "
               f"vision-tower and {len(self.skipped_mtp)} MTP-head tensors (decode reads neither)"]
        for heading, names in self.problems().items():
            if not names:
                continue
            out.append(f"{heading}: {len(names)}")
            out.extend(f"    {n}" for n in names[:show])
            if len(names) > show:
                out.append(f"    ... and {len(names) - show} more")
        return "\n".join(out)


# -- catalogue ---------------------------------------------------------------------------------


class _Entry(NamedTuple):
    shard: Path
    dtype: str
    shape: tuple[int, ...]


def _header(shard: Path) -> dict[str, _Entry]:
    """Tensor name -> entry from a safetensors file's header alone: an 8-byte little-endian
    length, then that many bytes of JSON (``{name: {dtype, shape, data_offsets}}`` plus an
    optional ``__metadata__``). No weight data is read."""
    with open(shard, "rb") as f:
        head = f.read(8)
        if len(head) != 8:
            raise WeightMappingError(f"{shard} is too short to be a safetensors file")
        (size,) = struct.unpack("<Q", head)
        meta = json.loads(f.read(size))
    return {name: _Entry(shard, m["dtype"], tuple(m["shape"])) for name, m in meta.items() if name != "__metadata__"}


def _catalogue(path: Path) -> dict[str, _Entry]:
    """Every tensor of a checkpoint: one file, a directory with a sharded index (the index
    decides which shard holds each name), or a directory of ``*.safetensors`` files."""
    if path.is_file():
        return _header(path)
    index = path / "model.safetensors.index.json"
    if index.exists():
        owner: dict[str, str] = json.loads(index.read_text())["weight_map"]
        headers = {f: _header(path / f) for f in sorted(set(owner.values()))}
        absent = [n for n, f in owner.items() if n not in headers[f]]
        if absent:
            raise WeightMappingError(f"the index places {len(absent)} tensors in shards that lack them, "
                                     f"e.g. {absent[0]!r} in {owner[absent[0]]}")
        return {n: headers[f][n] for n, f in owner.items()}
    files = sorted(path.glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"{path} holds no safetensors checkpoint (no file, index or *.safetensors)")
    found: dict[str, _Entry] = {}
    for shard in files:
        for name, entry in _header(shard).items():
            if name in found:
                raise WeightMappingError(f"{name!r} is stored twice, in {found[name].shard.name} and {shard.name}")
            found[name] = entry
    return found


# -- conversion --------------------------------------------------------------------------------


def _quantised(t: torch.Tensor, device) -> CanonicalInt4:
    q = quantise_int4_k_major(t.to(device))
    return CanonicalInt4(q.packed.cpu(), q.scale.cpu())


def _converter(target: str, linear_names: set[str], tied: bool):
    """The function that puts a checkpoint tensor for ``target`` into the model."""
    if target in linear_names:
        def put(model, t, device):
            model.linears[target] = _quantised(t, device)
    elif target == "embed_tokens.weight":
        def put(model, t, device):
            table = t.to(torch.bfloat16)
            model.params[target] = table
            if tied:  # the head is the embedding table, quantised like every linear
                model.linears["lm_head"] = _quantised(table, device)
    elif target == "lm_head.weight":
        def put(model, t, device):
            model.linears["lm_head"] = _quantised(t, device)
    else:
        def put(model, t, device):
            model.params[target] = t.to(torch.bfloat16)
    return put


def load_checkpoint(path: str | Path, config: ModelConfig, *, strict: bool = True,
                    device: str | torch.device = "cpu") -> tuple[SynthModel, LoadReport]:
    """Read a safetensors checkpoint (a file, a directory of shards, or a sharded index).

    Returns the model in this build's format and the load report. Linears are quantised on
    ``device``; a GPU makes the 4B model's 248 matrices take seconds rather than minutes.
    ``strict`` raises ``WeightMappingError`` unless the report is ``ok``, before any weight
    data is read.
    """
    from safetensors import safe_open

    expected = checkpoint_shapes(config)
    catalogue = _catalogue(Path(path))

    skipped: dict[str, list[str]] = {"vision": [], "mtp": []}
    unmapped: list[str] = []
    mismatched: list[str] = []
    plan: dict[str, str] = {}  # model parameter -> checkpoint name
    for name in sorted(catalogue):
        r = _route(name)
        if r.kind in skipped:
            skipped[r.kind].append(name)
        elif r.kind == "foreign" or r.target not in expected:  # e.g. lm_head.weight of a tied model
            unmapped.append(name)
        elif catalogue[name].shape != expected[r.target]:
            mismatched.append(f"{name}: {catalogue[name].shape} in the checkpoint, {expected[r.target]} in the model")
        else:
            plan[r.target] = name

    report = LoadReport(loaded=tuple(sorted(plan.values())), skipped_vision=tuple(skipped["vision"]),
                        skipped_mtp=tuple(skipped["mtp"]), missing=tuple(sorted(set(expected) - set(plan))),
                        unmapped=tuple(unmapped), mismatched=tuple(mismatched))
    if strict and not report.ok:
        raise WeightMappingError(f"refusing a partial load of {path}:\n{report.summary()}")

    linear_names = {name for name, _, _ in linear_shapes(config) if name != "lm_head"}
    by_shard: dict[Path, list[tuple[str, str]]] = defaultdict(list)
    for target, name in plan.items():
        by_shard[catalogue[name].shard].append((target, name))
    model = SynthModel(config)
    for shard, items in by_shard.items():
        with safe_open(str(shard), framework="pt") as handle:
            for target, name in items:
                _converter(target, linear_names, config.tie_word_embeddings)(model, handle.get_tensor(name), device)
    return model, report
