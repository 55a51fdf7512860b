"""Write golden vectors by running the reference itself. Runs ONLY in the build container.

The reference (``/root/reference/src/deltaforge``) is pure PyTorch. This script imports it
on the CPU and records inputs and outputs for the functions whose *composition* no closed
form pins: ``ReferenceModel.forward`` with ``DecodeCache`` (prefill + greedy decode, tiny and
mid configs), the int4 champion head/linear expression installed through the reference's
own installer, ``torch_dequant_gemv_int4`` at a small shape, and ``RotaryEmbedding`` (the
mRoPE interleave at equal rows). Only the vectors are committed (``*.safetensors`` beside
this file); the reference never travels.

    python tests/golden/make_golden.py          # rewrites tests/golden/*.safetensors
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import torch
from safetensors.torch import save_file

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, "/root/reference/src")

from deltaforge import config as ref_config  # noqa: E402
from deltaforge.kernels.tiled_gemv import dequantise_int4_k_major, quantise_int4_k_major  # noqa: E402
from deltaforge.kernels.visible_int4_head import (  # noqa: E402
    install_int4_wide_torch_dequant,
    torch_dequant_gemv_int4,
)
from deltaforge.reference import ReferenceModel, RotaryEmbedding  # noqa: E402

from deltaforge_amd.config import ModelConfig, mid_config, tiny_config  # noqa: E402
from tests.golden.golden_params import checksum, make_params  # noqa: E402


def to_ref_config(c: ModelConfig):
    return ref_config.ModelConfig(
        hidden_size=c.hidden_size, intermediate_size=c.intermediate_size,
        num_hidden_layers=c.num_hidden_layers, vocab_size=c.vocab_size, layer_types=c.layer_types,
        rms_norm_eps=c.rms_norm_eps, num_attention_heads=c.num_attention_heads,
        num_key_value_heads=c.num_key_value_heads, head_dim=c.head_dim,
        linear_num_key_heads=c.linear_num_key_heads, linear_num_value_heads=c.linear_num_value_heads,
        linear_key_head_dim=c.linear_key_head_dim, linear_value_head_dim=c.linear_value_head_dim,
        linear_conv_kernel_dim=c.linear_conv_kernel_dim, rope_theta=c.rope_theta,
        partial_rotary_factor=c.partial_rotary_factor, mrope_section=c.mrope_section,
        max_position_embeddings=c.max_position_embeddings, name=c.name,
    )


def build(c: ModelConfig, seed: int):
    model = ReferenceModel(to_ref_config(c)).to(dtype=torch.bfloat16).eval()
    params = make_params(c, seed)
    model.load_state_dict(params, strict=True)
    return model, params


@torch.no_grad()
def step_logits(model, prompt, steps: int):
    """Prefill, then ``steps`` greedy tokens, keeping each step's logits."""
    cache = model.new_cache(1, prompt.shape[1] + steps)
    logits, _ = model(prompt, cache)
    out = [logits]
    token = logits[:, -1].argmax(-1, keepdim=True)
    tokens = [token]
    for _ in range(steps - 1):
        logits, _ = model(token, cache, num_logits_to_keep=1)
        out.append(logits)
        token = logits[:, -1].argmax(-1, keepdim=True)
        tokens.append(token)
    return out, torch.cat(tokens, dim=1), cache


def model_case(name: str, c: ModelConfig, seed: int, prompt_len: int, steps: int, int4: bool = False):
    model, params = build(c, seed)
    if int4:
        install_int4_wide_torch_dequant(model)
    prompt = torch.randint(0, c.vocab_size, (1, prompt_len), generator=torch.Generator().manual_seed(seed + 1))
    logits, tokens, cache = step_logits(model, prompt, steps)
    record = {
        "prompt": prompt,
        "prefill_logits": logits[0].contiguous(),
        "decode_logits": torch.cat(logits[1:], dim=1).contiguous(),
        "tokens": tokens,
        "param_checksums": checksum(params),
    }
    for i, layer in enumerate(cache.layers):
        if hasattr(layer, "recurrent"):
            record[f"cache.{i}.conv"] = layer.conv.contiguous()
            record[f"cache.{i}.recurrent_head0"] = layer.recurrent[:, :2].contiguous()
        else:
            end = cache.seq_len
            record[f"cache.{i}.keys"] = layer.keys[:, :, :end].contiguous()
            record[f"cache.{i}.values"] = layer.values[:, :, :end].contiguous()
    if int4:
        # Small configs keep the reference's packed weights verbatim; larger ones keep a
        # checksum per tensor, and the tests re-quantise with the oracle and compare.
        verbatim = c.hidden_size <= 128
        for mod_name, mod in model.named_modules():
            if hasattr(mod, "w_k_major"):
                key = "lm_head" if mod_name == "tiled_lm_head" else mod_name + ".weight"
                if verbatim:
                    record[f"int4.{key}.packed"] = mod.w_k_major.contiguous()
                    record[f"int4.{key}.scale"] = mod.qscale.contiguous()
                else:
                    record[f"int4sum.{key}"] = torch.tensor(
                        [float(mod.w_k_major.double().sum()), float(mod.qscale.double().sum()),
                         float(mod.qscale.double().pow(2).sum())], dtype=torch.float64)
    save_file(record, str(HERE / f"{name}.safetensors"))
    print(name, {k: tuple(v.shape) for k, v in record.items() if not k.startswith("int4")})


def int4_gemv_case():
    gen = torch.Generator().manual_seed(31)
    weight = (torch.randn((64, 256), generator=gen) * 0.05).to(torch.bfloat16)
    x = torch.randn((2, 256), generator=gen).to(torch.bfloat16)
    q = quantise_int4_k_major(weight)
    out = torch_dequant_gemv_int4(x, q.qweight, q.scale, q.group_size)
    dense = dequantise_int4_k_major(q.qweight, q.scale, group_size=q.group_size)
    save_file({"weight": weight, "x": x, "packed": q.qweight, "scale": q.scale,
               "group": torch.tensor([q.group_size]), "dequant_f32": dense, "out": out},
              str(HERE / "int4_gemv.safetensors"))
    print("int4_gemv", tuple(out.shape), q.group_size)


def rope_case():
    cfg = to_ref_config(mid_config(4))
    rope = RotaryEmbedding(cfg)
    positions = torch.tensor([[0, 1, 2, 33, 4095, 4096, 32768, 131071, 131072, 262143]])
    cos, sin = rope(positions, torch.bfloat16)
    cos3, sin3 = rope(positions.unsqueeze(0).expand(3, -1, -1), torch.bfloat16)
    cos32, sin32 = rope(positions, torch.float32)
    save_file({"positions": positions, "cos": cos, "sin": sin, "cos_mrope3": cos3, "sin_mrope3": sin3,
               "cos_f32": cos32, "sin_f32": sin32}, str(HERE / "rope.safetensors"))
    print("rope", tuple(cos.shape))


def main() -> None:
    torch.manual_seed(0)
    model_case("tiny_dense", tiny_config(), seed=11, prompt_len=12, steps=5)
    model_case("tiny_int4", tiny_config(), seed=11, prompt_len=12, steps=5, int4=True)
    model_case("mid_dense", mid_config(4), seed=21, prompt_len=6, steps=4)
    model_case("mid_int4", mid_config(4), seed=21, prompt_len=6, steps=4, int4=True)
    int4_gemv_case()
    rope_case()
    (HERE / "README.json").write_text(json.dumps({
        "generated_by": "tests/golden/make_golden.py",
        "reference": "LoveManna/deltaforge src/deltaforge (reference.py, model.py, kernels/tiled_gemv.py, "
                     "kernels/visible_int4_head.py)",
        "torch": torch.__version__,
    }, indent=2) + "\n")


if __name__ == "__main__":
    main()
