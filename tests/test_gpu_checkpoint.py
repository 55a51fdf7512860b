"""A checkpoint through the whole real-checkpoint path on the GPU.

A safetensors checkpoint of the mid config (the 4B model's head geometry, 4 layers) is written
with random bf16 weights under the published names, with fp32 ``A_log`` and gated-norm
weights as in the real files. It goes through ``load_checkpoint``: the name map, the shape
checks and install-time int4 quantisation on the GPU. Its own bf16 embedding table is kept,
untied from the int4 head. The per-op engine and the persistent kernel then decode it,
teacher-forced against the CPU oracle of the same loaded model (KL and top-1, the layer-2 bar
of the other model tests).
"""

from __future__ import annotations

import pytest
import torch
from safetensors.torch import save_file

from deltaforge_amd import synth
from deltaforge_amd.checkpoint import TEXT_PREFIX, checkpoint_shapes, load_checkpoint
from deltaforge_amd.config import mid_config
from deltaforge_amd.engine import DecodeEngine
from deltaforge_amd.harness.correctness import kl_and_agreement
from deltaforge_amd.persistent import PersistentDecoder

from .test_gpu_engine import oracle_for

pytestmark = pytest.mark.gpu


def _tensors(cfg, seed=11):
    gen = torch.Generator().manual_seed(seed)
    out = {}
    for target, shape in checkpoint_shapes(cfg).items():
        std, mean, dtype = 0.05, 0.0, torch.bfloat16
        if target.endswith("conv1d.weight"):
            std = 0.3
        elif target.endswith("A_log"):
            std, dtype = 0.5, torch.float32
        elif target.endswith("linear_attn.norm.weight"):
            mean, std, dtype = 1.0, 0.02, torch.float32
        elif target.endswith("norm.weight"):
            std = 0.02
        elif target == "embed_tokens.weight":
            std = 1.0
        out[TEXT_PREFIX + target] = (torch.randn(shape, generator=gen) * std + mean).to(dtype)
    return out


@pytest.fixture(scope="module")
def loaded(tmp_path_factory):
    cfg = mid_config(4)
    path = tmp_path_factory.mktemp("ckpt") / "model.safetensors"
    save_file(_tensors(cfg), str(path))
    model, report = load_checkpoint(path, cfg, device="cuda")
    print(report.summary(), flush=True)
    assert report.ok and "embed_tokens.weight" in model.params
    prompt = synth.prompt_ids(cfg.vocab_size, 24, seed=12)
    oracle = oracle_for(model)
    with torch.no_grad():
        ref_tokens, ref_logits = oracle.greedy(prompt, 8)
    return cfg, model, prompt, ref_tokens, ref_logits


def _teacher_forced(dec, prompt, ref_tokens, check=lambda: None):
    dec.prefill(prompt.cuda())
    check()
    got = [dec.logits.float().cpu().clone()]
    for t in range(ref_tokens.shape[1] - 1):
        dec.tokens.copy_(ref_tokens[:, t].cuda())
        dec.decode(1)
        check()
        got.append(dec.logits.float().cpu().clone())
    return torch.stack(got, dim=1)


@pytest.mark.parametrize("engine", ["graph", "persistent"])
def test_loaded_checkpoint_decodes_like_the_oracle(loaded, engine):
    cfg, model, prompt, ref_tokens, ref_logits = loaded
    print(f"checkpoint decode: {engine}", flush=True)
    if engine == "graph":
        dec = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
        got = _teacher_forced(dec, prompt, ref_tokens)
    else:
        dec = PersistentDecoder(model, max_seq_len=64, max_new_tokens=16)
        got = _teacher_forced(dec, prompt, ref_tokens, dec.check)
    assert dec.embed_table is not None
    kl, agree = kl_and_agreement(ref_logits.float(), got)
    print(f"{engine}: agreement {float(agree.float().mean()):.4f}, mean KL {float(kl.mean()):.3e}", flush=True)
    assert float(kl.mean()) < 1e-3
    assert float(agree.float().mean()) >= 7 / 8


def test_embedding_table_equal_to_the_head_changes_nothing():
    """The bf16-table path and the int4-head path must agree bit for bit when the table is the
    dequantised head (the synthetic model's tie)."""
    from oracle.int4 import dequantise_int4_k_major

    cfg = mid_config(4)
    model = synth.synth_model(cfg, seed=5)
    prompt = synth.prompt_ids(cfg.vocab_size, 16, seed=6).cuda()
    head = model.linears["lm_head"]
    tied = synth.SynthModel(cfg, dict(model.linears), dict(model.params))
    tied.params["embed_tokens.weight"] = dequantise_int4_k_major(head.packed, head.scale, 128).to(
        torch.bfloat16).t().contiguous()
    for cls in (DecodeEngine, PersistentDecoder):
        a, b = cls(model, max_seq_len=48, max_new_tokens=8), cls(tied, max_seq_len=48, max_new_tokens=8)
        assert a.embed_table is None and b.embed_table is not None
        for d in (a, b):
            d.prefill(prompt)
            d.decode(4)
        torch.cuda.synchronize()
        assert torch.equal(a.logits, b.logits), cls.__name__
        assert torch.equal(a.token_log[:, :4], b.token_log[:, :4]), cls.__name__
