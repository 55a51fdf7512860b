"""GPU parity of the drop-in surface: the ``deltaforge_amd::`` custom ops against the CPU
oracle, and ``greedy_decode`` through installed champions against the oracle's greedy run."""

from __future__ import annotations

import pytest
import torch

from deltaforge_amd import synth
from deltaforge_amd.config import mid_config, qwen3_5_4b_config
from deltaforge_amd.kernels import hip_ops
from deltaforge_amd.model import apply_champions, greedy_decode
from oracle import ops as oracle_ops
from oracle.int4 import dequant_gemv

from .test_gpu_engine import oracle_for
from .test_gpu_kernels import ATOL, RTOL, STATE_TOL, close

pytestmark = pytest.mark.gpu
DEV = "cuda"
BF16 = torch.bfloat16


@pytest.mark.parametrize("shape,n", [((1, 2560), 1024), ((20, 512), 128), ((2, 3, 256), 64)])
def test_tiled_gemv_int4_op_matches_reference_expression(shape, n):
    gen = torch.Generator().manual_seed(n + shape[-1])
    w = synth.draw_int4(gen, shape[-1], n)
    x = torch.randn(shape, generator=gen).to(BF16)
    got = hip_ops.tiled_gemv_int4(x.to(DEV), w.packed.to(DEV), w.scale.to(DEV), 128)
    want = dequant_gemv(x.reshape(-1, shape[-1]), w.packed, w.scale, 128).reshape(*shape[:-1], n)
    assert got.shape == want.shape
    close(got, want, what=f"tiled_gemv_int4 {shape} x {n}")


def test_tiled_gemv_int4_repack_cache_sees_in_place_updates():
    gen = torch.Generator().manual_seed(7)
    w = synth.draw_int4(gen, 256, 64)
    x = torch.randn((1, 256), generator=gen).to(BF16).to(DEV)
    packed, scale = w.packed.to(DEV), w.scale.to(DEV)
    a = hip_ops.tiled_gemv_int4(x, packed, scale, 128)
    packed.bitwise_xor_(0x11)  # every nibble changes; the cached tiling must not be reused
    b = hip_ops.tiled_gemv_int4(x, packed, scale, 128)
    close(b, dequant_gemv(x.cpu(), packed.cpu(), scale.cpu(), 128), what="after in-place update")
    assert not torch.equal(a, b)


def test_gated_delta_decode_op():
    inp = synth.delta_inputs(seed=2, batch=2)
    state = inp["state"].to(DEV).contiguous()
    conv = inp["conv_state"].to(DEV).contiguous()
    out = hip_ops.gated_delta_decode(inp["qkv"].to(DEV), inp["a"].to(DEV), inp["b"].to(DEV), inp["A_log"].to(DEV),
                                     inp["dt_bias"].to(DEV), inp["conv_w"].to(DEV).reshape(-1, 1, 4), conv, state,
                                     inp["num_k_heads"])
    w_out, w_state, w_conv = oracle_ops.delta_step(inp["qkv"], inp["conv_state"], inp["conv_w"], inp["a"], inp["b"],
                                                   inp["A_log"], inp["dt_bias"], inp["state"], inp["num_k_heads"])
    close(out, w_out, what="delta op out")
    close(state, w_state, atol=STATE_TOL, rtol=0, what="delta op state")
    assert torch.equal(conv.cpu(), w_conv)


def test_gated_attention_decode_op():
    cfg = qwen3_5_4b_config()
    context = 300
    inp = synth.attention_inputs(seed=4, batch=1, context=context, slack=16)
    kc, vc = inp["k_cache"].to(DEV), inp["v_cache"].to(DEV)
    position = torch.tensor([context], dtype=torch.int32, device=DEV)
    got = hip_ops.gated_attention_decode(inp["q"].to(DEV), inp["k"].to(DEV), inp["v"].to(DEV), inp["q_norm_w"].to(DEV),
                                         inp["k_norm_w"].to(DEV), synth.inv_freq(cfg).to(DEV), kc, vc, position,
                                         cfg.num_attention_heads, True, cfg.rms_norm_eps)
    wk, wv = inp["k_cache"].clone(), inp["v_cache"].clone()
    want = oracle_ops.attention_decode(inp["q"], inp["k"], inp["v"], inp["q_norm_w"], inp["k_norm_w"], wk, wv,
                                       context, cfg)
    close(got, want, what="attention op")
    assert torch.equal(vc[:, :, context].cpu(), wv[:, :, context])


def test_greedy_decode_through_installed_champions():
    cfg = mid_config(4)
    model = synth.synth_model(cfg, seed=5)
    prompt = synth.prompt_ids(cfg.vocab_size, 24, seed=6)
    apply_champions(model)
    got = greedy_decode(model, prompt, 6)
    with torch.no_grad():
        want, _ = oracle_for(model).greedy(prompt, 6)
    print(f"greedy_decode tokens {got.tolist()} oracle {want.tolist()}")
    assert got.shape == (1, 6)
    # bf16 near-ties may flip late tokens; the first four are the engine test's bar too
    assert torch.equal(got[:, :4], want[:, :4])
    again = greedy_decode(model, prompt, 6)  # the cached engine is reset and reused
    assert torch.equal(again, got)
