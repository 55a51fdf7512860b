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


# -- the reference's standalone ops: deltaforge::delta_rule_step, split_kv_decode_attention --


def _delta_inputs(batch, seed):
    gen = torch.Generator().manual_seed(seed)
    state = torch.randn((batch, 32, 128, 128), generator=gen) * 0.1
    q = torch.nn.functional.normalize(torch.randn((batch, 32, 128), generator=gen), dim=-1) / 128 ** 0.5
    k = torch.nn.functional.normalize(torch.randn((batch, 32, 128), generator=gen), dim=-1)
    v = torch.randn((batch, 32, 128), generator=gen)
    g = -torch.nn.functional.softplus(torch.randn((batch, 32), generator=gen))
    beta = torch.sigmoid(torch.randn((batch, 32), generator=gen))
    return state, q, k, v, g, beta


@pytest.mark.parametrize("batch", [1, 8])
def test_delta_rule_step_op_matches_reference_step(batch):
    """deltaforge_amd::delta_rule_step against the reference loop body (reference.py:450-458):
    fp32 state within 1e-4, fp32 output within atol 2e-2 / rtol 1e-2; the input state is not
    modified (the op returns a new state, as the reference's does)."""
    from oracle.model import delta_rule_step as oracle_step

    inputs = _delta_inputs(batch, 30 + batch)
    want_out, want_state = oracle_step(*inputs)
    dev = [t.to(DEV) for t in inputs]
    before = dev[0].clone()
    out, state = hip_ops.delta_rule_step(*dev)
    assert out.dtype == torch.float32 and out.shape == (batch, 32, 128)
    close(state, want_state, atol=STATE_TOL, rtol=0, what=f"delta_rule_step state B={batch}")
    close(out, want_out, what=f"delta_rule_step out B={batch}")
    assert torch.equal(dev[0], before)


def test_delta_rule_step_in_place_and_sequence():
    """Eight steps in place (state_out = state) equal the oracle's sequential rule over the same
    eight tokens (reference.py:407-461 on pre-normalised inputs)."""
    from deltaforge_amd import ops
    from oracle.model import delta_rule_step as oracle_step

    state, *_ = _delta_inputs(2, 50)
    want = state.clone()
    dstate = state.to(DEV)
    for t in range(8):
        _, q, k, v, g, beta = _delta_inputs(2, 60 + t)
        want_out, want = oracle_step(want, q, k, v, g, beta)
        out, _ = ops.delta_rule_step(dstate, q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV),
                                     state_out=dstate)
    close(dstate, want, atol=STATE_TOL, rtol=0, what="in-place state after 8 steps")
    close(out, want_out, what="output of step 8")


@pytest.mark.parametrize("batch,key_len,splits", [(1, 2048, 8), (32, 2048, 8), (1, 3, 8), (1, 33, 8), (1, 1, 1),
                                                  (2, 4096, 64), (1, 4097, 256)])
def test_split_kv_decode_attention_op_matches_reference(batch, key_len, splits):
    """The reference's cases for the op (flash_decode_splitkv.py:365-372) and more split counts,
    against the reference layer's expression (gqa_decode.py:322-335)."""
    gen = torch.Generator().manual_seed(batch * 1000 + key_len)
    q = torch.randn((batch, 16, 256), generator=gen).to(BF16)
    k = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
    v = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
    want = oracle_ops.decode_attention(q, k, v, 256 ** -0.5)
    got = hip_ops.split_kv_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), 256 ** -0.5, splits)
    assert got.shape == q.shape and got.dtype == BF16
    close(got, want, what=f"split_kv B={batch} L={key_len} S={splits}")


def test_standalone_op_check_builders_pass():
    from deltaforge_amd.kernels import CHECK_BUILDERS

    for name in ("hip_delta_rule_step", "hip_split_kv_decode_attention", "hip_tiled_gemv_int4"):
        for chk in CHECK_BUILDERS[name](None, device=DEV):
            print(chk.name, chk.passed, f"{chk.max_abs_err:.3g}", flush=True)
            assert chk.passed, chk


def test_split_kv_workspace_reused_across_shapes():
    """Calls of different shapes share one workspace (an earlier counter-based merge once let
    a (batch 1, 256 splits) call's partials land on the counters of a later batch-32 call).
    Alternating shapes, each call against the oracle."""
    gen = torch.Generator().manual_seed(11)
    scale = 256 ** -0.5
    for batch, key_len, splits in ((1, 4097, 256), (32, 2048, 8), (1, 4097, 256), (32, 2048, 8), (8, 300, 64)):
        q = torch.randn((batch, 16, 256), generator=gen).to(BF16)
        k = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
        v = torch.randn((batch, 4, key_len, 256), generator=gen).to(BF16)
        want = oracle_ops.decode_attention(q, k, v, scale)
        got = hip_ops.split_kv_decode_attention(q.to(DEV), k.to(DEV), v.to(DEV), scale, splits)
        close(got, want, what=f"split_kv B={batch} L={key_len} S={splits}")


@pytest.mark.parametrize("batch", [1, 3])
def test_delta_step_inputs_match_the_reference_prologue(batch):
    """The inputs the standalone step is composed with, against the oracle's expressions of
    the reference's prologue (l2norm, the Dk^-1/2 scale, key heads repeated over value
    heads, beta = bf16(sigmoid(b)), g = -exp(A_log) softplus(a + dt_bias))."""
    import torch.nn.functional as F

    from deltaforge_amd import ops
    from oracle.model import l2norm

    gen = torch.Generator().manual_seed(40 + batch)
    hk, hv, dk, dv = 16, 32, 128, 128
    mixed = torch.randn((batch, 2 * hk * dk + hv * dv), generator=gen).to(BF16)
    ab = torch.randn((batch, 2 * hv + 5), generator=gen).to(BF16)  # a | b | padding: strided rows
    a, b = ab[:, :hv], ab[:, hv:2 * hv]
    A_log = torch.randn(hv, generator=gen).to(BF16)
    dt_bias = torch.randn(hv, generator=gen).to(BF16)
    got = ops.delta_step_inputs(mixed.to(DEV), ab.to(DEV)[:, :hv], ab.to(DEV)[:, hv:2 * hv], A_log.to(DEV),
                                dt_bias.to(DEV), num_k_heads=hk, head_v_dim=dv)
    q = mixed[:, :hk * dk].float().view(batch, hk, dk).repeat_interleave(hv // hk, dim=1)
    k = mixed[:, hk * dk:2 * hk * dk].float().view(batch, hk, dk).repeat_interleave(hv // hk, dim=1)
    want = (l2norm(q) / dk ** 0.5, l2norm(k), mixed[:, 2 * hk * dk:].float().view(batch, hv, dv),
            -A_log.float().exp() * F.softplus(a.float() + dt_bias.float()), b.sigmoid().float())
    for name, g_, w_ in zip(("query", "key", "value", "g", "beta"), got, want):
        assert g_.dtype == torch.float32 and g_.shape == w_.shape, name
        torch.testing.assert_close(g_.cpu(), w_, atol=2e-6, rtol=2e-6, msg=name)
