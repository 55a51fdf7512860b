"""Pins of the CPU oracle that do not go through the reference's golden vectors.

Each check is independent of the function it pins (a closed form, a brute force, a known
answer, or the golden-pinned ``OracleModel`` path), chosen so a plausible slip -- a dropped
term, a sign, a swapped nibble, a transposed operand -- fails:

* int4: brute force over all 256 byte values x scales (integer/float64 arithmetic), the
  K-major pairing (reference tiled_gemv.py:242-288), quantiser range and round trip;
* RMSNorm (1 + w) known answer (reference reference_test.py:113-129), rotate_half, RoPE at
  position 0, the partial-RoPE tail;
* causal conv known answer (reference inline_causal_conv_test.py:94-109);
* delta rule: float64 closed form, step == whole == two chunks, beta = 0, causality
  (reference reference_test.py:230-306);
* ``oracle.ops`` per-config compositions against ``OracleModel``'s own layers (which the
  golden vectors pin bit-for-bit against the reference).
"""

from __future__ import annotations

import math

import numpy as np
import torch

from deltaforge_amd.config import mid_config
from deltaforge_amd.synth import synth_model
from oracle import ops as oracle_ops
from oracle.int4 import (
    bf16_bits_from_f32,
    dequant_gemv,
    dequantise_int4_k_major,
    dequantise_int4_k_major_np,
    quantise_int4_k_major,
)
from oracle.model import (
    OracleModel,
    apply_partial_rope,
    causal_conv,
    gated_delta_rule,
    gated_rms_norm,
    rms_norm,
    rope_cos_sin,
    rotate_half,
)

BF16 = torch.bfloat16


# -- int4 -----------------------------------------------------------------------------------


def _bf16_rne_from_float64(v: float) -> int:
    """Round a float64 (here always exactly representable in fp32) to bf16 bits, by hand."""
    f32 = np.float32(v)
    assert float(f32) == v
    bits = int(np.array([f32]).view(np.uint32)[0])
    return ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) & 0xFFFF


def test_int4_dequant_brute_force_all_bytes():
    rng = np.random.default_rng(0)
    scales = np.concatenate([
        np.array([1.0, 0.5, 3.0, 1e-3, 7.25, 1e-30, 1e30], dtype=np.float32),
        (rng.standard_normal(25) * 0.02).astype(np.float32),
    ])
    sbits = bf16_bits_from_f32(scales)  # scales as stored (bf16)
    packed = np.arange(256, dtype=np.uint8).reshape(128, 2).repeat(16, axis=1)  # [128, 32]: K=256, N=32
    n = packed.shape[1]
    scale_bits = np.tile(sbits[:n], (2, 1)).astype(np.uint16)  # [2, 32]
    got = dequantise_int4_k_major_np(packed, scale_bits, 128)
    tq = dequantise_int4_k_major(torch.from_numpy(packed), torch.from_numpy(scale_bits.view(np.int16)).view(BF16), 128)
    assert np.array_equal(tq.to(BF16).view(torch.int16).numpy().view(np.uint16), got)
    for j in range(128):
        for c in range(n):
            byte = int(packed[j, c])
            s = float(np.array([int(scale_bits[0, c]) << 16], dtype=np.uint32).view(np.float32)[0])
            lo_want = _bf16_rne_from_float64(((byte & 0xF) - 8) * s)
            hi_s = float(np.array([int(scale_bits[1, c]) << 16], dtype=np.uint32).view(np.float32)[0])
            hi_want = _bf16_rne_from_float64(((byte >> 4) - 8) * hi_s)
            assert got[j, c] == lo_want, (j, c)  # low nibble is row j
            assert got[j + 128, c] == hi_want, (j, c)  # high nibble is row j + K/2


def test_int4_k_major_pairing_and_group_scales():
    k, n = 512, 16
    packed = torch.zeros((k // 2, n), dtype=torch.uint8)
    packed[3, 5] = 0x9C  # low nibble 12 (+4) at k=3, high nibble 9 (+1) at k=259
    scale = torch.ones((k // 128, n), dtype=BF16)
    scale[0, 5] = 0.5
    scale[2, 5] = 2.0  # k=259 is in group 2
    w = dequantise_int4_k_major(packed, scale, 128)
    assert w[3, 5] == 4 * 0.5 and w[259, 5] == 1 * 2.0
    assert w[0, 0] == -8.0  # nibble 0 is -8
    x = torch.zeros((1, k), dtype=BF16)
    x[0, 259] = 1.0
    assert float(dequant_gemv(x, packed, scale, 128)[0, 5]) == 2.0


def test_quantiser_range_and_round_trip():
    gen = torch.Generator().manual_seed(1)
    weight = torch.randn((64, 512), generator=gen)
    packed, scale, group = quantise_int4_k_major(weight, scale_dtype=torch.float32)
    nib = torch.cat((packed & 0xF, packed >> 4), 0)
    assert int(nib.min()) >= 1 and int(nib.max()) <= 15  # symmetric [-7, 7] + 8: nibble 0 never
    back = dequantise_int4_k_major(packed, scale, group).t()
    s_full = scale.t().repeat_interleave(group, dim=1)
    assert bool(((back - weight).abs() <= s_full / 2 + 1e-7).all())


# -- norms, RoPE, conv ------------------------------------------------------------------------


def test_rms_norm_known_answer_one_plus_weight():
    x = torch.tensor([[1.0, 2.0, 3.0, 4.0]])
    rms = 1.0 / math.sqrt((1 + 4 + 9 + 16) / 4 + 1e-6)
    torch.testing.assert_close(rms_norm(x, torch.zeros(4), 1e-6), x * rms)
    torch.testing.assert_close(rms_norm(x, torch.ones(4), 1e-6), x * rms * 2.0)


def test_gated_rms_norm_closed_form():
    x = torch.tensor([[3.0, -4.0]], dtype=torch.float32)
    z = torch.tensor([[0.0, 2.0]])
    w = torch.tensor([2.0, 0.5])
    r = 1.0 / math.sqrt((9 + 16) / 2 + 1e-6)
    want = torch.tensor([[2.0 * 3.0 * r * 0.0, 0.5 * -4.0 * r * (2.0 / (1.0 + math.exp(-2.0)))]])
    torch.testing.assert_close(gated_rms_norm(x, z, w, 1e-6), want)


def test_rotate_half_and_rope_identity_at_zero():
    assert torch.equal(rotate_half(torch.tensor([1.0, 2.0, 3.0, 4.0])), torch.tensor([-3.0, -4.0, 1.0, 2.0]))
    cfg = mid_config(4)
    cos, sin = rope_cos_sin(torch.zeros((1, 1), dtype=torch.long), cfg, torch.float32)
    x = torch.randn((1, 2, 1, cfg.head_dim))
    assert torch.equal(apply_partial_rope(x, cos, sin), x)
    cos, sin = rope_cos_sin(torch.full((1, 1), 37, dtype=torch.long), cfg, torch.float32)
    y = apply_partial_rope(x, cos, sin)
    assert torch.equal(y[..., cfg.rotary_dim:], x[..., cfg.rotary_dim:])  # tail passes through
    assert not torch.equal(y[..., :cfg.rotary_dim], x[..., :cfg.rotary_dim])
    # rotation preserves each (i, i + R/2) pair's norm
    half = cfg.rotary_dim // 2
    n0 = x[..., :half] ** 2 + x[..., half:cfg.rotary_dim] ** 2
    n1 = y[..., :half] ** 2 + y[..., half:cfg.rotary_dim] ** 2
    torch.testing.assert_close(n0, n1)


def test_causal_conv_known_answer():
    hist = torch.tensor([[[1.0, 2.0, 3.0]]])
    w = torch.tensor([[[0.5, -1.0, 2.0, 0.25]]])
    out, new_hist = causal_conv(torch.tensor([[[4.0]]]), hist, w)
    assert torch.equal(new_hist, torch.tensor([[[2.0, 3.0, 4.0]]]))
    acc = 1 * 0.5 + 2 * -1.0 + 3 * 2.0 + 4 * 0.25
    torch.testing.assert_close(out, torch.tensor([[[acc / (1 + math.exp(-acc))]]]))


# -- delta rule -------------------------------------------------------------------------------


def _delta_inputs(steps, heads=3, dk=8, dv=5, seed=0):
    gen = torch.Generator().manual_seed(seed)
    return dict(
        query=torch.randn((1, steps, heads, dk), generator=gen),
        key=torch.randn((1, steps, heads, dk), generator=gen),
        value=torch.randn((1, steps, heads, dv), generator=gen),
        g=-torch.rand((1, steps, heads), generator=gen),
        beta=torch.rand((1, steps, heads), generator=gen),
    )


def _delta_float64(query, key, value, g, beta, state=None):
    """Independent float64 restatement, element loops (reference.py:407-461)."""
    _, steps, heads, dk = query.shape
    dv = value.shape[-1]
    s = np.zeros((heads, dk, dv)) if state is None else state[0].double().numpy().copy()
    out = np.zeros((steps, heads, dv))
    for t in range(steps):
        for h in range(heads):
            q = query[0, t, h].double().numpy()
            k = key[0, t, h].double().numpy()
            q = q / math.sqrt((q * q).sum() + 1e-6) / math.sqrt(dk)
            k = k / math.sqrt((k * k).sum() + 1e-6)
            s[h] *= math.exp(float(g[0, t, h]))
            for j in range(dv):
                recalled = sum(s[h, i, j] * k[i] for i in range(dk))
                d = (float(value[0, t, h, j]) - recalled) * float(beta[0, t, h])
                for i in range(dk):
                    s[h, i, j] += k[i] * d
                out[t, h, j] = sum(s[h, i, j] * q[i] for i in range(dk))
    return out, s


def test_delta_rule_matches_float64_closed_form():
    inp = _delta_inputs(4)
    out, state = gated_delta_rule(**inp)
    want, want_state = _delta_float64(**inp)
    np.testing.assert_allclose(out[0].double().numpy(), want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(state[0].double().numpy(), want_state, rtol=1e-5, atol=1e-6)


def test_delta_rule_step_equals_whole_equals_chunks():
    inp = _delta_inputs(9)
    whole, whole_state = gated_delta_rule(**inp)
    outs, state = [], None
    for t in range(9):
        o, state = gated_delta_rule(**{k: v[:, t:t + 1] for k, v in inp.items()}, initial_state=state)
        outs.append(o)
    torch.testing.assert_close(torch.cat(outs, 1), whole, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(state, whole_state, rtol=1e-5, atol=1e-6)
    a, st = gated_delta_rule(**{k: v[:, :4] for k, v in inp.items()})
    b, st = gated_delta_rule(**{k: v[:, 4:] for k, v in inp.items()}, initial_state=st)
    torch.testing.assert_close(torch.cat((a, b), 1), whole, rtol=1e-5, atol=1e-6)


def test_delta_rule_zero_beta_and_causality():
    inp = _delta_inputs(3)
    inp["beta"] = torch.zeros_like(inp["beta"])
    out, state = gated_delta_rule(**inp)
    assert float(out.abs().max()) == 0.0 and float(state.abs().max()) == 0.0
    inp = _delta_inputs(6)
    base, _ = gated_delta_rule(**inp)
    inp["value"][:, 3] += 10.0
    after, _ = gated_delta_rule(**inp)
    torch.testing.assert_close(after[:, :3], base[:, :3], rtol=0, atol=0)
    assert not torch.allclose(after[:, 3], base[:, 3])


# -- oracle.ops compositions vs the golden-pinned OracleModel layers ---------------------------


def _mid_model():
    cfg = mid_config(4)
    m = synth_model(cfg, seed=9)
    params = dict(m.params)
    head = m.linears["lm_head"]
    params["embed_tokens.weight"] = dequantise_int4_k_major(head.packed, head.scale, 128).to(BF16).t().contiguous()
    return cfg, m, OracleModel(cfg, params, {n: (w.packed, w.scale, 128) for n, w in m.linears.items()})


def test_ops_delta_step_is_the_model_layer():
    cfg, m, model = _mid_model()
    i = cfg.layer_types.index("linear_attention")
    p = f"layers.{i}.linear_attn."
    gen = torch.Generator().manual_seed(2)
    h = torch.randn((1, 1, cfg.hidden_size), generator=gen).to(BF16)
    c = cfg.linear_conv_dim
    cache = {"conv": (torch.randn((1, c, 3), generator=gen) * 0.5).to(BF16),
             "recurrent": torch.randn((1, cfg.linear_num_value_heads, 128, 128), generator=gen) * 0.1}
    conv0, state0 = cache["conv"].clone(), cache["recurrent"].clone()
    want = model._delta_net(i, h, cache)
    qkv = model.linear(h, p + "in_proj_qkv.weight")[:, 0]
    a = model.linear(h, p + "in_proj_a.weight")[:, 0]
    b = model.linear(h, p + "in_proj_b.weight")[:, 0]
    z = model.linear(h, p + "in_proj_z.weight")[:, 0]
    out, state, hist = oracle_ops.delta_step(qkv, conv0, m.params[p + "conv1d.weight"], a, b, m.params[p + "A_log"],
                                             m.params[p + "dt_bias"], state0, cfg.linear_num_key_heads)
    core = gated_rms_norm(out.reshape(-1, 128), z.reshape(-1, 128), m.params[p + "norm.weight"], cfg.rms_norm_eps)
    got = model.linear(core.reshape(1, 1, -1), p + "out_proj.weight")
    assert torch.equal(got, want)
    assert torch.equal(state, cache["recurrent"]) and torch.equal(hist, cache["conv"])


def test_ops_attention_decode_is_the_model_layer():
    cfg, m, model = _mid_model()
    i = cfg.layer_types.index("full_attention")
    p = f"layers.{i}.self_attn."
    gen = torch.Generator().manual_seed(3)
    pos, max_len = 9, 16
    h = torch.randn((1, 1, cfg.hidden_size), generator=gen).to(BF16)
    kc = torch.randn((1, cfg.num_key_value_heads, max_len, cfg.head_dim), generator=gen).to(BF16)
    vc = torch.randn((1, cfg.num_key_value_heads, max_len, cfg.head_dim), generator=gen).to(BF16)
    cache = {"keys": kc.clone(), "values": vc.clone()}
    cos, sin = rope_cos_sin(torch.full((1, 1), pos, dtype=torch.long), cfg, BF16, inv_freq_dtype=BF16)
    want = model._attention(i, h, cos, sin, cache, pos)
    attn = oracle_ops.attention_decode(model.linear(h, p + "q_proj.weight")[:, 0], model.linear(h, p + "k_proj.weight")[:, 0],
                                       model.linear(h, p + "v_proj.weight")[:, 0], m.params[p + "q_norm.weight"],
                                       m.params[p + "k_norm.weight"], kc, vc, pos, cfg)
    got = model.linear(attn.reshape(1, 1, -1), p + "o_proj.weight")
    assert torch.equal(got, want)
    assert torch.equal(kc[:, :, :pos + 1], cache["keys"][:, :, :pos + 1])


def test_ops_mlp_and_head_are_the_model_path():
    cfg, m, model = _mid_model()
    gen = torch.Generator().manual_seed(4)
    x = torch.randn((2, cfg.hidden_size), generator=gen).to(BF16)
    pre = "layers.0.mlp."
    nw = m.params["layers.0.post_attention_layernorm.weight"]
    want = x + model._mlp(0, rms_norm(x, nw, cfg.rms_norm_eps))
    lin = m.linears
    got = oracle_ops.mlp_block(x, nw, (lin[pre + "gate_proj.weight"].packed, lin[pre + "gate_proj.weight"].scale),
                               (lin[pre + "up_proj.weight"].packed, lin[pre + "up_proj.weight"].scale),
                               (lin[pre + "down_proj.weight"].packed, lin[pre + "down_proj.weight"].scale), cfg.rms_norm_eps)
    assert torch.equal(got, want)
    r = torch.randn((2, cfg.hidden_size), generator=gen).to(BF16)
    fn = m.params["norm.weight"]
    want = model.project_logits(rms_norm(r + x, fn, cfg.rms_norm_eps))
    got = oracle_ops.head(x, r, fn, lin["lm_head"].packed, lin["lm_head"].scale, 128, cfg.rms_norm_eps)
    assert torch.equal(got, want)


def test_dequant_gemv_variants_are_the_stated_changes():
    """The sensitivity probes of the full-size parity test change one arithmetic choice each:
    the default variant is the reference expression bit for bit; float64 accumulation of the
    same bf16 weights and the exact (unrounded) weights agree with a float64 dense product."""
    import functools

    from deltaforge_amd.synth import draw_int4
    from oracle.int4 import dequant_gemv, dequant_gemv_variant, dequantise_int4_k_major

    gen = torch.Generator().manual_seed(9)
    w = draw_int4(gen, 512, 96, symmetric=True)
    x = torch.randn((3, 512), generator=gen).to(torch.bfloat16)
    assert torch.equal(dequant_gemv_variant(x, w.packed, w.scale, 128), dequant_gemv(x, w.packed, w.scale, 128))
    exact = dequantise_int4_k_major(w.packed, w.scale, 128).double()
    rounded = exact.to(torch.bfloat16).double()
    f64 = functools.partial(dequant_gemv_variant, accumulate=torch.float64)
    assert torch.equal(f64(x, w.packed, w.scale, 128), (x.double() @ rounded).to(torch.bfloat16))
    ex = dequant_gemv_variant(x, w.packed, w.scale, 128, round_weights=False).double()
    want = x.double() @ exact
    assert float((ex - want).abs().max()) <= float(want.abs().max()) * 2 ** -8
    # symmetric draws never hold nibble 0 (n - 8 = -8)
    assert int((w.packed & 0x0F).min()) >= 1 and int((w.packed >> 4).min()) >= 1
