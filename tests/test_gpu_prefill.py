"""GPU parity of the prompt prefill (csrc/prefill.hip) against the CPU oracle's forward.

Kernel by kernel:
- the int4 GEMM against ``dequant_gemv``, the reference expression;
- the conv bit for bit against ``F.conv1d`` (the oracle's ``causal_conv``);
- the chunked delta rule against the token-by-token scan, at chunk edges (1, 63, 64, 65,
  200 tokens) and from a nonzero state.

Layer by layer, against ``OracleModel._delta_net`` / ``_attention`` with their caches. Then
the whole mid-config model against ``OracleModel.forward``:
- last-position KL and top-1;
- every cache;
- the greedy continuation of a ``PersistentDecoder`` filled by ``Prefiller.fill``.

Bars:
- bf16 outputs atol 2e-2 / rtol 1e-2, the kernel tests' bar;
- fp32 states 1e-4 of their scale for the kernel alone, 1e-3 for one layer, and 2e-2 deep in
  the model, where the inputs already differ by ulps.

The chunked scan reassociates fp32 sums, so nothing beyond the conv is bit-exact.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from deltaforge_amd import _native as N
from deltaforge_amd import ops, synth
from deltaforge_amd.config import FULL_ATTENTION, LINEAR_ATTENTION, mid_config
from deltaforge_amd.harness.correctness import kl_and_agreement
from deltaforge_amd.persistent import PersistentDecoder
from deltaforge_amd.prefill import (Prefiller, causal_conv_prefill, delta_rule_prefill, gated_rms_norm_rows,
                                    int4_gemm)
from oracle.int4 import dequant_gemv
from oracle.model import causal_conv, gated_delta_rule, gated_rms_norm, rope_cos_sin

from .test_gpu_engine import oracle_for
from .test_gpu_kernels import close, repack

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _rel_close(got, want, rel, what):
    got, want = got.float().cpu(), want.float().cpu()
    err = float((got - want).abs().max())
    scale = float(want.abs().max())
    assert err <= rel * max(scale, 1e-30), f"{what}: max err {err:.3g} vs scale {scale:.3g}"


# -- GEMM -----------------------------------------------------------------------------------


@pytest.mark.parametrize("m,k,n", [(1, 256, 64), (77, 512, 192), (300, 2560, 1088), (129, 9216, 256)])
def test_int4_gemm_is_the_dequantised_product(m, k, n):
    print(f"gemm {m}x{k}x{n}", flush=True)
    gen = torch.Generator().manual_seed(m + k + n)
    w = synth.draw_int4(gen, k, n)
    x = torch.randn((m, k), generator=gen).to(torch.bfloat16)
    got = int4_gemm(x.to(DEV), repack(w))
    close(got, dequant_gemv(x, w.packed, w.scale, 128), what=f"gemm {m}x{k}x{n}", flip_frac=1e-3)


def test_int4_gemm_strided_rows_and_swiglu_epilogue():
    gen = torch.Generator().manual_seed(3)
    m, k, inter = 150, 512, 320
    gate, up = synth.draw_int4(gen, k, inter), synth.draw_int4(gen, k, inter)
    wide = torch.randn((m, k + 64), generator=gen).to(torch.bfloat16)
    x = wide[:, 32:32 + k]  # row stride k + 64, 64-byte offset
    gp, gs = ops.interleave_gate_up(gate.packed, gate.scale, up.packed, up.scale)
    gu = ops.int4_repack(gp.to(DEV), gs.to(DEV))
    got = int4_gemm(wide.to(DEV)[:, 32:32 + k], gu, epilogue=N.EPI_SWIGLU)
    want = F.silu(dequant_gemv(x, gate.packed, gate.scale, 128)) * dequant_gemv(x, up.packed, up.scale, 128)
    close(got, want, what="gate|up + SwiGLU", flip_frac=2e-3)


def test_int4_gemm_rejects_bad_shapes():
    gen = torch.Generator().manual_seed(4)
    w = repack(synth.draw_int4(gen, 256, 64))
    with pytest.raises(ValueError):
        int4_gemm(torch.zeros((4, 128), dtype=torch.bfloat16, device=DEV), w)
    with pytest.raises(RuntimeError):
        int4_gemm(torch.zeros((4, 256), dtype=torch.bfloat16), w)


# -- conv, delta rule, gated norm ----------------------------------------------------------


@pytest.mark.parametrize("tokens,pos0", [(1, 0), (2, 0), (37, 0), (37, 5)])
def test_causal_conv_prefill_is_conv1d(tokens, pos0):
    gen = torch.Generator().manual_seed(tokens + pos0)
    channels = 8192
    x = torch.randn((tokens, channels), generator=gen).to(torch.bfloat16)
    w = (torch.randn((channels, 1, 4), generator=gen) * 0.3).to(torch.bfloat16)
    hist = torch.zeros((1, channels, 3), dtype=torch.bfloat16)
    ring = torch.zeros((channels, 4), dtype=torch.bfloat16)
    if pos0:
        hist = torch.randn((1, channels, 3), generator=gen).to(torch.bfloat16)
        for j in range(3):  # positions pos0-3 .. pos0-1
            ring[:, (pos0 - 3 + j) % 4] = hist[0, :, j]
    ring_d = ring.to(DEV)
    got = causal_conv_prefill(x.to(DEV), w.reshape(channels, 4).to(DEV), ring_d, pos0=pos0)
    want, new_hist = causal_conv(x.t().unsqueeze(0), hist, w)
    assert torch.equal(got.cpu(), want[0].t()), "conv output"
    ring_h = ring_d.cpu()
    end = pos0 + tokens
    got_hist = torch.stack([ring_h[:, (end - 3 + j) % 4] for j in range(3)], dim=-1)
    assert torch.equal(got_hist, new_hist[0]), "history ring"


def _delta_case(tokens, seed, hk=16, hv=32):
    gen = torch.Generator().manual_seed(seed)
    mixed = (torch.randn((tokens, (2 * hk + hv) * 128), generator=gen)).to(torch.bfloat16)
    ab = torch.randn((tokens, 2 * hv + 8), generator=gen).to(torch.bfloat16)
    A_log = (torch.randn(hv, generator=gen) * 0.5).to(torch.bfloat16)
    dt_bias = (torch.randn(hv, generator=gen) * 0.5).to(torch.bfloat16)
    state = torch.randn((hv, 128, 128), generator=gen) * 0.1
    return mixed, ab, A_log, dt_bias, state


def _delta_oracle(mixed, ab, A_log, dt_bias, state, hk, hv):
    """The oracle's _delta_net between the conv and the gated norm (reference.py:518-545)."""
    tokens = mixed.shape[0]
    q, k, v = torch.split(mixed.unsqueeze(0), [hk * 128, hk * 128, hv * 128], dim=-1)
    q = q.reshape(1, tokens, hk, 128).repeat_interleave(hv // hk, dim=2)
    k = k.reshape(1, tokens, hk, 128).repeat_interleave(hv // hk, dim=2)
    v = v.reshape(1, tokens, hv, 128)
    a, b = ab[:, :hv].unsqueeze(0), ab[:, hv:2 * hv].unsqueeze(0)
    beta = b.sigmoid()
    g = -A_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    out, new_state = gated_delta_rule(q, k, v, g, beta, state.unsqueeze(0))
    return out[0].reshape(tokens, hv * 128), new_state[0]


@pytest.mark.parametrize("tokens", [1, 63, 64, 65, 200])
def test_delta_rule_prefill_matches_the_scan(tokens):
    print(f"delta prefill {tokens}", flush=True)
    hk, hv = 16, 32
    mixed, ab, A_log, dt_bias, state = _delta_case(tokens, seed=tokens)
    st = state.to(DEV).contiguous()
    ab_d = ab.to(DEV)
    got = delta_rule_prefill(mixed.to(DEV), ab_d[:, :hv], ab_d[:, hv:], A_log.to(DEV), dt_bias.to(DEV), st,
                             num_k_heads=hk)
    want, want_state = _delta_oracle(mixed, ab, A_log, dt_bias, state, hk, hv)
    close(got, want, what=f"delta out P={tokens}", flip_frac=1e-3)
    _rel_close(st, want_state, 1e-4, f"delta state P={tokens}")


def test_gated_rms_norm_rows():
    gen = torch.Generator().manual_seed(9)
    tokens, heads = 70, 32
    x = torch.randn((tokens, heads * 128), generator=gen).to(torch.bfloat16)
    zw = torch.randn((tokens, heads * 128 + 64), generator=gen).to(torch.bfloat16)
    w = (1.0 + 0.02 * torch.randn(128, generator=gen)).to(torch.bfloat16)
    got = gated_rms_norm_rows(x.to(DEV), zw.to(DEV)[:, 64:], w.to(DEV), 1e-6)
    want = gated_rms_norm(x.reshape(-1, 128), zw[:, 64:].reshape(-1, 128), w, 1e-6).reshape(tokens, -1)
    close(got, want, what="gated norm rows")


# -- layers and the model -------------------------------------------------------------------


@pytest.fixture(scope="module")
def mid():
    cfg = mid_config(4)
    model = synth.synth_model(cfg, seed=21, symmetric=True)
    return cfg, model, oracle_for(model), Prefiller(model)


def _caches(cfg, max_len):
    out = []
    for kind in cfg.layer_types:
        if kind == FULL_ATTENTION:
            k = torch.zeros((cfg.num_key_value_heads, max_len, cfg.head_dim), dtype=torch.bfloat16, device=DEV)
            out.append({"k_cache": k, "v_cache": torch.zeros_like(k)})
        else:
            out.append({"conv_ring": torch.zeros((cfg.linear_conv_dim, 4), dtype=torch.bfloat16, device=DEV),
                        "state": torch.zeros((cfg.linear_num_value_heads, 128, 128), dtype=torch.float32,
                                             device=DEV)})
    return out


@pytest.mark.parametrize("kind", [LINEAR_ATTENTION, FULL_ATTENTION])
def test_one_layer_against_the_oracle(mid, kind):
    """One token mixer over 150 tokens (two full chunks and a partial): its output and its
    cache, from the input-normed rows."""
    cfg, model, oracle, pre = mid
    i = cfg.layer_types.index(kind)
    tokens, max_len = 150, 192
    gen = torch.Generator().manual_seed(30 + i)
    x = torch.randn((1, tokens, cfg.hidden_size), generator=gen).to(torch.bfloat16)
    ocache = oracle.new_cache(1, max_len)
    caches = _caches(cfg, max_len)
    layer = pre.layers[i]
    xd = x[0].to(DEV)
    from deltaforge_amd import prefill as P

    if kind == LINEAR_ATTENTION:
        want = oracle._delta_net(i, x, ocache.layers[i])[0]
        c = cfg
        proj = int4_gemm(xd, layer["proj"])
        conv_c, vd, hv = c.linear_conv_dim, c.linear_value_dim, c.linear_num_value_heads
        mixed = causal_conv_prefill(proj[:, :conv_c], layer["conv_w"], caches[i]["conv_ring"])
        core = delta_rule_prefill(mixed, proj[:, conv_c + vd:], proj[:, conv_c + vd + hv:], layer["A_log"],
                                  layer["dt_bias"], caches[i]["state"], num_k_heads=c.linear_num_key_heads)
        y = gated_rms_norm_rows(core, proj[:, conv_c:conv_c + vd], layer["gnorm_w"], c.rms_norm_eps)
        got = int4_gemm(y, layer["out"])
        close(got, want, what="DeltaNet layer", flip_frac=5e-3)
        _rel_close(caches[i]["state"], ocache.layers[i]["recurrent"][0], 1e-3, "recurrent state")
        ring = caches[i]["conv_ring"].cpu()
        hist = torch.stack([ring[:, (tokens - 3 + j) % 4] for j in range(3)], dim=-1)
        close(hist, ocache.layers[i]["conv"][0], what="conv history", flip_frac=1e-3)
    else:
        positions = torch.arange(tokens).unsqueeze(0)
        cos, sin = rope_cos_sin(positions, cfg, torch.bfloat16, inv_freq_dtype=torch.bfloat16)
        want = oracle._attention(i, x, cos, sin, ocache.layers[i], 0)[0]
        qd, kvd = 2 * cfg.num_attention_heads * cfg.head_dim, cfg.num_key_value_heads * cfg.head_dim
        proj = int4_gemm(xd, layer["proj"])
        q = P.qk_norm_rope_prefill(proj, layer["q_norm"], layer["k_norm"], pre.inv_freq, caches[i]["k_cache"],
                                   caches[i]["v_cache"], num_q_heads=cfg.num_attention_heads, k_col=qd,
                                   v_col=qd + kvd)
        attn = P.attention_prefill(q, caches[i]["k_cache"], caches[i]["v_cache"], proj[:, cfg.head_dim:],
                                   gate_head_stride=2 * cfg.head_dim)
        got = int4_gemm(attn, layer["out"])
        close(got, want, what="attention layer", flip_frac=5e-3)
        close(caches[i]["k_cache"][:, :tokens].cpu(), ocache.layers[i]["keys"][0, :, :tokens], what="k cache",
              flip_frac=1e-3)
        close(caches[i]["v_cache"][:, :tokens].cpu(), ocache.layers[i]["values"][0, :, :tokens], what="v cache",
              flip_frac=1e-3)


@pytest.mark.parametrize("tokens", [1, 100])
def test_prefill_logits_and_caches_match_the_oracle_forward(mid, tokens):
    cfg, model, oracle, pre = mid
    prompt = synth.prompt_ids(cfg.vocab_size, tokens, seed=40 + tokens)
    ocache = oracle.new_cache(1, 128)
    with torch.no_grad():
        want = oracle.forward(prompt, ocache)[:, -1]
    caches = _caches(cfg, 128)
    got = pre.forward(prompt[0].to(DEV), caches)
    kl, agree = kl_and_agreement(want.float().unsqueeze(1), got.float().cpu().unsqueeze(1))
    print(f"prefill P={tokens}: KL {float(kl.mean()):.3e}, top-1 agrees {bool(agree.all())}", flush=True)
    assert float(kl.mean()) < 1e-3 and bool(agree.all())
    for i, kind in enumerate(cfg.layer_types):
        # a deeper layer's input has passed through earlier layers whose bf16 outputs differ
        # from the oracle's by summation-order ulps, so its caches are held normwise (the largest
        # error against the largest value); the single-layer test holds them elementwise
        if kind == FULL_ATTENTION:
            _rel_close(caches[i]["k_cache"][:, :tokens], ocache.layers[i]["keys"][0, :, :tokens], 2e-2,
                       f"layer {i} keys")
            _rel_close(caches[i]["v_cache"][:, :tokens], ocache.layers[i]["values"][0, :, :tokens], 2e-2,
                       f"layer {i} values")
        else:
            _rel_close(caches[i]["state"], ocache.layers[i]["recurrent"][0], 2e-2, f"layer {i} state")


def _teacher_forced(dec, ref_tokens):
    got = [dec.logits.float().cpu().clone()]
    for t in range(ref_tokens.shape[1] - 1):
        dec.tokens.copy_(ref_tokens[:, t].to(DEV))  # teacher forcing with the oracle's continuation
        dec.decode(1)
        dec.check()
        got.append(dec.logits.float().cpu().clone())
    return torch.stack(got, dim=1)


def test_filled_persistent_decoder_continues_like_the_oracle(mid):
    """The same decoder, prefilled token by token (its own launch) and by ``Prefiller.fill``,
    teacher-forced through the oracle's greedy continuation. The filled one must agree on top-1
    and stay within twice the own-prefill decoder's KL (this symmetric-weight model's noise
    floor against the oracle), or 1e-3 if that is larger."""
    cfg, model, oracle, pre = mid
    prompt = synth.prompt_ids(cfg.vocab_size, 90, seed=50)
    with torch.no_grad():
        ref_tokens, ref_logits = oracle.greedy(prompt, 8)
    own = PersistentDecoder(model, max_seq_len=128, max_new_tokens=16)
    own.prefill(prompt.to(DEV))
    own.check()
    kl_own, agree_own = kl_and_agreement(ref_logits.float(), _teacher_forced(own, ref_tokens))
    dec = PersistentDecoder(model, max_seq_len=128, max_new_tokens=16)
    pre.fill(dec, prompt.to(DEV))
    kl, agree = kl_and_agreement(ref_logits.float(), _teacher_forced(dec, ref_tokens))
    print(f"own prefill: agreement {float(agree_own.float().mean()):.4f}, KL {float(kl_own.mean()):.3e}; "
          f"filled: agreement {float(agree.float().mean()):.4f}, KL {float(kl.mean()):.3e}", flush=True)
    assert float(kl.mean()) < max(1e-3, 2 * float(kl_own.mean()))
    assert float(agree.float().mean()) >= min(7 / 8, float(agree_own.float().mean()))


def test_fill_in_chunks_equals_one_pass(mid):
    """``Prefiller.fill`` runs a long prompt in chunks (positions continuing from the caches).
    With chunk boundaries on the delta rule's 64-token chunks the arithmetic is the single
    pass's, so 200 tokens filled 64 at a time must leave bit-identical caches, logits and first
    token; chunk sizes off that grid are refused."""
    cfg, model, oracle, pre = mid
    prompt = synth.prompt_ids(cfg.vocab_size, 200, seed=60).to(DEV)
    one = PersistentDecoder(model, max_seq_len=256, max_new_tokens=16)
    pre.fill(one, prompt)
    parts = PersistentDecoder(model, max_seq_len=256, max_new_tokens=16)
    pre.fill(parts, prompt, chunk=64)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(one.layer_state, parts.layer_state)):
        for name in a:
            assert torch.equal(a[name], b[name]), f"layer {i} {name}"
    assert torch.equal(one.logits, parts.logits) and torch.equal(one.tokens, parts.tokens)
    assert int(parts.position.item()) == 200
    for bad in (32, 100, 65536):
        with pytest.raises(ValueError):
            pre.fill(parts, prompt, chunk=bad)
