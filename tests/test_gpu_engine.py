"""End-to-end decode parity of the HIP engine against the CPU oracle (layer 2).

The mid config keeps Qwen3.5-4B's head geometry (128-wide Gated DeltaNet heads, 256-wide
attention heads, 16/4 and 16/32 head counts, partial RoPE) on a narrow 4-layer stack
(3 linear + 1 full), so every kernel runs at its production head shape while the oracle
finishes in seconds. The check mirrors the reference's layer-2 gate
(harness/correctness.py:383-464): teacher-force both models over prompt + the oracle's
greedy continuation, then score top-1 agreement and mean KL(P_oracle || P_engine) in fp32.
"""

from __future__ import annotations

import pytest
import torch

from deltaforge_amd import synth
from deltaforge_amd.config import mid_config
from deltaforge_amd.engine import DecodeEngine
from deltaforge_amd.harness.correctness import kl_and_agreement
from oracle.int4 import dequantise_int4_k_major
from oracle.model import OracleModel

pytestmark = pytest.mark.gpu


def oracle_for(model: synth.SynthModel) -> OracleModel:
    """The same int4 model as the oracle sees it: every linear int4; the embedding is the model's
    own bf16 table when it has one (a loaded checkpoint), else the dequantised head."""
    params = dict(model.params)
    head = model.linears["lm_head"]
    if "embed_tokens.weight" not in params:
        params["embed_tokens.weight"] = dequantise_int4_k_major(head.packed, head.scale, 128).to(torch.bfloat16).t().contiguous()
    table = {name: (w.packed, w.scale, 128) for name, w in model.linears.items()}
    return OracleModel(model.config, params, table)


@pytest.fixture(scope="module")
def mid():
    cfg = mid_config(4)
    model = synth.synth_model(cfg, seed=5)
    prompt = synth.prompt_ids(cfg.vocab_size, 24, seed=6)
    oracle = oracle_for(model)
    with torch.no_grad():
        ref_tokens, ref_logits = oracle.greedy(prompt, 8)
    return cfg, model, prompt, ref_tokens, ref_logits


def test_engine_teacher_forced_matches_oracle(mid):
    cfg, model, prompt, ref_tokens, ref_logits = mid
    eng = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
    eng.prefill(prompt.cuda())
    got = [eng.logits.float().cpu().clone()]
    for t in range(ref_tokens.shape[1] - 1):
        eng.tokens.copy_(ref_tokens[:, t].cuda())  # teacher forcing with the oracle's continuation
        eng.decode(1)
        got.append(eng.logits.float().cpu().clone())
    got = torch.stack(got, dim=1)  # [1, steps, V]
    kl, agree = kl_and_agreement(ref_logits.float(), got)
    print(f"mid-config layer 2: agreement {float(agree.float().mean()):.4f}, mean KL {float(kl.mean()):.3e} nats, "
          f"max KL {float(kl.max()):.3e}")
    assert float(kl.mean()) < 1e-3
    assert float(agree.float().mean()) >= 7 / 8


def test_engine_greedy_tokens_match_oracle(mid):
    cfg, model, prompt, ref_tokens, _ = mid
    eng = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
    eng.prefill(prompt.cuda())
    first = eng.tokens.clone()
    eng.decode(ref_tokens.shape[1] - 1)
    got = torch.cat([first.cpu().unsqueeze(1), eng.token_log[:, : ref_tokens.shape[1] - 1].cpu()], dim=1)
    # Free-running: report the first divergence (a near-tie can flip; teacher forcing above is the gate).
    diverge = next((i for i in range(got.shape[1]) if got[0, i] != ref_tokens[0, i]), None)
    print(f"greedy tokens: engine {got.tolist()} oracle {ref_tokens.tolist()} first divergence {diverge}")
    assert int(eng.position) == prompt.shape[1] + ref_tokens.shape[1] - 1
    assert diverge is None or diverge >= 4


def test_graph_replay_equals_eager_launches(mid):
    cfg, model, prompt, _, _ = mid
    a = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
    b = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
    a.prefill(prompt.cuda(), graph=True)
    b.prefill(prompt.cuda(), graph=False)
    a.decode(6, graph=True)
    b.decode(6, graph=False)
    torch.cuda.synchronize()
    assert torch.equal(a.token_log[:, :6], b.token_log[:, :6])
    assert torch.equal(a.logits, b.logits)
    for x, y in zip(a.state_tensors(), b.state_tensors()):
        assert torch.equal(x, y)


def test_snapshot_restore_replays_identically(mid):
    cfg, model, prompt, _, _ = mid
    eng = DecodeEngine(model, max_seq_len=64, max_new_tokens=16)
    eng.prefill(prompt.cuda())
    snap = eng.snapshot()
    eng.decode(5)
    first = eng.token_log[:, :5].clone()
    logits = eng.logits.clone()
    eng.restore(snap)
    eng.decode(5)
    assert torch.equal(eng.token_log[:, :5], first)
    assert torch.equal(eng.logits, logits)
