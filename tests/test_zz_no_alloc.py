"""The allocation-free attention entry point (``df_attention_decode_static``) against the
workspace entry point (``df_attention_decode``) it shares its kernel with, through the C ABI:
two calls in a row, the second with a smaller input (fewer sequences, a shorter context,
fewer splits), each compared with the workspace entry point on identical inputs. The static
scratch keeps the first call's contents, so the second call also shows that nothing stale
leaks into it."""

from __future__ import annotations

import ctypes as C

import pytest
import torch

from deltaforge_amd import _native as N
from deltaforge_amd import ops, synth
from deltaforge_amd.config import qwen3_5_4b_config

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _args(inp, kc, vc, position, out, splits):
    cfg = qwen3_5_4b_config()
    inv = synth.inv_freq(cfg).to(DEV)
    q, k, v = inp["q"].to(DEV), inp["k"].to(DEV), inp["v"].to(DEV)
    qn, kn = inp["q_norm_w"].to(DEV), inp["k_norm_w"].to(DEV)
    keep = (q, k, v, qn, kn, inv)
    a = N.AttnDecodeArgs(
        q=q.data_ptr(), k=k.data_ptr(), v=v.data_ptr(), q_norm_w=qn.data_ptr(), k_norm_w=kn.data_ptr(),
        inv_freq=inv.data_ptr(), k_cache=kc.data_ptr(), v_cache=vc.data_ptr(), position=position.data_ptr(),
        out=out.data_ptr(), batch=q.shape[0], ld_q=q.stride(0), ld_kv=k.stride(0), num_q_heads=16, num_kv_heads=4,
        head_dim=256, rotary_dim=64, max_len=kc.shape[2], splits=splits, gate=0, eps=1e-6)
    return a, keep


def _run_both(batch, context, splits, seed):
    print(f"no-alloc attention: B={batch} L={context} splits={splits}", flush=True)
    inp = synth.attention_inputs(seed=seed, batch=batch, context=context, slack=16)
    position = torch.tensor([context], dtype=torch.int32, device=DEV)
    lib = N.lib()
    stream = torch.cuda.current_stream().cuda_stream
    results = []
    for static in (False, True):
        kc, vc = inp["k_cache"].to(DEV), inp["v_cache"].to(DEV)
        out = torch.full((batch, 16 * 256), 7.0, dtype=torch.bfloat16, device=DEV)
        a, keep = _args(inp, kc, vc, position, out, splits)
        if static:
            N.check(lib.df_attention_decode_static(C.byref(a), stream), "attention_decode_static")
        else:
            nbytes = int(lib.df_attention_decode_workspace_bytes(batch, 16, 4, 256, splits))
            ws = torch.zeros(nbytes, dtype=torch.uint8, device=DEV)
            N.check(lib.df_attention_decode(C.byref(a), ws.data_ptr(), nbytes, stream), "attention_decode")
        torch.cuda.synchronize()
        results.append((out.cpu(), kc[:, :, context].cpu(), vc[:, :, context].cpu()))
        del keep
    (o0, k0, v0), (o1, k1, v1) = results
    # same kernel, same inputs, same split count: bit-identical outputs and cache writes
    assert torch.equal(o0, o1), f"B={batch} L={context}: max diff {float((o0.float() - o1.float()).abs().max())}"
    assert torch.equal(k0, k1) and torch.equal(v0, v1)


def test_static_entry_point_matches_workspace_entry_point_twice():
    _run_both(8, 4096, 32, seed=21)
    _run_both(1, 300, 8, seed=22)


def test_static_entry_point_rejects_oversized_calls():
    lib = N.lib()
    cap = int(lib.df_attention_decode_static_capacity())
    assert 8_000_000 < cap < 9_000_000
    inp = synth.attention_inputs(seed=3, batch=1, context=8, slack=8)
    kc, vc = inp["k_cache"].to(DEV), inp["v_cache"].to(DEV)
    position = torch.tensor([8], dtype=torch.int32, device=DEV)
    out = torch.empty((1, 16 * 256), dtype=torch.bfloat16, device=DEV)
    a, keep = _args(inp, kc, vc, position, out, 256)
    a.batch = 3  # 3 x 16 x 256 rows > 8192: refused before any launch
    assert lib.df_attention_decode_static(C.byref(a), torch.cuda.current_stream().cuda_stream) == 3
    del keep
