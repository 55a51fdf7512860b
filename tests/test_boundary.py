"""The drop-in boundary on the CPU: the C ABI's exported surface, the registry's invariants,
the custom ops' error order and fake kernels, and champion installation.

Nothing here launches a kernel; the GPU parity of the same ops is in test_gpu_boundary.py.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest
import torch

from deltaforge_amd import _native as N
from deltaforge_amd.config import mid_config
from deltaforge_amd.kernels import (
    REGISTRY,
    REPLACEABLE_OPS,
    KernelRegistry,
    KernelStatus,
    RegistryError,
    hip_ops,
)
from deltaforge_amd.model import INSTALLERS, InstallerMissing, apply_champions, greedy_decode

ROOT = Path(__file__).resolve().parents[1]
BF16 = torch.bfloat16


def header_symbols() -> set[str]:
    names = set()
    for h in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names |= set(re.findall(r"^\s*(?:int|size_t|void)\s+(df_\w+)\s*\(", text, flags=re.M))
    return names


@pytest.fixture(scope="module")
def built_library() -> ctypes.CDLL:
    if not N.LIB_PATH.exists():
        from deltaforge_amd import build

        build.build()
    return ctypes.CDLL(str(N.LIB_PATH))


def test_library_exports_every_header_symbol(built_library):
    names = header_symbols()
    assert len(names) >= 17, names
    missing = [n for n in sorted(names) if not hasattr(built_library, n)]
    assert not missing, f"declared in include/ but not exported: {missing}"
    # and the ctypes table binds exactly the declared surface
    assert set(N.SIGNATURES) <= names, set(N.SIGNATURES) - names


def test_python_binding_loads(built_library):
    lib = N.lib()  # no device call happens at load time
    for name in N.SIGNATURES:
        assert getattr(lib, name).restype is not None or True


# -- registry -----------------------------------------------------------------------------


def test_replaceable_ops_are_the_reference_slots():
    # reference kernels/__init__.py:56-80
    assert REPLACEABLE_OPS == {
        "rms_norm", "rms_norm_residual", "swiglu_mlp", "qkv_projection_rope", "gated_delta_rule",
        "gqa_attention", "kv_cache_update", "decode_step", "causal_conv", "decode_cache",
    }


def test_one_champion_per_op_and_promote_swaps_atomically():
    reg = KernelRegistry()
    reg.register("a", impl=lambda: None, replaces="rms_norm", status=KernelStatus.CHAMPION)
    with pytest.raises(RegistryError):
        reg.register("b", impl=lambda: None, replaces="rms_norm", status=KernelStatus.CHAMPION)
    reg.register("b", impl=lambda: None, replaces="rms_norm")
    reg.promote("b")
    assert reg.champion("rms_norm").name == "b"
    assert reg.get("a").status is KernelStatus.RETIRED
    with pytest.raises(RegistryError):
        reg.register("c", impl=lambda: None, replaces="no_such_op")
    with pytest.raises(RegistryError):
        reg.register("b", impl=lambda: None, replaces="rms_norm")
    reg.check_invariants()


def test_shipped_champions_cover_the_hot_path():
    REGISTRY.check_invariants()
    champs = {op: e.name for op, e in REGISTRY.champions().items()}
    for op in ("decode_step", "swiglu_mlp", "rms_norm", "rms_norm_residual", "qkv_projection_rope",
               "causal_conv", "gated_delta_rule", "gqa_attention", "decode_cache"):
        assert op in champs, op
    for name in champs.values():
        assert name in INSTALLERS, f"champion {name} has no installer"


def test_apply_champions_refuses_a_champion_without_installer():
    reg = KernelRegistry()
    reg.register("orphan", impl=lambda: None, replaces="rms_norm", status=KernelStatus.CHAMPION)
    with pytest.raises(InstallerMissing):
        apply_champions(object(), reg, installers={})


def test_apply_champions_installs_the_decode_loop():
    from deltaforge_amd.synth import synth_model

    model = synth_model(mid_config(num_layers=4), seed=0)
    applied = apply_champions(model)
    assert set(applied) == {e.name for e in REGISTRY.champions().values()}
    assert callable(model.decode_loop)
    with pytest.raises(ValueError):
        greedy_decode(model, torch.zeros((1, 4), dtype=torch.int64), 0)


def _promoted_persistent_registry() -> KernelRegistry:
    """A copy of the shipped registry with the persistent decoder promoted (the global one is
    left as shipped)."""
    reg = KernelRegistry()
    for e in REGISTRY:
        reg.register(e.name, impl=e.impl, replaces=e.replaces, status=e.status, notes=e.notes)
    reg.promote("hip_persistent_decode")
    return reg


def test_persistent_decoder_is_a_decode_cache_candidate():
    e = REGISTRY.get("hip_persistent_decode")
    assert e.replaces == "decode_cache" and e.status is KernelStatus.CANDIDATE
    assert "hip_persistent_decode" in INSTALLERS


def test_promoted_persistent_decoder_installs_its_loop_and_refuses_batches():
    from deltaforge_amd.model import PersistentDecodeLoop
    from deltaforge_amd.synth import synth_model

    model = synth_model(mid_config(num_layers=4), seed=0)
    reg = _promoted_persistent_registry()
    applied = apply_champions(model, reg)
    assert "hip_persistent_decode" in applied and "hip_decode_engine" not in applied
    assert isinstance(model.decode_loop, PersistentDecodeLoop)
    with pytest.raises(ValueError, match="batch 1"):
        greedy_decode(model, torch.zeros((2, 4), dtype=torch.int64), 2)


def test_persistent_installer_refuses_other_head_geometry():
    from deltaforge_amd.config import tiny_config
    from deltaforge_amd.synth import synth_model

    model = synth_model(tiny_config(), seed=0)
    with pytest.raises(ValueError, match="hip_persistent_decode does not support"):
        INSTALLERS["hip_persistent_decode"](model, REGISTRY.get("hip_persistent_decode"))
    assert getattr(model, "decode_loop", None) is None


def test_greedy_decode_without_loop_fails_loudly():
    class Bare:
        pass

    with pytest.raises(InstallerMissing):
        greedy_decode(Bare(), torch.zeros((1, 4), dtype=torch.int64), 2)


# -- custom ops: errors before device, no fallback, fakes ----------------------------------


def _int4(k=256, n=64, device="cpu"):
    packed = torch.zeros((k // 2, n), dtype=torch.uint8, device=device)
    scale = torch.ones((k // 128, n), dtype=BF16, device=device)
    return packed, scale


def test_tiled_gemv_int4_shape_errors_come_first():
    packed, scale = _int4()
    with pytest.raises(ValueError):
        hip_ops.tiled_gemv_int4(torch.zeros((1, 128), dtype=BF16), packed, scale, 128)  # wrong K
    with pytest.raises(ValueError):
        hip_ops.tiled_gemv_int4(torch.zeros((1, 256), dtype=BF16), packed, scale, 64)  # wrong group
    with pytest.raises(ValueError):
        hip_ops.tiled_gemv_int4(torch.zeros((1, 256), dtype=torch.float32), packed, scale, 128)
    with pytest.raises(ValueError):
        hip_ops.tiled_gemv_int4(torch.zeros((1, 256), dtype=BF16), packed, scale.float(), 128)
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        hip_ops.tiled_gemv_int4(torch.zeros((1, 256), dtype=BF16), packed, scale, 128)


@pytest.mark.parametrize(
    "call",
    [
        lambda: hip_ops.silu_mul(torch.zeros(8, dtype=BF16), torch.zeros(8, dtype=BF16)),
        lambda: hip_ops.rms_norm(torch.zeros((2, 8), dtype=BF16), torch.zeros(8, dtype=BF16), 1e-6),
        lambda: hip_ops.add_rms_norm(torch.zeros((2, 8), dtype=BF16), torch.zeros((2, 8), dtype=BF16),
                                     torch.zeros(8, dtype=BF16), 1e-6),
        lambda: hip_ops.apply_partial_rope(torch.zeros((1, 2, 1, 8), dtype=BF16), torch.zeros((1, 1, 4), dtype=BF16),
                                           torch.zeros((1, 1, 4), dtype=BF16)),
        lambda: hip_ops.fused_causal_conv_step(torch.zeros((1, 8, 1), dtype=BF16), torch.zeros((1, 8, 3), dtype=BF16),
                                               torch.zeros((8, 1, 4), dtype=BF16)),
    ],
)
def test_cpu_tensors_raise_without_fallback(call):
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        call()


@pytest.mark.parametrize(
    "call",
    [
        lambda: hip_ops.silu_mul(torch.zeros(8, dtype=BF16), torch.zeros(9, dtype=BF16)),
        lambda: hip_ops.rms_norm(torch.zeros((2, 8), dtype=BF16), torch.zeros(7, dtype=BF16), 1e-6),
        lambda: hip_ops.apply_partial_rope(torch.zeros((1, 2, 1, 8), dtype=BF16), torch.zeros((1, 1, 3), dtype=BF16),
                                           torch.zeros((1, 1, 3), dtype=BF16)),
        lambda: hip_ops.fused_causal_conv_step(torch.zeros((1, 8, 2), dtype=BF16), torch.zeros((1, 8, 3), dtype=BF16),
                                               torch.zeros((8, 1, 4), dtype=BF16)),
    ],
)
def test_bad_shapes_raise_value_error_before_the_device_check(call):
    with pytest.raises(ValueError):
        call()


def test_delta_and_attention_ops_validate_before_device():
    c = mid_config(num_layers=4)
    hv, hk, dk = c.linear_num_value_heads, c.linear_num_key_heads, 128
    ch = 2 * hk * dk + hv * dk
    state = torch.zeros((1, hv, dk, dk), dtype=torch.float32)
    args = dict(mixed_qkv=torch.zeros((1, ch), dtype=BF16), a=torch.zeros((1, hv), dtype=BF16),
                b=torch.zeros((1, hv), dtype=BF16), A_log=torch.zeros(hv, dtype=BF16), dt_bias=torch.zeros(hv, dtype=BF16),
                conv_weight=torch.zeros((ch, 1, 4), dtype=BF16), conv_cache=torch.zeros((1, ch, 3), dtype=BF16),
                state=state, num_k_heads=hk)
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        hip_ops.gated_delta_decode(**args)
    with pytest.raises(ValueError):
        hip_ops.gated_delta_decode(**{**args, "state": state.to(BF16)})
    hq, hkv, d = c.num_attention_heads, c.num_key_value_heads, c.head_dim
    att = dict(q_gate=torch.zeros((1, hq * 2 * d), dtype=BF16), k=torch.zeros((1, hkv * d), dtype=BF16),
               v=torch.zeros((1, hkv * d), dtype=BF16), q_norm_w=torch.zeros(d, dtype=BF16),
               k_norm_w=torch.zeros(d, dtype=BF16), inv_freq=torch.zeros(32, dtype=torch.float32),
               k_cache=torch.zeros((1, hkv, 16, d), dtype=BF16), v_cache=torch.zeros((1, hkv, 16, d), dtype=BF16),
               position=torch.zeros(1, dtype=torch.int32), num_q_heads=hq, sigmoid_gate=True, eps=1e-6)
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        hip_ops.gated_attention_decode(**att)
    with pytest.raises(ValueError):
        hip_ops.gated_attention_decode(**{**att, "num_q_heads": hq + 1})


def test_fake_kernels_give_the_output_shapes():
    m = "meta"
    packed, scale = _int4(512, 128, m)
    assert hip_ops.tiled_gemv_int4(torch.empty((3, 5, 512), dtype=BF16, device=m), packed, scale, 128).shape == (3, 5, 128)
    assert hip_ops.silu_mul(torch.empty(8, dtype=BF16, device=m), torch.empty(8, dtype=BF16, device=m)).shape == (8,)
    r, y = hip_ops.add_rms_norm(*(torch.empty((2, 8), dtype=BF16, device=m) for _ in range(2)),
                                torch.empty(8, dtype=BF16, device=m), 1e-6)
    assert r.shape == y.shape == (2, 8)
    st = torch.empty((2, 4, 128, 128), dtype=torch.float32, device=m)
    out = hip_ops.gated_delta_decode(torch.empty((2, 2048), dtype=BF16, device=m), torch.empty((2, 4), dtype=BF16, device=m),
                                     torch.empty((2, 4), dtype=BF16, device=m), torch.empty(4, dtype=BF16, device=m),
                                     torch.empty(4, dtype=BF16, device=m), torch.empty((2048, 1, 4), dtype=BF16, device=m),
                                     torch.empty((2, 2048, 3), dtype=BF16, device=m), st, 4)
    assert out.shape == (2, 4, 128)


# -- argument checks that guard the kernels' pointers ----------------------------------------


def _delta_args(hv=32, hk=16, dk=128):
    from deltaforge_amd import ops

    ch = 2 * hk * dk + hv * dk
    return ops, dict(qkv=torch.zeros((1, ch), dtype=BF16), a=torch.zeros((1, hv), dtype=BF16),
                     b=torch.zeros((1, hv), dtype=BF16), A_log=torch.zeros(hv, dtype=BF16),
                     dt_bias=torch.zeros(hv, dtype=BF16), conv_w=torch.zeros((ch, 1, 4), dtype=BF16),
                     state=torch.zeros((1, hv, dk, dk), dtype=torch.float32), num_k_heads=hk,
                     conv_ring=torch.zeros((1, ch, 4), dtype=BF16), position=torch.zeros(1, dtype=torch.int32))


def test_gated_delta_step_rejects_misread_dtypes_before_the_device():
    ops, args = _delta_args()
    for name in ("A_log", "dt_bias", "a", "b", "qkv"):
        bad = {**args, name: args[name].float()}
        with pytest.raises(ValueError, match=name):
            ops.gated_delta_step(**bad)
    with pytest.raises(ValueError):
        ops.gated_delta_step(**{**args, "A_log": torch.zeros(31, dtype=BF16)})
    with pytest.raises(ValueError):
        ops.gated_delta_step(**{**args, "position": torch.zeros(1, dtype=torch.int64)})
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        ops.gated_delta_step(**args)


def test_attention_decode_checks_rotary_width_and_caches():
    from deltaforge_amd import ops

    d, hkv = 256, 4
    base = dict(q=torch.zeros((1, 16 * 2 * d), dtype=BF16), k=torch.zeros((1, hkv * d), dtype=BF16),
                v=torch.zeros((1, hkv * d), dtype=BF16), q_norm_w=torch.zeros(d, dtype=BF16),
                k_norm_w=torch.zeros(d, dtype=BF16), inv_freq=torch.zeros(32, dtype=torch.float32),
                k_cache=torch.zeros((1, hkv, 16, d), dtype=BF16), v_cache=torch.zeros((1, hkv, 16, d), dtype=BF16),
                position=torch.zeros(1, dtype=torch.int32), num_q_heads=16)
    # rotary 48 and 96: rotary/8 not a power of two, the xor partner shuffle would pair wrong dims
    for half in (24, 48, 3):
        with pytest.raises(ValueError, match="rotary_dim"):
            ops.attention_decode(**{**base, "inv_freq": torch.zeros(half, dtype=torch.float32)})
    with pytest.raises(ValueError, match="contiguous"):
        kc = torch.zeros((1, hkv, d, 16), dtype=BF16).transpose(2, 3)
        ops.attention_decode(**{**base, "k_cache": kc})
    with pytest.raises(ValueError):
        ops.attention_decode(**{**base, "q_norm_w": torch.zeros(d, dtype=torch.float32)})
    # every tensor the kernel dereferences must be on the GPU: a CPU position alone is refused
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        ops.attention_decode(**base)


def test_reference_signature_ops_validate_in_reference_order():
    ops_mod = hip_ops
    state = torch.zeros((1, 4, 128, 128))
    q = torch.zeros((1, 4, 128))
    with pytest.raises(ValueError, match="query"):
        ops_mod.delta_rule_step(state, torch.zeros((1, 4, 64)), q, q, torch.zeros((1, 4)), torch.zeros((1, 4)))
    with pytest.raises(ValueError, match="fp32"):
        ops_mod.delta_rule_step(state.to(BF16), q, q, q, torch.zeros((1, 4)), torch.zeros((1, 4)))
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        ops_mod.delta_rule_step(state, q, q, q, torch.zeros((1, 4)), torch.zeros((1, 4)))
    qa = torch.zeros((1, 16, 256), dtype=BF16)
    kv = torch.zeros((1, 4, 8, 256), dtype=BF16)
    with pytest.raises(ValueError, match="power of two"):
        ops_mod.split_kv_decode_attention(qa, kv, kv, 0.0625, 3)
    with pytest.raises(ValueError, match="empty"):
        ops_mod.split_kv_decode_attention(qa, kv[:, :, :0], kv[:, :, :0], 0.0625, 8)
    with pytest.raises(ValueError, match="divide"):
        ops_mod.split_kv_decode_attention(torch.zeros((1, 6, 256), dtype=BF16), kv, kv, 0.0625, 8)
    with pytest.raises(RuntimeError, match="no PyTorch fallback"):
        ops_mod.split_kv_decode_attention(qa, kv, kv, 0.0625, 8)
    meta = "meta"
    o, s = ops_mod.delta_rule_step(*(torch.empty(t.shape, device=meta) for t in (state, q, q, q)),
                                   torch.empty((1, 4), device=meta), torch.empty((1, 4), device=meta))
    assert o.shape == (1, 4, 128) and s.shape == state.shape
    assert ops_mod.split_kv_decode_attention(qa.to(meta), kv.to(meta), kv.to(meta), 0.0625, 8).shape == qa.shape


def test_standalone_ops_are_registered_candidates_with_checks():
    from deltaforge_amd.kernels import CHECK_BUILDERS

    for name, op in (("hip_delta_rule_step", "gated_delta_rule"), ("hip_split_kv_decode_attention", "gqa_attention")):
        e = REGISTRY.get(name)
        assert e.replaces == op and e.status is KernelStatus.CANDIDATE
        assert name in INSTALLERS and name in CHECK_BUILDERS


def test_check_builders_definitions_agree_with_the_oracle():
    """The package's check builders carry their own fp32 definitions of the two standalone
    ops (the package never imports the oracle); those definitions agree with the oracle's
    restatement of the reference on the builders' shapes."""
    from oracle.model import delta_rule_step as oracle_step
    from oracle.ops import decode_attention

    gen = torch.Generator().manual_seed(5)
    state = torch.randn((2, 4, 128, 128), generator=gen) * 0.1
    q = torch.nn.functional.normalize(torch.randn((2, 4, 128), generator=gen), dim=-1) / 128 ** 0.5
    k = torch.nn.functional.normalize(torch.randn((2, 4, 128), generator=gen), dim=-1)
    v = torch.randn((2, 4, 128), generator=gen)
    g = -torch.nn.functional.softplus(torch.randn((2, 4), generator=gen))
    beta = torch.sigmoid(torch.randn((2, 4), generator=gen))
    got_out, got_state = hip_ops._delta_rule_definition(state, q, k, v, g, beta)
    want_out, want_state = oracle_step(state, q, k, v, g, beta)
    torch.testing.assert_close(got_state, want_state, atol=1e-5, rtol=0)
    torch.testing.assert_close(got_out, want_out, atol=1e-5, rtol=0)
    # a wrong sign on the recall term moves the state far past the bar
    bad = hip_ops._delta_rule_definition(state, q, -k, v, g, beta)[1]
    assert (bad - want_state).abs().max() > 1e-2

    qa = torch.randn((2, 16, 256), generator=gen).to(BF16)
    ka = torch.randn((2, 4, 33, 256), generator=gen).to(BF16)
    va = torch.randn((2, 4, 33, 256), generator=gen).to(BF16)
    torch.testing.assert_close(hip_ops._attention_definition(qa, ka, va, 0.0625),
                               decode_attention(qa, ka, va, 0.0625), atol=2e-2, rtol=1e-2)


def test_product_package_never_imports_the_oracle():
    pkg = ROOT / "deltaforge_amd"
    offenders = [str(p.relative_to(ROOT)) for p in pkg.rglob("*.py")
                 if re.search(r"^\s*(from|import)\s+oracle\b", p.read_text(), flags=re.M)]
    assert not offenders, offenders


def test_registry_index_detects_an_entry_changed_behind_its_back():
    import dataclasses

    reg = KernelRegistry()
    reg.register("a", impl=lambda: None, replaces="rms_norm", status=KernelStatus.CHAMPION)
    reg.register("b", impl=lambda: None, replaces="rms_norm")
    reg.check_invariants()
    reg._entries["b"] = dataclasses.replace(reg._entries["b"], status=KernelStatus.CHAMPION)
    with pytest.raises(RegistryError):
        reg.check_invariants()
    reg.unregister("a")
    reg._entries["b"] = dataclasses.replace(reg._entries["b"], status=KernelStatus.CANDIDATE)
    reg.check_invariants()
    assert reg.champion("rms_norm") is None
    reg.promote("b")
    assert reg.champion("rms_norm").name == "b"


def test_persistent_rope_table_matches_the_oracle_bit_for_bit():
    """The persistent kernel reads cos/sin from a host-built table: pair j of position p must be
    the oracle's bf16 cos/sin of p * bf16(inv_freq_j) (reference.py:165-200)."""
    from deltaforge_amd.config import qwen3_5_4b_config
    from deltaforge_amd.persistent import rope_table
    from oracle.model import rope_cos_sin

    cfg = qwen3_5_4b_config()
    positions = torch.tensor([0, 1, 2, 7, 4095, 4096, 32767, 131071])
    table = rope_table(cfg, 131072)[positions]
    cos, sin = rope_cos_sin(positions.view(1, -1), cfg, torch.bfloat16, inv_freq_dtype=torch.bfloat16)
    half = cfg.rotary_dim // 2
    want_cos = cos[0, :, :half].contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    want_sin = sin[0, :, :half].contiguous().view(torch.int16).to(torch.int32) & 0xFFFF
    assert torch.equal(table & 0xFFFF, want_cos)
    assert torch.equal((table >> 16) & 0xFFFF, want_sin)


# -- prefill host checks --------------------------------------------------------------------


def _attention_prefill_args(tokens=3, hkv=1, max_len=8):
    q = torch.zeros((tokens, 4 * hkv, 256), dtype=BF16)
    kc = torch.zeros((hkv, max_len, 256), dtype=BF16)
    gate = torch.zeros((tokens, 2 * 256 * 4 * hkv), dtype=BF16)
    return q, kc, kc.clone(), gate


def test_attention_prefill_checks_gate_and_out_extents_before_the_device():
    from deltaforge_amd.prefill import attention_prefill

    q, kc, vc, gate = _attention_prefill_args()
    # gate one column short of head 3's last element at stride 512
    with pytest.raises(ValueError, match="gate must be"):
        attention_prefill(q, kc, vc, gate[:, :3 * 512 + 255], gate_head_stride=512)
    with pytest.raises(ValueError, match="gate must be"):
        attention_prefill(q, kc, vc, gate[:2], gate_head_stride=512)
    with pytest.raises(ValueError, match="gate must be"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=-1)
    with pytest.raises(ValueError, match="contiguous rows"):
        attention_prefill(q, kc, vc, gate[:, ::2], gate_head_stride=256)
    with pytest.raises(ValueError, match="out must be"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, out=torch.empty((3, 1023), dtype=BF16))
    with pytest.raises(ValueError, match="out must be"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, out=torch.empty((2, 1024), dtype=BF16))
    with pytest.raises(ValueError, match="out must be"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, out=torch.empty((3, 1024), dtype=torch.float32))
    with pytest.raises(ValueError, match="contiguous rows"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, out=torch.empty((1024, 3), dtype=BF16).t())
    with pytest.raises(ValueError, match="do not fit"):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, pos0=6)
    # every extent in range: the next stop is the device check
    with pytest.raises(RuntimeError):
        attention_prefill(q, kc, vc, gate, gate_head_stride=512, out=torch.empty((3, 1024), dtype=BF16))


def test_prefiller_fill_rejects_token_ids_outside_the_vocabulary():
    from types import SimpleNamespace

    from deltaforge_amd.prefill import Prefiller

    pre = Prefiller.__new__(Prefiller)  # the checks run before any weight or device use
    pre.config = mid_config()
    pre.device = torch.device("cpu")
    decoder = SimpleNamespace(max_new_tokens=4, max_seq_len=64,
                              reset=lambda: pytest.fail("reset ran before the id check"))
    vocab = pre.config.vocab_size
    for bad in (torch.tensor([[1, vocab, 2]]), torch.tensor([[-1, 0]])):
        with pytest.raises(ValueError, match="token ids"):
            pre.fill(decoder, bad)
    with pytest.raises(ValueError, match="at least one token"):
        pre.fill(decoder, torch.zeros((1, 0), dtype=torch.int64))


# -- slots: the decode step calls what the registry's champions say ---------------------------


def _registry_with(*promoted: str) -> KernelRegistry:
    reg = KernelRegistry()
    for e in REGISTRY:
        reg.register(e.name, impl=e.impl, replaces=e.replaces, status=e.status, notes=e.notes)
    for name in promoted:
        reg.promote(name)
    return reg


def test_shipped_champions_plan_the_fused_step():
    from deltaforge_amd.model import STEP_SLOTS, installed_slots, step_plan
    from deltaforge_amd.synth import synth_model

    model = synth_model(mid_config(num_layers=4), seed=0)
    apply_champions(model)
    slots = installed_slots(model)
    assert {op: e.name for op, e in slots.items() if op in STEP_SLOTS} == {op: n[0] for op, n in STEP_SLOTS.items()}
    assert step_plan(model) == {}


@pytest.mark.parametrize("standalone,composed", [
    ("hip_delta_rule_step", {"gated_delta_rule": "hip_delta_rule_step", "causal_conv": "hip_causal_conv_step"}),
    ("hip_split_kv_decode_attention", {"gqa_attention": "hip_split_kv_decode_attention", "rms_norm": "hip_rms_norm",
                                       "qkv_projection_rope": "hip_partial_rope"}),
])
def test_promoting_a_standalone_op_composes_its_slot_from_installed_entries(standalone, composed):
    from deltaforge_amd.model import PersistentDecodeLoop, step_plan
    from deltaforge_amd.synth import synth_model

    model = synth_model(mid_config(num_layers=4), seed=0)
    applied = apply_champions(model, _registry_with(standalone))
    assert standalone in applied
    plan = step_plan(model)
    assert {op: model.kernel_slots[op].name for op in plan} == composed
    # the impls are the registry entries' own callables
    for op, impl in plan.items():
        assert impl is REGISTRY.get(composed[op]).impl
    # the persistent kernel fuses every slot itself, so it refuses such a registry
    with pytest.raises(InstallerMissing, match="standalone"):
        PersistentDecodeLoop()(model, torch.zeros((1, 4), dtype=torch.int64), 2)


def test_a_slot_kernel_without_a_call_site_is_refused():
    from deltaforge_amd.model import step_plan
    from deltaforge_amd.synth import synth_model

    reg = _registry_with()
    reg.register("third_party_delta", impl=lambda *a: None, replaces="gated_delta_rule")
    reg.promote("third_party_delta")
    model = synth_model(mid_config(num_layers=4), seed=0)
    apply_champions(model, reg, installers={**INSTALLERS, "third_party_delta": INSTALLERS["hip_delta_rule_step"]})
    with pytest.raises(InstallerMissing, match="no call site"):
        step_plan(model)
    with pytest.raises(InstallerMissing):
        greedy_decode(model, torch.zeros((1, 4), dtype=torch.int64), 2)


def test_prefill_geometry_rule():
    from deltaforge_amd.config import qwen3_5_4b_config, tiny_config
    from deltaforge_amd.prefill import unsupported_geometry

    assert unsupported_geometry(qwen3_5_4b_config()) is None
    assert unsupported_geometry(mid_config(num_layers=4)) is None
    assert unsupported_geometry(tiny_config()) is not None
