"""ctypes binding of ``libdeltaforge_hip.so`` (declared in ``include/deltaforge_hip.h``).

There is no fallback: if the library is missing or fails to load, every op raises. The
library is built in-tree by ``python -m deltaforge_amd.build`` (or ``__graft_entry__.build``).
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libdeltaforge_hip.so"

STATUS = {0: "ok", 1: "bad argument", 2: "kernel launch failed", 3: "workspace too small"}

PRO_NONE, PRO_RMSNORM, PRO_ADD_RMSNORM, PRO_GATED_RMSNORM = 0, 1, 2, 3
EPI_STORE, EPI_RESIDUAL, EPI_SWIGLU, EPI_LOGITS = 0, 1, 2, 3

_vp = C.c_void_p
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t


class Int4GemvArgs(C.Structure):
    _fields_ = [
        ("w", _vp), ("s", _vp), ("x", _vp), ("x2", _vp), ("norm_w", _vp), ("res", _vp),
        ("out", _vp), ("h_out", _vp), ("part", _vp),
        ("rows", _i), ("K", _i), ("N", _i), ("ldx", _i), ("ldx2", _i), ("ldo", _i),
        ("tiles_per_workgroup", _i), ("ksplit", _i), ("groups_per_split", _i),
        ("prologue", _i), ("epilogue", _i),
        ("eps", _f),
    ]


class GatedDeltaArgs(C.Structure):
    _fields_ = [
        ("qkv", _vp), ("a", _vp), ("b", _vp), ("A_log", _vp), ("dt_bias", _vp), ("conv_w", _vp),
        ("conv_in", _vp), ("conv_out", _vp), ("conv_ring", _vp), ("position", _vp),
        ("state", _vp), ("out", _vp),
        ("batch", _i), ("ld_qkv", _i), ("ld_ab", _i),
        ("num_k_heads", _i), ("num_v_heads", _i), ("head_k_dim", _i), ("head_v_dim", _i),
        ("conv_mode", _i),
    ]


class DeltaRuleArgs(C.Structure):
    _fields_ = [
        ("state_in", _vp), ("state_out", _vp), ("query", _vp), ("key", _vp), ("value", _vp), ("g", _vp),
        ("beta", _vp), ("out", _vp),
        ("batch", _i), ("heads", _i), ("key_dim", _i), ("value_dim", _i),
    ]


class DeltaInputsArgs(C.Structure):
    _fields_ = [
        ("mixed", _vp), ("a", _vp), ("b", _vp), ("A_log", _vp), ("dt_bias", _vp),
        ("query", _vp), ("key", _vp), ("value", _vp), ("g", _vp), ("beta", _vp),
        ("ld_mixed", _i), ("ld_ab", _i),
        ("batch", _i), ("num_k_heads", _i), ("num_v_heads", _i), ("head_k_dim", _i), ("head_v_dim", _i),
        ("eps", _f),
    ]


class AttnDecodeArgs(C.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("q_norm_w", _vp), ("k_norm_w", _vp), ("inv_freq", _vp),
        ("k_cache", _vp), ("v_cache", _vp), ("position", _vp), ("out", _vp),
        ("batch", _i), ("ld_q", _i), ("ld_kv", _i), ("num_q_heads", _i), ("num_kv_heads", _i), ("head_dim", _i),
        ("rotary_dim", _i), ("max_len", _i), ("splits", _i), ("gate", _i), ("eps", _f),
    ]


class PersistLayer(C.Structure):
    _fields_ = [
        ("kind", _i),
        ("in_norm", _vp), ("post_norm", _vp),
        ("proj_w", _vp), ("proj_s", _vp), ("out_w", _vp), ("out_s", _vp),
        ("gu_w", _vp), ("gu_s", _vp), ("down_w", _vp), ("down_s", _vp),
        ("conv_w", _vp), ("A_log", _vp), ("dt_bias", _vp), ("gnorm_w", _vp),
        ("conv_ring", _vp), ("state", _vp),
        ("q_norm", _vp), ("k_norm", _vp), ("k_cache", _vp), ("v_cache", _vp),
    ]


class PersistModel(C.Structure):
    _fields_ = [
        ("hidden", _i), ("inter", _i), ("vocab", _i), ("num_layers", _i), ("max_len", _i), ("gate_kind", _i),
        ("eps", _f),
        ("layers", _vp), ("head_w", _vp), ("head_s", _vp), ("final_norm", _vp), ("rope", _vp),
        ("position", _vp), ("tokens", _vp), ("prompt", _vp), ("prompt_len", _i),
        ("token_log", _vp), ("log_capacity", _i), ("step", _vp), ("logits", _vp),
        ("trace", _vp), ("trace_step", _i), ("trace_capacity", _i), ("embed_table", _vp),
    ]


class Int4GemmArgs(C.Structure):
    _fields_ = [("x", _vp), ("w", _vp), ("s", _vp), ("out", _vp),
                ("M", _i), ("K", _i), ("N", _i), ("ldx", _i), ("ldo", _i), ("epilogue", _i)]


class DeltaPrefillArgs(C.Structure):
    _fields_ = [("mixed", _vp), ("a", _vp), ("b", _vp), ("A_log", _vp), ("dt_bias", _vp), ("state", _vp),
                ("out", _vp), ("ld_mixed", _i), ("ld_ab", _i), ("ld_out", _i),
                ("tokens", _i), ("num_k_heads", _i), ("num_v_heads", _i)]


class QkPrefillArgs(C.Structure):
    _fields_ = [("proj", _vp), ("q_norm", _vp), ("k_norm", _vp), ("inv_freq", _vp), ("q_out", _vp),
                ("k_cache", _vp), ("v_cache", _vp), ("ld_proj", _i), ("k_col", _i), ("v_col", _i),
                ("tokens", _i), ("pos0", _i), ("max_len", _i), ("num_q_heads", _i), ("num_kv_heads", _i),
                ("rotary_dim", _i), ("eps", _f)]


class AttnPrefillArgs(C.Structure):
    _fields_ = [("q", _vp), ("k_cache", _vp), ("v_cache", _vp), ("gate", _vp), ("out", _vp),
                ("ld_gate", _i), ("gate_head_stride", _i), ("ld_out", _i),
                ("tokens", _i), ("pos0", _i), ("max_len", _i), ("num_q_heads", _i), ("num_kv_heads", _i),
                ("gate_kind", _i), ("scale", _f)]


# name -> (restype, argtypes); the exported surface of include/deltaforge_hip.h
SIGNATURES = {
    "df_int4_gemv_plan": (_i, [_i, _i, _i, _i, _i, C.POINTER(_i), C.POINTER(_i), C.POINTER(_i), C.POINTER(_sz)]),
    "df_int4_gemv_workspace_bytes": (_sz, [_i, _i, _i]),
    "df_int4_gemv": (_i, [C.POINTER(Int4GemvArgs), _vp, _sz, _vp]),
    "df_int4_repack": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp]),
    "df_int4_dequant": (_i, [_vp, _vp, _i, _i, _vp, _vp]),
    "df_gated_delta_step": (_i, [C.POINTER(GatedDeltaArgs), _vp]),
    "df_delta_rule_step": (_i, [C.POINTER(DeltaRuleArgs), _vp]),
    "df_delta_step_inputs": (_i, [C.POINTER(DeltaInputsArgs), _vp]),
    "df_split_kv_decode_attention": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _f, _i, _vp, _vp, _sz, _vp]),
    "df_attention_decode_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "df_attention_decode_splits": (_i, [_i, _i, _i]),
    "df_attention_decode": (_i, [C.POINTER(AttnDecodeArgs), _vp, _sz, _vp]),
    "df_attention_decode_static_capacity": (_sz, []),
    "df_attention_decode_static": (_i, [C.POINTER(AttnDecodeArgs), _vp]),
    "df_rms_norm": (_i, [_vp, _vp, _f, _i, _i, _vp, _vp]),
    "df_add_rms_norm": (_i, [_vp, _vp, _vp, _f, _i, _i, _vp, _vp, _vp]),
    "df_silu_mul": (_i, [_vp, _vp, _sz, _vp, _vp]),
    "df_partial_rope": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _vp]),
    "df_causal_conv_step": (_i, [_vp, _vp, _vp, _i, _i, _vp, _vp]),
    "df_embed_int4": (_i, [_vp, _vp, _i, _vp, _i, _vp, _vp, _i, _i, _vp, _vp]),
    "df_embed_bf16": (_i, [_vp, _vp, _i, _vp, _i, _vp, _i, _i, _vp, _vp]),
    "df_int4_gemm": (_i, [C.POINTER(Int4GemmArgs), _vp]),
    "df_causal_conv_prefill": (_i, [_vp, _i, _i, _i, _vp, _vp, _i, _vp, _i, _vp]),
    "df_delta_rule_prefill_workspace_bytes": (_sz, [_i, _i]),
    "df_delta_rule_prefill": (_i, [C.POINTER(DeltaPrefillArgs), _vp, _sz, _vp]),
    "df_gated_rms_norm_rows": (_i, [_vp, _i, _vp, _i, _vp, _f, _i, _i, _vp, _i, _vp]),
    "df_qk_norm_rope_prefill": (_i, [C.POINTER(QkPrefillArgs), _vp]),
    "df_attention_prefill": (_i, [C.POINTER(AttnPrefillArgs), _vp]),
    "df_argmax_workspace_bytes": (_sz, [_i, _i]),
    "df_argmax": (_i, [_vp, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _vp, _sz, _vp]),
    "df_decode_persistent_workspace_bytes": (_sz, [_i]),
    "df_decode_persistent": (_i, [C.POINTER(PersistModel), _i, _i, _vp, _sz, _vp]),
}

_LIB: C.CDLL | None = None


class NativeError(RuntimeError):
    """A library entry point returned a non-zero status."""


def load(path: str | Path, names=None) -> C.CDLL:
    """A library file with the declared signatures bound (all of them, or ``names``): the
    in-tree build, or another build of the same sources for an A/B comparison."""
    path = Path(path)
    if not path.exists():
        raise RuntimeError(
            f"{path} is missing; build it with `python -m deltaforge_amd.build`. "
            "deltaforge_amd has no fallback path."
        )
    handle = C.CDLL(str(path))
    for name, (restype, argtypes) in SIGNATURES.items():
        if names is not None and name not in names:
            continue
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return handle


def lib() -> C.CDLL:
    """Load the in-tree HIP library once. Raises if it is missing: there is no CPU fallback."""
    global _LIB
    if _LIB is None:
        _LIB = load(LIB_PATH)
    return _LIB


def check(status: int, op: str) -> None:
    if status != 0:
        raise NativeError(f"deltaforge::{op}: {STATUS.get(status, status)} (status {status})")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()
