"""Persistent bs=1 decode: the whole decode step, many tokens per launch.

``PersistentDecoder`` holds the model in the layout ``df_decode_persistent`` expects (see
``include/deltaforge_hip.h``) and the static decode state, and exposes the same driving
surface as ``DecodeEngine`` (``reset``, ``prefill``, ``decode``, ``snapshot``/``restore``,
``tokens``, ``token_log``, ``logits``). One cooperative launch runs any number of steps;
the 256 workgroups act as 8 tensor-parallel ranks, one per XCD.

The input projections are stored with their columns in XCD-major order so that each XCD's
slice is one contiguous run of 16-column tiles (``linear_proj_columns``,
``attention_proj_columns``); everything else keeps the engine's layout.
"""

from __future__ import annotations

import ctypes as C

import torch

from . import _native as N
from . import ops
from .config import FULL_ATTENTION, SIGMOID_GATE, ModelConfig
from .synth import SynthModel, inv_freq

__all__ = ["PersistentDecoder", "attention_proj_columns", "check_geometry", "linear_proj_columns", "rope_table"]

BF16 = torch.bfloat16
XCD = 8
LIN_COLS = 1552  # per XCD: q 256, k 256, v 512, z 512, a 4, b 4, 8 zero columns
ATTN_COLS = 1536  # per XCD: 2 x (query 256 | gate 256), k 256, v 256
#: Trace buffer layout of the traced build: the control wave's row, then 8 compute-wave rows.
TRACE_CONTROL, TRACE_WAVE = 2048, 240
TRACE_ROWS = 4096

ERRORS = {1: "a cross-workgroup hand-off timed out", 2: "a workgroup ran on an unexpected XCD",
          3: "position, prompt or token log out of range", 4: "token id out of range",
          5: "control/compute barrier schedules disagree"}


def linear_proj_columns(c: ModelConfig) -> torch.Tensor:
    """Indices into the canonical ``[q | k | v | z | a | b]`` in_proj columns, XCD-major; -1 = zero."""
    kd, vd, hv = c.linear_key_dim, c.linear_value_dim, c.linear_num_value_heads
    cols = []
    for x in range(XCD):
        q = torch.arange(2 * x * 128, (2 * x + 2) * 128)
        k = kd + q
        v = torch.arange(2 * kd + 4 * x * 128, 2 * kd + (4 * x + 4) * 128)
        z = torch.arange(2 * kd + vd + 4 * x * 128, 2 * kd + vd + (4 * x + 4) * 128)
        a = torch.arange(2 * kd + 2 * vd + 4 * x, 2 * kd + 2 * vd + 4 * x + 4)
        b = a + hv
        cols += [q, k, v, z, a, b, torch.full((8,), -1)]
    out = torch.cat(cols)
    assert out.numel() == XCD * LIN_COLS
    return out


def attention_proj_columns(c: ModelConfig) -> torch.Tensor:
    """Indices into the canonical ``[q_proj | k_proj | v_proj]`` columns, XCD-major."""
    qd, d = 2 * c.num_attention_heads * c.head_dim, c.head_dim
    kvd = c.num_key_value_heads * d
    cols = []
    for x in range(XCD):
        qg = torch.arange(2 * x * 2 * d, (2 * x + 2) * 2 * d)
        k = torch.arange(qd + (x // 2) * d, qd + (x // 2 + 1) * d)
        cols += [qg, k, k + kvd]
    out = torch.cat(cols)
    assert out.numel() == XCD * ATTN_COLS
    return out


def _select_cols(packed: torch.Tensor, scale: torch.Tensor, cols: torch.Tensor):
    """Columns ``cols`` of a canonical int4 matrix; -1 gives an all-zero column (nibbles 8, scale 0)."""
    idx = cols.clamp(min=0)
    p = packed[:, idx].clone()
    s = scale[:, idx].clone()
    pad = cols < 0
    p[:, pad] = 0x88
    s[:, pad] = 0
    return p.contiguous(), s.contiguous()


def rope_table(c: ModelConfig, max_len: int) -> torch.Tensor:
    """The persistent kernel's RoPE table: int32 ``[max_len, rotary/2]``, pair j of position p
    as ``bf16(cos(p * f_j)) | bf16(sin(p * f_j)) << 16``, where ``f_j`` is the bf16-rounded
    inverse frequency and the angle is an fp32 product: the reference's cos/sin
    (reference.py:165-200 with the module buffer cast to bf16), computed once on the host
    instead of by the kernel for every attention layer of every token."""
    f = inv_freq(c)  # fp32 holding the bf16-rounded values
    ang = torch.arange(max_len, dtype=torch.float32).unsqueeze(1) * f.unsqueeze(0)
    cs = ang.cos().to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    sn = ang.sin().to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
    return (cs | (sn << 16)).contiguous()


def check_geometry(c: ModelConfig) -> None:
    ok = (c.linear_num_key_heads == 16 and c.linear_num_value_heads == 32 and c.linear_key_head_dim == 128
          and c.linear_value_head_dim == 128 and c.num_attention_heads == 16 and c.num_key_value_heads == 4
          and c.head_dim == 256 and c.rotary_dim == 64 and c.linear_conv_kernel_dim == 4)
    if not ok:
        raise ValueError("the persistent decoder is written for Qwen3.5-4B's head geometry")
    if c.hidden_size % 512 or c.hidden_size > 2560 or c.intermediate_size % 1024 or c.vocab_size % 128:
        raise ValueError(f"needs hidden % 512 == 0 (<= 2560), inter % 1024 == 0, vocab % 128 == 0; got "
                         f"{c.hidden_size}, {c.intermediate_size}, {c.vocab_size}")


class PersistentDecoder:
    """Greedy bs=1 decode of a ``SynthModel`` (canonical int4 weights) in persistent launches."""

    def __init__(self, model: SynthModel, *, max_seq_len: int, device: str | torch.device = "cuda",
                 max_new_tokens: int = 256, lib=None) -> None:
        c = model.config
        check_geometry(c)
        if c.output_gate_type not in (SIGMOID_GATE, "swish"):
            raise ValueError(f"unknown gate {c.output_gate_type}")
        self.config = c
        self.batch = 1
        self.max_seq_len = max_seq_len
        self.max_new_tokens = max_new_tokens
        self.device = dev = torch.device(device)
        ops.require_gpu(torch.empty(0, device=dev), "decode_persistent")
        p = {k: v.to(dev) for k, v in model.params.items()}
        lin = model.linears

        def repack(packed, scale) -> ops.Int4Weight:
            return ops.int4_repack(packed.to(dev).contiguous(), scale.to(dev).contiguous())

        lin_cols, attn_cols = linear_proj_columns(c), attention_proj_columns(c)
        self._keep: list = []  # every tensor a layer struct points at
        structs = []
        self.layer_state: list[dict] = []
        for i, kind in enumerate(c.layer_types):
            pre = f"layers.{i}."
            gu = ops.interleave_gate_up(lin[pre + "mlp.gate_proj.weight"].packed, lin[pre + "mlp.gate_proj.weight"].scale,
                                        lin[pre + "mlp.up_proj.weight"].packed, lin[pre + "mlp.up_proj.weight"].scale)
            gu_w = repack(*gu)
            down = repack(lin[pre + "mlp.down_proj.weight"].packed, lin[pre + "mlp.down_proj.weight"].scale)
            st = N.PersistLayer()
            st.in_norm = p[pre + "input_layernorm.weight"].data_ptr()
            st.post_norm = p[pre + "post_attention_layernorm.weight"].data_ptr()
            state: dict = {}
            if kind == FULL_ATTENTION:
                a = pre + "self_attn."
                parts = [lin[a + "q_proj.weight"], lin[a + "k_proj.weight"], lin[a + "v_proj.weight"]]
                cat_p = torch.cat([w.packed for w in parts], 1)
                cat_s = torch.cat([w.scale for w in parts], 1)
                proj = repack(*_select_cols(cat_p, cat_s, attn_cols))
                out = repack(lin[a + "o_proj.weight"].packed, lin[a + "o_proj.weight"].scale)
                state["k_cache"] = torch.zeros((c.num_key_value_heads, max_seq_len, c.head_dim), dtype=BF16, device=dev)
                state["v_cache"] = torch.zeros_like(state["k_cache"])
                st.kind = 1
                st.q_norm = p[a + "q_norm.weight"].data_ptr()
                st.k_norm = p[a + "k_norm.weight"].data_ptr()
                st.k_cache = state["k_cache"].data_ptr()
                st.v_cache = state["v_cache"].data_ptr()
            else:
                a = pre + "linear_attn."
                parts = [lin[a + "in_proj_qkv.weight"], lin[a + "in_proj_z.weight"], lin[a + "in_proj_a.weight"],
                         lin[a + "in_proj_b.weight"]]
                cat_p = torch.cat([w.packed for w in parts], 1)
                cat_s = torch.cat([w.scale for w in parts], 1)
                proj = repack(*_select_cols(cat_p, cat_s, lin_cols))
                out = repack(lin[a + "out_proj.weight"].packed, lin[a + "out_proj.weight"].scale)
                conv_w = p[a + "conv1d.weight"].reshape(c.linear_conv_dim, -1).contiguous()
                state["conv_ring"] = torch.zeros((c.linear_conv_dim, 4), dtype=BF16, device=dev)
                state["state"] = torch.zeros((c.linear_num_value_heads, c.linear_key_head_dim, c.linear_value_head_dim),
                                             dtype=torch.float32, device=dev)
                st.kind = 0
                st.conv_w = conv_w.data_ptr()
                st.A_log = p[a + "A_log"].data_ptr()
                st.dt_bias = p[a + "dt_bias"].data_ptr()
                st.gnorm_w = p[a + "norm.weight"].data_ptr()
                st.conv_ring = state["conv_ring"].data_ptr()
                st.state = state["state"].data_ptr()
                self._keep.append(conv_w)
            st.proj_w, st.proj_s = proj.w.data_ptr(), proj.s.data_ptr()
            st.out_w, st.out_s = out.w.data_ptr(), out.s.data_ptr()
            st.gu_w, st.gu_s = gu_w.w.data_ptr(), gu_w.s.data_ptr()
            st.down_w, st.down_s = down.w.data_ptr(), down.s.data_ptr()
            self._keep += [proj, out, gu_w, down]
            structs.append(st)
            self.layer_state.append(state)
        self.params = p
        self.head = repack(lin["lm_head"].packed, lin["lm_head"].scale)
        self.final_norm = p["norm.weight"]
        self.rope = rope_table(c, max_seq_len).to(dev)
        # a checkpoint's own bf16 embedding table (``checkpoint.load_checkpoint``); without one the
        # token rows come from the tied int4 head, which is the synthetic model's table
        table = p.get("embed_tokens.weight")
        if table is not None and tuple(table.shape) != (c.vocab_size, c.hidden_size):
            raise ValueError(f"embed_tokens.weight must be [{c.vocab_size}, {c.hidden_size}], got {tuple(table.shape)}")
        self.embed_table = table.to(torch.bfloat16).contiguous() if table is not None else None
        raw = b"".join(bytes(s) for s in structs)
        self.layers_dev = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(dev)

        self.position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step_index = torch.zeros(1, dtype=torch.int32, device=dev)
        self.tokens = torch.zeros(1, dtype=torch.int64, device=dev)
        self.token_log = torch.zeros((1, max_new_tokens), dtype=torch.int64, device=dev)
        self.logits = torch.zeros((1, c.vocab_size), dtype=BF16, device=dev)
        self.prompt = torch.zeros(max_seq_len, dtype=torch.int64, device=dev)
        self.prompt_len = 0
        self._trace: torch.Tensor | None = None
        self._trace_step = 0
        # the library whose decode kernel this decoder launches (another build of the same
        # sources for an A/B comparison; the in-tree build by default)
        self.lib = lib if lib is not None else N.lib()
        nbytes = int(self.lib.df_decode_persistent_workspace_bytes(c.hidden_size))
        self.workspace = torch.zeros(nbytes, dtype=torch.uint8, device=dev)

    # -- launches -----------------------------------------------------------------------

    def _model(self) -> N.PersistModel:
        c = self.config
        m = N.PersistModel()
        m.hidden, m.inter, m.vocab = c.hidden_size, c.intermediate_size, c.vocab_size
        m.num_layers, m.max_len = c.num_hidden_layers, self.max_seq_len
        m.gate_kind = 0 if c.output_gate_type == SIGMOID_GATE else 1
        m.eps = c.rms_norm_eps
        m.layers = self.layers_dev.data_ptr()
        m.head_w, m.head_s = self.head.w.data_ptr(), self.head.s.data_ptr()
        m.final_norm = self.final_norm.data_ptr()
        m.rope = self.rope.data_ptr()
        m.position, m.tokens = self.position.data_ptr(), self.tokens.data_ptr()
        m.prompt, m.prompt_len = self.prompt.data_ptr(), self.prompt_len
        m.token_log, m.log_capacity = self.token_log.data_ptr(), self.max_new_tokens
        m.step = self.step_index.data_ptr()
        m.logits = self.logits.data_ptr()
        m.embed_table = self.embed_table.data_ptr() if self.embed_table is not None else None
        if self._trace is not None:
            m.trace, m.trace_step, m.trace_capacity = self._trace.data_ptr(), self._trace_step, self._trace.numel()
        return m

    def trace_decode(self, steps: int, trace_step: int) -> dict:
        """Greedy ``steps`` with the phase trace of step ``trace_step`` from workgroup (XCD 0,
        rank 0): ``{"control": [...], "waves": [[...] x 8]}``, each stamp s_memrealtime (100 MHz)
        << 8 | tag. The control wave stamps each phase's start, its hand-off landing and its
        signal (trace rows 0..2047); each compute wave stamps its GEMV consume and attention
        split points in a row of 240 after them. Only the traced build of the library stamps
        (``python -m deltaforge_amd.build --trace``, loaded with ``lib=``); the product build
        compiles the stamps out and returns empty lists. ``harness.phase_trace`` reads it."""
        self._trace = torch.zeros(TRACE_ROWS, dtype=torch.int64, device=self.device)
        self._trace_step = trace_step
        try:
            self.decode(steps)
            self.check()
        finally:
            stamps = self._trace.cpu().tolist()
            self._trace = None
        ctl = [t for t in stamps[:TRACE_CONTROL] if t]
        waves = [[t for t in stamps[TRACE_CONTROL + TRACE_WAVE * w:TRACE_CONTROL + TRACE_WAVE * (w + 1)] if t]
                 for w in range(8)]
        return {"control": ctl, "waves": waves}

    def launch(self, steps: int, *, teacher_forced: bool) -> None:
        """Enqueue ``steps`` decode steps on the current stream (no host synchronisation)."""
        m = self._model()
        stream = torch.cuda.current_stream(self.device).cuda_stream
        N.check(self.lib.df_decode_persistent(C.byref(m), steps, int(teacher_forced), self.workspace.data_ptr(),
                                             self.workspace.numel(), stream), "decode_persistent")

    def check(self) -> None:
        """Synchronise and raise if a launch aborted (its outputs are then invalid)."""
        torch.cuda.synchronize(self.device)
        ctl = self.workspace[:16].view(torch.int32).cpu()
        if int(ctl[1]):
            err = int(ctl[2])
            raise N.NativeError(f"deltaforge::decode_persistent aborted: {ERRORS.get(err, err)}")

    def reset_workspace(self) -> None:
        """Clear the hand-off state (after an aborted launch)."""
        self.workspace.zero_()

    # -- the DecodeEngine surface ----------------------------------------------------------

    def reset(self) -> None:
        """Empty caches at position 0 and a cleared hand-off workspace.

        The workspace is cleared whole, not just its abort word: an aborted launch leaves
        tagged hand-off words at epochs above the stored epoch, which a launch that kept them
        would take for fresh data. So after an abort (``check`` raises) the decoder is usable
        again from the next ``reset`` / ``prefill``."""
        for st in self.layer_state:
            for t in st.values():
                t.zero_()
        self.workspace.zero_()
        self.position.zero_()
        self.step_index.zero_()
        self.tokens.zero_()

    def prefill(self, prompt: torch.Tensor) -> None:
        """Teacher-force ``prompt`` ``[1, P]`` through the decode step; the last step's argmax is
        the first generated token (``tokens``)."""
        if prompt.dim() != 2 or prompt.shape[0] != 1:
            raise ValueError(f"prompt must be [1, P], got {tuple(prompt.shape)}")
        plen = prompt.shape[1]
        if plen + self.max_new_tokens > self.max_seq_len:
            raise ValueError("prompt + max_new_tokens exceeds the cache")
        self.reset()
        self.prompt[:plen].copy_(prompt[0].to(self.device, torch.int64))
        self.prompt_len = plen
        self.launch(plen, teacher_forced=True)
        self.step_index.zero_()

    def decode(self, steps: int) -> None:
        """Greedy steps from ``tokens``; the argmax of step k lands in ``token_log[0, k]``."""
        self.launch(steps, teacher_forced=False)

    def state_tensors(self) -> list[torch.Tensor]:
        out = [t for st in self.layer_state for t in st.values()]
        return out + [self.position, self.step_index, self.tokens]

    def snapshot(self) -> list[torch.Tensor]:
        return [t.clone() for t in self.state_tensors()]

    def restore(self, snap: list[torch.Tensor]) -> None:
        for t, s in zip(self.state_tensors(), snap):
            t.copy_(s)

    def weight_bytes(self) -> int:
        return self.head.nbytes + sum(w.nbytes for w in self._keep if isinstance(w, ops.Int4Weight))
