"""The MI355X decode engine: int4 weights in HBM, static decode state, graph-captured steps.

One greedy decode step of the hybrid model (reference ``ReferenceModel.forward`` at
seq_len 1, reference.py:779-817, driven by ``greedy_decode``, model.py:108-148) is this
fixed launch sequence on one HIP stream, every buffer preallocated and every position read
from a device scalar, so the whole step is captured once in a HIP graph and replayed:

    embed (tied int4 head row)
    per Gated DeltaNet layer:  [RMSNorm + in_proj qkv|z|a|b]  [conv + delta rule]
                               [GatedRMSNorm + out_proj + residual]
    per attention layer:       [RMSNorm + q|k|v proj]  [q/k norm + RoPE + KV write + split-KV
                               attention + gate]  [o_proj + residual]
    per layer:                 [RMSNorm + gate|up + SwiGLU]  [down + residual]
    [final RMSNorm + tied head]  [argmax -> next token, position += 1]

Layouts in HBM: linears in the int4 device tiling (``ops.int4_repack``), projections that
read the same input concatenated along N (qkv|z|a|b, q|k|v, gate/up tile-interleaved); KV
cache ``[B, Hkv, max_len, 256]`` bf16 (the reference's layout); conv history as a 4-slot
ring ``[B, C, 4]`` indexed by position; recurrent state ``[B, Hv, 128, 128]`` fp32.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _native as N
from . import ops
from .config import FULL_ATTENTION, SIGMOID_GATE, ModelConfig
from .synth import SynthModel, inv_freq

BF16 = torch.bfloat16

__all__ = ["DecodeEngine", "STANDALONE_SLOTS"]

#: Split count the standalone attention op is called with (the reference's DEFAULT_SPLITS at
#: the call site its installer swaps in, kernels/flash_decode_splitkv.py:46, 322-324).
STANDALONE_SPLITS = 8

#: Slots whose champion may be a standalone op instead of the fused kernel, and the other
#: slots the standalone composition calls at its sites (their champions' impls go along).
STANDALONE_SLOTS = {
    "gated_delta_rule": ("causal_conv",),
    "gqa_attention": ("rms_norm", "qkv_projection_rope"),
    "causal_conv": (),
    "rms_norm": (),
    "qkv_projection_rope": (),
}


@dataclass
class _Gemv:
    weight: ops.Int4Weight
    plan: ops.GemvPlan
    ws: torch.Tensor | None


@dataclass
class _Layer:
    kind: str
    in_norm: torch.Tensor
    post_norm: torch.Tensor
    proj: _Gemv
    out: _Gemv
    gate_up: _Gemv
    down: _Gemv
    extra: dict = field(default_factory=dict)


def _cat_cols(parts):
    return torch.cat([p.packed for p in parts], dim=1), torch.cat([p.scale for p in parts], dim=1)


class DecodeEngine:
    """Greedy decode of a ``SynthModel`` (or any canonical int4 checkpoint) on one GPU."""

    def __init__(self, model: SynthModel, *, batch: int = 1, max_seq_len: int = 4096 + 256 + 64,
                 device: str | torch.device = "cuda", max_new_tokens: int = 256,
                 standalone: dict | None = None) -> None:
        c: ModelConfig = model.config
        if c.output_gate_type != SIGMOID_GATE and c.output_gate_type != "swish":
            raise ValueError(f"unknown gate {c.output_gate_type}")
        self.standalone = dict(standalone or {})
        unknown = set(self.standalone) - set(STANDALONE_SLOTS)
        if unknown:
            raise ValueError(f"no standalone composition for {sorted(unknown)}; known: {sorted(STANDALONE_SLOTS)}")
        for slot, needs in STANDALONE_SLOTS.items():
            if slot in self.standalone:
                absent = [n for n in needs if n not in self.standalone]
                if absent:
                    raise ValueError(f"the standalone {slot} step also calls {absent}; pass their kernels too")
        self.config = c
        self.batch = batch
        self.max_seq_len = max_seq_len
        self.device = dev = torch.device(device)
        self.max_new_tokens = max_new_tokens
        p = {k: v.to(dev) for k, v in model.params.items()}
        lin = model.linears

        def gemv(packed, scale, rows=batch, epilogue=N.EPI_STORE) -> _Gemv:
            w = ops.int4_repack(packed.to(dev), scale.to(dev))
            plan = ops.gemv_plan(rows, w.K, w.N, epilogue)
            ws = torch.zeros(plan.workspace_bytes, dtype=torch.uint8, device=dev) if plan.workspace_bytes else None
            return _Gemv(w, plan, ws)

        self.layers: list[_Layer] = []
        for i, kind in enumerate(c.layer_types):
            pre = f"layers.{i}."
            gu = ops.interleave_gate_up(lin[pre + "mlp.gate_proj.weight"].packed, lin[pre + "mlp.gate_proj.weight"].scale,
                                        lin[pre + "mlp.up_proj.weight"].packed, lin[pre + "mlp.up_proj.weight"].scale)
            mlp_gu = gemv(*gu, epilogue=N.EPI_SWIGLU)
            mlp_down = gemv(lin[pre + "mlp.down_proj.weight"].packed, lin[pre + "mlp.down_proj.weight"].scale)
            if kind == FULL_ATTENTION:
                a = pre + "self_attn."
                proj = gemv(*_cat_cols([lin[a + "q_proj.weight"], lin[a + "k_proj.weight"], lin[a + "v_proj.weight"]]))
                out = gemv(lin[a + "o_proj.weight"].packed, lin[a + "o_proj.weight"].scale)
                cache_shape = (batch, c.num_key_value_heads, max_seq_len, c.head_dim)
                extra = {
                    "q_norm": p[a + "q_norm.weight"], "k_norm": p[a + "k_norm.weight"],
                    "k_cache": torch.zeros(cache_shape, dtype=BF16, device=dev),
                    "v_cache": torch.zeros(cache_shape, dtype=BF16, device=dev),
                }
            else:
                a = pre + "linear_attn."
                proj = gemv(*_cat_cols([lin[a + "in_proj_qkv.weight"], lin[a + "in_proj_z.weight"],
                                        lin[a + "in_proj_a.weight"], lin[a + "in_proj_b.weight"]]))
                out = gemv(lin[a + "out_proj.weight"].packed, lin[a + "out_proj.weight"].scale)
                extra = {
                    "conv_w": p[a + "conv1d.weight"].reshape(c.linear_conv_dim, -1).contiguous(),
                    "A_log": p[a + "A_log"], "dt_bias": p[a + "dt_bias"], "gnorm": p[a + "norm.weight"],
                    "conv_ring": torch.zeros((batch, c.linear_conv_dim, 4), dtype=BF16, device=dev),
                    "state": torch.zeros((batch, c.linear_num_value_heads, c.linear_key_head_dim,
                                          c.linear_value_head_dim), dtype=torch.float32, device=dev),
                }
                if "gated_delta_rule" in self.standalone:  # the conv op keeps a shifting 3-tap history
                    extra["conv_hist"] = torch.zeros((batch, c.linear_conv_dim, 3), dtype=BF16, device=dev)
            self.layers.append(_Layer(kind, p[pre + "input_layernorm.weight"], p[pre + "post_attention_layernorm.weight"],
                                      proj, out, mlp_gu, mlp_down, extra))
        self.head = gemv(lin["lm_head"].packed, lin["lm_head"].scale)
        self.final_norm = p["norm.weight"]
        self.inv_freq = inv_freq(c).to(dev)
        # a checkpoint's own bf16 embedding table (``checkpoint.load_checkpoint``); without one the
        # token rows come from the tied int4 head, which is the synthetic model's table
        table = p.get("embed_tokens.weight")
        if table is not None and tuple(table.shape) != (c.vocab_size, c.hidden_size):
            raise ValueError(f"embed_tokens.weight must be [{c.vocab_size}, {c.hidden_size}], got {tuple(table.shape)}")
        self.embed_table = table.to(torch.bfloat16).contiguous() if table is not None else None
        self.splits = ops.attention_splits(batch, c.num_key_value_heads, max_seq_len)
        attn_ws = int(N.lib().df_attention_decode_workspace_bytes(batch, c.num_attention_heads, c.num_key_value_heads,
                                                                  c.head_dim, self.splits))
        self.attn_ws = torch.zeros(attn_ws, dtype=torch.uint8, device=dev)
        self.argmax_ws = torch.zeros(int(N.lib().df_argmax_workspace_bytes(batch, c.vocab_size)),
                                     dtype=torch.uint8, device=dev)

        # Activations and decode-loop state.
        width = max(c.linear_conv_dim + c.linear_value_dim + 2 * c.linear_num_value_heads,
                    2 * c.num_attention_heads * c.head_dim + 2 * c.num_key_value_heads * c.head_dim)
        self.h = torch.zeros((batch, c.hidden_size), dtype=BF16, device=dev)
        self.proj = torch.zeros((batch, width), dtype=BF16, device=dev)
        self.core = torch.zeros((batch, max(c.linear_value_dim, c.num_attention_heads * c.head_dim)),
                                dtype=BF16, device=dev)
        self.act = torch.zeros((batch, c.intermediate_size), dtype=BF16, device=dev)
        self.logits = torch.zeros((batch, c.vocab_size), dtype=BF16, device=dev)
        self.tokens = torch.zeros(batch, dtype=torch.int64, device=dev)
        self.token_log = torch.zeros((batch, max_new_tokens), dtype=torch.int64, device=dev)
        self.position = torch.zeros(1, dtype=torch.int32, device=dev)
        self.step_index = torch.zeros(1, dtype=torch.int32, device=dev)
        # A standalone attention op takes the cache up to the current key as a tensor, so its
        # length is read on the host: such steps run eagerly and keep this mirror in step.
        self.host_position = 0
        self.prompt: torch.Tensor | None = None
        self._graphs: dict[str, torch.cuda.CUDAGraph] = {}

    # -- the step -------------------------------------------------------------------------

    def _gemv(self, g: _Gemv, x, **kw):
        return ops.int4_gemv(x, g.weight, plan=g.plan, ws=g.ws, eps=self.config.rms_norm_eps, **kw)

    def _standalone_delta(self, layer: _Layer, core: torch.Tensor) -> None:
        """The Gated DeltaNet middle through the standalone ops at their call sites, composed
        as the reference composes them when its ``delta_rule_step`` is installed
        (kernels/gated_delta_step.py:231-300): the causal conv op over a 3-tap history, the
        step's inputs (L2 norms, q scale, gates), the delta-rule op on the fp32 state, and
        the output cast to bf16 for the gated norm."""
        c, e = self.config, layer.extra
        conv_c, vd, hv = c.linear_conv_dim, c.linear_value_dim, c.linear_num_value_heads
        conv = self.standalone["causal_conv"](self.proj[:, :conv_c].unsqueeze(-1), e["conv_hist"], e["conv_w"])
        q, k, v, g, beta = ops.delta_step_inputs(conv.squeeze(-1), self.proj[:, conv_c + vd:conv_c + vd + hv],
                                                 self.proj[:, conv_c + vd + hv:conv_c + vd + 2 * hv], e["A_log"],
                                                 e["dt_bias"], num_k_heads=c.linear_num_key_heads,
                                                 head_v_dim=c.linear_value_head_dim)
        out, state = self.standalone["gated_delta_rule"](e["state"], q, k, v, g, beta)
        e["state"].copy_(state)
        core.copy_(out)

    def _standalone_attention(self, layer: _Layer) -> None:
        """Gated attention through the standalone ops at their call sites, composed as the
        reference composes them when its split-KV op is installed
        (kernels/flash_decode_splitkv.py:289-334): q/k RMSNorm, partial RoPE, the key and
        value written at the position, the split-KV op over the cache so far, the output gate."""
        c, e = self.config, layer.extra
        b, hq, hkv, d = self.batch, c.num_attention_heads, c.num_key_value_heads, c.head_dim
        qd, kd, pos, eps = 2 * hq * d, hkv * d, self.host_position, c.rms_norm_eps
        if pos >= self.max_seq_len:
            raise ValueError(f"position {pos} is past the cache ({self.max_seq_len})")
        q_gate = self.proj[:, :qd].view(b, hq, 2, d)
        norm, rope = self.standalone["rms_norm"], self.standalone["qkv_projection_rope"]
        query = norm(q_gate[:, :, 0].contiguous(), e["q_norm"], eps)
        key = norm(self.proj[:, qd:qd + kd].reshape(b, hkv, d).contiguous(), e["k_norm"], eps)
        angles = float(pos) * self.inv_freq
        emb = torch.cat((angles, angles)).view(1, 1, -1).expand(b, 1, -1)
        cos, sin = emb.cos().to(BF16), emb.sin().to(BF16)
        query = rope(query.unsqueeze(2), cos, sin)[:, :, 0]
        key = rope(key.unsqueeze(2), cos, sin)[:, :, 0]
        e["k_cache"][:, :, pos] = key
        e["v_cache"][:, :, pos] = self.proj[:, qd + kd:qd + 2 * kd].reshape(b, hkv, d)
        attn = self.standalone["gqa_attention"](query.contiguous(), e["k_cache"][:, :, :pos + 1].contiguous(),
                                                e["v_cache"][:, :, :pos + 1].contiguous(), d ** -0.5, STANDALONE_SPLITS)
        gate = q_gate[:, :, 1].reshape(b, hq * d).float()
        gate = (torch.sigmoid(gate) if c.output_gate_type == SIGMOID_GATE else torch.nn.functional.silu(gate)).to(BF16)
        torch.mul(attn.reshape(b, hq * d), gate, out=self.core[:, :hq * d])

    def enqueue_step(self, *, from_prompt: bool = False, log_token: bool = True) -> None:
        """Launch one decode step on the current stream (no host sync, no allocation; with a
        standalone slot the step allocates its op outputs and must run eagerly)."""
        c = self.config
        if self.embed_table is not None:
            ops.embed_bf16(self.tokens, self.embed_table, self.h, prompt=self.prompt if from_prompt else None,
                           position=self.position if from_prompt else None)
        else:
            ops.embed_int4(self.tokens, self.head.weight, self.h, prompt=self.prompt if from_prompt else None,
                           position=self.position if from_prompt else None)
        conv_c, vd, hv = c.linear_conv_dim, c.linear_value_dim, c.linear_num_value_heads
        qd, kd = 2 * c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim
        for layer in self.layers:
            e = layer.extra
            self._gemv(layer.proj, self.h, prologue=N.PRO_RMSNORM, norm_w=layer.in_norm,
                       out=self.proj[:, :layer.proj.weight.N])
            if layer.kind == FULL_ATTENTION and "gqa_attention" in self.standalone:
                self._standalone_attention(layer)
                self._gemv(layer.out, self.core[:, :c.num_attention_heads * c.head_dim],
                           epilogue=N.EPI_RESIDUAL, res=self.h, out=self.h)
            elif layer.kind == FULL_ATTENTION:
                ops.attention_decode(self.proj[:, :qd], self.proj[:, qd:qd + kd], self.proj[:, qd + kd:qd + 2 * kd],
                                     e["q_norm"], e["k_norm"], self.inv_freq, e["k_cache"], e["v_cache"],
                                     self.position, num_q_heads=c.num_attention_heads, splits=self.splits,
                                     gate=0 if c.output_gate_type == SIGMOID_GATE else 1, eps=c.rms_norm_eps,
                                     out=self.core[:, :c.num_attention_heads * c.head_dim], ws=self.attn_ws)
                self._gemv(layer.out, self.core[:, :c.num_attention_heads * c.head_dim],
                           epilogue=N.EPI_RESIDUAL, res=self.h, out=self.h)
            else:
                core = self.core[:, :vd].view(self.batch, hv, c.linear_value_head_dim)
                if "gated_delta_rule" in self.standalone:
                    self._standalone_delta(layer, core)
                else:
                    ops.gated_delta_step(self.proj[:, :conv_c], self.proj[:, conv_c + vd:conv_c + vd + hv],
                                         self.proj[:, conv_c + vd + hv:conv_c + vd + 2 * hv], e["A_log"],
                                         e["dt_bias"], e["conv_w"], e["state"], num_k_heads=c.linear_num_key_heads,
                                         conv_ring=e["conv_ring"], position=self.position, out=core)
                self._gemv(layer.out, self.core[:, :vd], prologue=N.PRO_GATED_RMSNORM,
                           x2=self.proj[:, conv_c:conv_c + vd], norm_w=e["gnorm"],
                           epilogue=N.EPI_RESIDUAL, res=self.h, out=self.h)
            self._gemv(layer.gate_up, self.h, prologue=N.PRO_RMSNORM, norm_w=layer.post_norm,
                       epilogue=N.EPI_SWIGLU, out=self.act)
            self._gemv(layer.down, self.act, epilogue=N.EPI_RESIDUAL, res=self.h, out=self.h)
        self._gemv(self.head, self.h, prologue=N.PRO_RMSNORM, norm_w=self.final_norm, epilogue=N.EPI_LOGITS,
                   out=self.logits)
        ops.argmax_tokens(self.logits, self.tokens, token_log=self.token_log if log_token else None,
                          position=self.position, advance=1, step=self.step_index, ws=self.argmax_ws)

    # -- graphs ---------------------------------------------------------------------------

    @property
    def capturable(self) -> bool:
        """Whether the step can be captured: not with a standalone slot, whose ops take the
        cache length from the host and allocate their outputs."""
        return not self.standalone

    def graph(self, kind: str) -> torch.cuda.CUDAGraph:
        """The captured step: ``"decode"`` (token from the last argmax) or ``"prefill"``."""
        if not self.capturable:
            raise RuntimeError(f"a step with standalone {sorted(self.standalone)} cannot be captured")
        if kind not in self._graphs:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.enqueue_step(from_prompt=kind == "prefill", log_token=kind == "decode")
            self._graphs[kind] = g
        return self._graphs[kind]

    # -- decode loop ----------------------------------------------------------------------

    def reset(self) -> None:
        for layer in self.layers:
            for t in layer.extra.values():
                if t.dtype in (BF16, torch.float32) and t.dim() >= 3:
                    t.zero_()
        self.position.zero_()
        self.step_index.zero_()
        self.host_position = 0

    def set_prompt(self, prompt: torch.Tensor) -> None:
        prompt = prompt.to(self.device, torch.int64).contiguous()
        if prompt.shape[0] != self.batch:
            raise ValueError(f"prompt batch {prompt.shape[0]} != engine batch {self.batch}")
        if self.prompt is None or self.prompt.shape != prompt.shape:
            self.prompt = prompt.clone()
            self._graphs.pop("prefill", None)
        else:
            self.prompt.copy_(prompt)

    def prefill(self, prompt: torch.Tensor, *, graph: bool = True) -> None:
        """Teacher-force the prompt through the decode step (the last step's argmax is the first
        generated token, in ``self.tokens``)."""
        self.reset()
        self.set_prompt(prompt)
        if prompt.shape[1] + self.max_new_tokens > self.max_seq_len:
            raise ValueError("prompt + max_new_tokens exceeds the cache")
        if graph and self.capturable:
            g = self.graph("prefill")
            for _ in range(prompt.shape[1]):
                g.replay()
            self.host_position += prompt.shape[1]
        else:
            for _ in range(prompt.shape[1]):
                self.enqueue_step(from_prompt=True, log_token=False)
                self.host_position += 1
        self.step_index.zero_()

    def decode(self, steps: int, *, graph: bool = True) -> None:
        """Greedy steps from ``self.tokens``; tokens land in ``token_log[:, step]``."""
        if graph and self.capturable:
            g = self.graph("decode")
            for _ in range(steps):
                g.replay()
            self.host_position += steps
        else:
            for _ in range(steps):
                self.enqueue_step()
                self.host_position += 1

    def row_caches(self, row: int) -> list[dict]:
        """Row ``row``'s caches per layer, as the prefill kernels take them: ``conv_ring``
        ``[C, 4]`` and ``state`` ``[Hv, 128, 128]``, or ``k_cache``/``v_cache``
        ``[Hkv, max_len, 256]`` (views, so a prefill writes the engine's own caches)."""
        keys = ("k_cache", "v_cache", "conv_ring", "state")
        return [{k: layer.extra[k][row] for k in keys if k in layer.extra} for layer in self.layers]

    def finish_fill(self, prompt_len: int) -> None:
        """After an external prefill of ``prompt_len`` tokens: the position, and the 3-tap
        histories a standalone conv step reads, taken from the rings (the last three inputs,
        oldest first, sit in slots ``prompt_len + 1 .. + 3`` mod 4)."""
        for layer in self.layers:
            hist = layer.extra.get("conv_hist")
            if hist is not None:
                slots = [(prompt_len + 1 + j) % 4 for j in range(3)]
                hist.copy_(layer.extra["conv_ring"][:, :, slots])
        self.position.fill_(prompt_len)
        self.step_index.zero_()
        self.host_position = prompt_len

    def state_tensors(self) -> list[torch.Tensor]:
        out = []
        for layer in self.layers:
            out += [t for t in layer.extra.values() if t.dim() >= 3]
        return out + [self.position, self.step_index, self.tokens, self.h]

    def snapshot(self) -> list[torch.Tensor]:
        return [t.clone() for t in self.state_tensors()]

    def restore(self, snap: list[torch.Tensor]) -> None:
        """Copy a snapshot back in place (addresses, and so the captured graphs, stay valid)."""
        for t, s in zip(self.state_tensors(), snap):
            t.copy_(s)
        self.host_position = int(self.position.item())

    # -- accounting -------------------------------------------------------------------------

    def weight_bytes(self) -> int:
        total = self.head.weight.nbytes
        for layer in self.layers:
            total += sum(g.weight.nbytes for g in (layer.proj, layer.out, layer.gate_up, layer.down))
        return total
