"""Per-kernel timing of the standalone ops at the benchmark's configs 1-4.

    python -m deltaforge_amd.harness.kernel_bench [--config 1 2 3 4] [--calls 50] [--rounds 7]

One JSON line per case on stdout: the median and IQR of the per-call time over ``--rounds``
rounds of ``--calls`` back-to-back calls (HIP events on the stream the ops launch on, torch's
current stream), the algorithmic bytes per call (``bytes_model``), GB/s and the fraction of
the 8 TB/s HBM peak. Cases follow the reference's config table: 1 the tied head with its
residual + RMSNorm prologue; 2 the gated delta step at B = 1, 8; 3 split-KV decode attention at
B = 1, 8 and contexts 4096, 32768, 131072; 4 the int4 MLP block (RMSNorm + gate|up + SwiGLU,
then down + residual) at 1 and 16 rows.

The MI355X's 256 MB last-level cache (MALL) would serve a repeated small input from cache, so
every case rotates through copies of its inputs whose total exceeds 512 MB (one copy when a
single one already does), and call i uses copy i mod n. Inputs are random device tensors of
the configs' shapes and distributions; the numerics of these ops are checked by the tests,
not here. ``--profile-calls N`` runs each case N times with no timing, for rocprofv3 runs
that take their durations from the kernel trace.
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from typing import Callable

import torch

from .. import _native as N
from .. import ops, synth
from ..config import qwen3_5_4b_config
from .bench import median, quantile
from .bytes_model import HBM_PEAK_BYTES_PER_S, attention_bytes, delta_bytes, head_bytes, mlp_bytes

BF16 = torch.bfloat16
ROTATE_BYTES = 512 << 20


def _copies(one_set_bytes: int) -> int:
    return max(1, -(-ROTATE_BYTES // max(one_set_bytes, 1)))


def _int4(gen: torch.Generator, k: int, n: int, dev) -> ops.Int4Weight:
    packed = torch.randint(0, 256, (k // 2, n), dtype=torch.uint8, device=dev, generator=gen)
    scale = (torch.randn((k // 128, n), device=dev, generator=gen).abs() * 0.02).to(BF16)
    return ops.int4_repack(packed, scale)


def _randn(gen, shape, dev, std=1.0, dtype=BF16):
    return (torch.randn(shape, device=dev, generator=gen) * std).to(dtype)


def _clone_weight(w: ops.Int4Weight) -> ops.Int4Weight:
    return ops.Int4Weight(w.w.clone(), w.s.clone(), w.K, w.N)


class Case:
    def __init__(self, config: int, name: str, nbytes: int, call: Callable[[int], None], copies: int):
        self.config, self.name, self.nbytes, self.call, self.copies = config, name, nbytes, call, copies


def head_case(dev, gen) -> list[Case]:
    """Config 1: logits = bf16(RMSNorm(x + r)) @ dequant(W_head), W 2560 x 248320."""
    nb = head_bytes()
    w0 = _int4(gen, 2560, 248320, dev)
    n = _copies(w0.nbytes)
    ws = [w0] + [_clone_weight(w0) for _ in range(n - 1)]
    x, r = _randn(gen, (1, 2560), dev), _randn(gen, (1, 2560), dev)
    nw = _randn(gen, (2560,), dev, 0.02)
    out = torch.empty((1, 248320), dtype=BF16, device=dev)
    h_out = torch.empty((1, 2560), dtype=BF16, device=dev)
    plan = ops.gemv_plan(1, 2560, 248320)

    def call(i: int) -> None:
        ops.int4_gemv(x, ws[i % n], prologue=N.PRO_ADD_RMSNORM, x2=r, norm_w=nw, eps=1e-6, out=out, h_out=h_out,
                      plan=plan)

    return [Case(1, "head 2560x248320 bs=1", nb, call, n)]


def delta_cases(dev, gen) -> list[Case]:
    """Config 2: conv + L2 norms + gates + delta rule, state [B, 32, 128, 128] fp32 in place."""
    out = []
    for batch in (1, 8):
        nb = delta_bytes(batch)
        n = _copies(nb)
        chans = 8192
        sets = []
        for _ in range(n):
            sets.append({
                "state": _randn(gen, (batch, 32, 128, 128), dev, 0.1, torch.float32),
                "qkv": _randn(gen, (batch, chans), dev),
                "conv_in": _randn(gen, (batch, chans, 3), dev),
                "conv_out": torch.empty((batch, chans, 3), dtype=BF16, device=dev),
                "a": _randn(gen, (batch, 32), dev),
                "b": _randn(gen, (batch, 32), dev),
                "out": torch.empty((batch, 32, 128), dtype=BF16, device=dev),
            })
        conv_w = _randn(gen, (chans, 4), dev, 0.3)
        zeros = torch.zeros(32, dtype=BF16, device=dev)

        def call(i: int, sets=sets, n=n, conv_w=conv_w, zeros=zeros) -> None:
            s = sets[i % n]
            ops.gated_delta_step(s["qkv"], s["a"], s["b"], zeros, zeros, conv_w, s["state"], num_k_heads=16,
                                 conv_in=s["conv_in"], conv_out=s["conv_out"], out=s["out"])

        out.append(Case(2, f"gated delta step B={batch}", nb, call, n))
    return out


def attention_cases(dev, gen, contexts=(4096, 32768, 131072), batches=(1, 8)) -> list[Case]:
    """Config 3: q/k norm + RoPE + KV write + split-KV GQA decode over context + 1 keys."""
    inv = synth.inv_freq(qwen3_5_4b_config()).to(dev)
    out = []
    for batch in batches:
        for ctx in contexts:
            nb = attention_bytes(batch, ctx)
            n = _copies(nb)
            max_len = ctx + 64
            sets = []
            for _ in range(n):
                kc = torch.empty((batch, 4, max_len, 256), dtype=BF16, device=dev)
                vc = torch.empty_like(kc)
                kc.normal_(generator=gen)
                vc.normal_(generator=gen)
                sets.append({"kc": kc, "vc": vc, "q": _randn(gen, (batch, 16 * 512), dev),
                             "k": _randn(gen, (batch, 1024), dev), "v": _randn(gen, (batch, 1024), dev),
                             "out": torch.empty((batch, 16 * 256), dtype=BF16, device=dev)})
            qn, kn = _randn(gen, (256,), dev, 0.02), _randn(gen, (256,), dev, 0.02)
            position = torch.tensor([ctx], dtype=torch.int32, device=dev)

            def call(i: int, sets=sets, n=n, qn=qn, kn=kn, position=position) -> None:
                s = sets[i % n]
                ops.attention_decode(s["q"], s["k"], s["v"], qn, kn, inv, s["kc"], s["vc"], position,
                                     num_q_heads=16, out=s["out"])

            out.append(Case(3, f"split-KV attention B={batch} L={ctx}", nb, call, n))
    return out


def mlp_cases(dev, gen) -> list[Case]:
    """Config 4: RMSNorm + gate|up (2560 x 18432) + SwiGLU, then down (9216 x 2560) + residual."""
    gu0, dn0 = _int4(gen, 2560, 18432, dev), _int4(gen, 9216, 2560, dev)
    n = _copies(gu0.nbytes + dn0.nbytes)
    gus = [gu0] + [_clone_weight(gu0) for _ in range(n - 1)]
    dns = [dn0] + [_clone_weight(dn0) for _ in range(n - 1)]
    nw = _randn(gen, (2560,), dev, 0.02)
    out = []
    for rows in (1, 16):
        x = _randn(gen, (rows, 2560), dev)
        act = torch.empty((rows, 9216), dtype=BF16, device=dev)
        y = torch.empty((rows, 2560), dtype=BF16, device=dev)
        p1 = ops.gemv_plan(rows, 2560, 18432, N.EPI_SWIGLU)
        p2 = ops.gemv_plan(rows, 9216, 2560, N.EPI_RESIDUAL)

        def call(i: int, x=x, act=act, y=y, p1=p1, p2=p2) -> None:
            ops.int4_gemv(x, gus[i % n], prologue=N.PRO_RMSNORM, epilogue=N.EPI_SWIGLU, norm_w=nw, out=act, plan=p1)
            ops.int4_gemv(act, dns[i % n], epilogue=N.EPI_RESIDUAL, res=x, out=y, plan=p2)

        out.append(Case(4, f"MLP block rows={rows}", mlp_bytes(rows), call, n))
    return out


BUILDERS = {1: head_case, 2: delta_cases, 3: attention_cases, 4: mlp_cases}


def time_case(case: Case, calls: int, rounds: int, warmup: int = 5) -> dict:
    for i in range(warmup):
        case.call(i)
    torch.cuda.synchronize()
    per_call = []
    for _ in range(rounds):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(calls):
            case.call(i)
        e1.record()
        e1.synchronize()
        per_call.append(e0.elapsed_time(e1) * 1e3 / calls)
    us = median(per_call)
    gbps = case.nbytes / (us * 1e-6) / 1e9
    return {
        "config": case.config, "case": case.name, "median_us": round(us, 3),
        "iqr_us": round(quantile(per_call, 0.75) - quantile(per_call, 0.25), 3),
        "calls_per_round": calls, "rounds": rounds, "input_copies": case.copies,
        "algorithmic_bytes": case.nbytes, "GB_per_s": round(gbps, 1),
        "frac_of_8TBps": round(gbps * 1e9 / HBM_PEAK_BYTES_PER_S, 4),
    }


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--config", type=int, nargs="+", default=[1, 2, 3, 4], choices=sorted(BUILDERS))
    ap.add_argument("--calls", type=int, default=50)
    ap.add_argument("--rounds", type=int, default=7)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--profile-calls", type=int, default=0)
    ap.add_argument("--calibration-copy", action="store_true",
                    help="first run three plain 256 MiB device copies (the known-size dispatch that "
                         "scales rocprofv3's FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("kernel_bench needs a GPU", file=sys.stderr)
        return 2
    dev = torch.device("cuda", 0)
    N.lib()  # fail loudly here if the HIP library is missing
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    if args.calibration_copy:
        a = torch.ones((256 << 20) // 2, dtype=BF16, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        del a, b
        print("[kernel_bench] calibration copy: 3 x (256 MiB read + 256 MiB written)", file=sys.stderr, flush=True)
    for cfg in args.config:
        t0 = time.time()
        cases = BUILDERS[cfg](dev, gen)
        print(f"[kernel_bench] config {cfg}: {len(cases)} cases built in {time.time() - t0:.1f}s",
              file=sys.stderr, flush=True)
        for case in cases:
            if args.profile_calls:
                for i in range(args.profile_calls):
                    case.call(i)
                torch.cuda.synchronize()
                print(f"[kernel_bench] {case.name}: {args.profile_calls} calls", file=sys.stderr, flush=True)
            else:
                print(json.dumps(time_case(case, args.calls, args.rounds)), flush=True)
        del cases
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
