"""Where a decode token's time goes inside the persistent kernel: one traced step, per phase.

    python -m deltaforge_amd.build --trace          # the stamping build, beside the product one
    python -m deltaforge_amd.harness.phase_trace    # on a GPU: prints the tables below

The config-5 model (``synth_model(seed=0)``) is prefilled with the benchmark's 4096-token
prompt, decodes a few tokens, and step ``--step`` of a ``--steps`` launch is traced from
workgroup (XCD 0, rank 0) (``PersistentDecoder.trace_decode``). The control wave's stamps give
the per-layer durations and the time from each phase's start to the next phase's start,
summed per phase kind over the token; the compute waves' stamps give, for one Gated DeltaNet
and one attention layer, when each wave finished its share of each GEMV phase. Stamps are
s_memrealtime (100 MHz, 10 ns).
"""

from __future__ import annotations

import argparse
import collections

PHASES = {1: "proj", 2: "delta", 3: "out", 4: "attn", 5: "merge", 6: "oproj", 7: "gateup", 8: "down", 9: "head",
          10: "embed", 11: "reduce"}
POINTS = {20: "staged", 30: "signal", 21: "dn-landed", 22: "dn-state", 23: "dn-done", 31: "ar-landed",
          32: "ar-local", 34: "gu-landed", 35: "head-consumed", 36: "head-done", 40: "consume", 42: "consumed",
          43: "dn-in", 44: "dn-conv", 45: "dn-math", 60: "at-staged", 61: "at-roped", 62: "at-qk",
          63: "at-softmax", 64: "at-pv", 65: "at-done"}


def decode_stamps(stamps: list[int]) -> list[tuple[float, str]]:
    """``(microseconds, name)`` per stamp."""
    return [((t >> 8) / 100.0, PHASES.get(t & 255) or POINTS.get(t & 255, str(t & 255))) for t in stamps]


def phase_totals(ctl: list[tuple[float, str]]) -> list[tuple[str, float, int]]:
    """``(phase, total us, count)``: each phase start to the next phase start, summed."""
    starts = [(t, n) for t, n in ctl if n in PHASES.values()]
    tot = collections.defaultdict(float)
    cnt = collections.Counter()
    for (t0, n), (t1, _) in zip(starts, starts[1:]):
        tot[n] += t1 - t0
        cnt[n] += 1
    return sorted(((n, tot[n], cnt[n]) for n in tot), key=lambda r: -r[1])


def layer_windows(ctl: list[tuple[float, str]]) -> list[tuple[float, float, bool]]:
    """``(start, end, is_attention)`` per layer: from one input projection to the next."""
    starts = [t for t, n in ctl if n == "proj"]
    heads = [t for t, n in ctl if n == "head"]
    ends = starts[1:] + heads[:1]
    out = []
    for s, e in zip(starts, ends):
        out.append((s, e, any(n == "attn" and s <= t < e for t, n in ctl)))
    return out


def report(trace: dict) -> str:
    ctl = decode_stamps(trace["control"])
    if not ctl:
        return "no stamps: load the traced build (python -m deltaforge_amd.build --trace)"
    base = ctl[0][0]
    lines = [f"traced step: {ctl[-1][0] - base:.1f} us from the embedding to the head's last stamp"]
    marks = {n: t for t, n in ctl if n in ("head", "head-consumed", "head-done")}
    if len(marks) == 3:
        lines.append(f"head: {marks['head-consumed'] - marks['head']:.1f} us of GEMV (this workgroup's tiles), "
                     f"{marks['head-done'] - marks['head-consumed']:.1f} us to the argmax over all workgroups")
    lines.append("")
    lines.append("| phase (start to next start) | total us | count | per phase us | share |")
    lines.append("|---|---:|---:|---:|---:|")
    rows = phase_totals(ctl)
    whole = sum(r[1] for r in rows)
    for n, tot, c in rows:
        lines.append(f"| {n} | {tot:.1f} | {c} | {tot / c:.2f} | {100 * tot / whole:.1f} % |")
    layers = layer_windows(ctl)
    dn = [e - s for s, e, a in layers if not a]
    at = [e - s for s, e, a in layers if a]
    lines.append("")
    if dn:
        lines.append(f"Gated DeltaNet layers: {len(dn)}, mean {sum(dn) / len(dn):.2f} us (min {min(dn):.2f}, "
                     f"max {max(dn):.2f})")
    if at:
        lines.append(f"attention layers: {len(at)}, mean {sum(at) / len(at):.2f} us (min {min(at):.2f}, "
                     f"max {max(at):.2f})")
    waves = [decode_stamps(w) for w in trace["waves"]]
    for label, pick in (("Gated DeltaNet", False), ("attention", True)):
        win = next(((s, e) for s, e, a in layers[4:] if a == pick), None)
        if win is None:
            continue
        s, e = win
        lines.append("")
        lines.append(f"One {label} layer (us from its input projection's start; C = control wave, "
                     "Wn = compute wave n's consume end):")
        ev = [(t, "C", n) for t, n in ctl if s <= t <= e]
        for w, row in enumerate(waves):
            ev += [(t, f"W{w}", n) for t, n in row if s <= t <= e and n in ("consumed", "at-done")]
        ev.sort()
        for t, who, n in ev:
            lines.append(f"    {t - s:7.2f}  {who:3s} {n}")
    return "\n".join(lines)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--lib", default=None, help="traced library (default: _lib/libdeltaforge_hip_trace.so)")
    ap.add_argument("--prompt-len", type=int, default=4096)
    ap.add_argument("--steps", type=int, default=6)
    ap.add_argument("--step", type=int, default=3)
    args = ap.parse_args(argv)

    from .. import _native as N
    from .. import synth
    from ..build import TRACE_LIB
    from ..config import qwen3_5_4b_config
    from ..persistent import PersistentDecoder
    from ..prefill import Prefiller

    lib = N.load(args.lib or str(TRACE_LIB), ("df_decode_persistent_workspace_bytes", "df_decode_persistent"))
    cfg = qwen3_5_4b_config()
    model = synth.synth_model(cfg, seed=0)
    prompt = synth.prompt_ids(cfg.vocab_size, args.prompt_len, seed=1).cuda()
    dec = PersistentDecoder(model, max_seq_len=args.prompt_len + 64, max_new_tokens=32, lib=lib)
    Prefiller(model).fill(dec, prompt)
    dec.check()
    snap = dec.snapshot()
    dec.decode(8)
    dec.check()
    dec.restore(snap)
    print(report(dec.trace_decode(args.steps, args.step)))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
