"""A/B of two builds of the decode library on config 5, with the interleaved harness.

    python -m deltaforge_amd.harness.ab --candidate path/to/libdeltaforge_hip.so \\
        [--baseline path/to/lib.so] [--tokens 64] [--rounds 9] [--record results.jsonl]

Three columns, each its own ``PersistentDecoder`` on the same model: ``baseline`` (the
in-tree build unless ``--baseline`` names another), ``candidate``, and ``identity`` (the
baseline build a second time: the calibration column, which must score 1.00 within the
noise band). Each decoder prefills the benchmark's prompt once; before every timed call a
setup restores its post-prefill caches (outside the timed region), and the timed call is one
persistent launch of ``--tokens`` greedy steps. Correctness: after the rounds the candidate's
and the identity's last-step logits are compared with the baseline's (KL, argmax, largest
difference). One JSON record (``ResultRecord``) goes to stdout and, with ``--record``, is
appended to that file.
"""

from __future__ import annotations

import argparse
import json
import sys
import time

import torch

from .. import _native as N
from .. import synth
from ..config import qwen3_5_4b_config
from ..persistent import PersistentDecoder
from .bench import BenchConfig, ResultRecord, calibration_holds, outcome, run_interleaved
from .bytes_model import mean_decode_bytes
from .correctness import kl_and_agreement


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--candidate", required=True)
    ap.add_argument("--baseline", default=str(N.LIB_PATH))
    ap.add_argument("--prompt-len", type=int, default=4096)
    ap.add_argument("--fill", choices=("steps", "parallel"), default="steps",
                    help="prompt fill: teacher-forced steps of each build's own kernel, or the parallel "
                         "prefill (the same caches for every column; long prompts in seconds)")
    ap.add_argument("--tokens", type=int, default=64)
    ap.add_argument("--rounds", type=int, default=9)
    ap.add_argument("--warmup-rounds", type=int, default=2)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--record", default=None)
    ap.add_argument("--name", default="persistent decode, config 5")
    args = ap.parse_args(argv)

    def log(msg: str) -> None:
        print(f"[ab] {msg}", file=sys.stderr, flush=True)

    cfg = qwen3_5_4b_config()
    model = synth.synth_model(cfg, seed=args.seed)
    prompt = synth.prompt_ids(cfg.vocab_size, args.prompt_len, seed=1).cuda()
    names = ("df_decode_persistent_workspace_bytes", "df_decode_persistent")
    libs = {"baseline": N.load(args.baseline, names), "candidate": N.load(args.candidate, names)}
    libs["identity"] = libs["baseline"]
    decoders, snaps = {}, {}
    filler = None
    if args.fill == "parallel":
        from ..prefill import Prefiller

        filler = Prefiller(model)
    for label, lib in libs.items():
        t0 = time.time()
        dec = PersistentDecoder(model, max_seq_len=args.prompt_len + args.tokens + 8, max_new_tokens=args.tokens,
                                lib=lib)
        if filler is not None:
            filler.fill(dec, prompt)
        else:
            dec.prefill(prompt)
        dec.check()
        decoders[label] = dec
        snaps[label] = dec.snapshot()
        log(f"{label}: loaded and prefilled {args.prompt_len} in {time.time() - t0:.1f}s")

    def column(label):
        return lambda: decoders[label].decode(args.tokens)

    def setup(label):
        return lambda: decoders[label].restore(snaps[label])

    per_token = mean_decode_bytes(cfg, args.prompt_len, args.tokens)
    config = BenchConfig(rounds=args.rounds, warmup_rounds=args.warmup_rounds, baseline="baseline",
                         bytes_per_call={k: per_token * args.tokens for k in decoders})
    res = run_interleaved({k: column(k) for k in decoders}, config, setups={k: setup(k) for k in decoders},
                          progress=lambda i, label, ms: log(f"round {i} {label}: {ms:.3f} ms"))
    for dec in decoders.values():
        dec.check()
    base_logits = decoders["baseline"].logits.float().cpu()
    corr = {}
    for label in ("candidate", "identity"):
        got = decoders[label].logits.float().cpu()
        kl, agree = kl_and_agreement(base_logits, got)
        same_tokens = bool(torch.equal(decoders[label].token_log[:, : args.tokens].cpu(),
                                       decoders["baseline"].token_log[:, : args.tokens].cpu()))
        corr[label] = {"kl_last_step": float(kl.mean()), "argmax_agrees": bool(agree.all()),
                       "max_abs_logit_diff": float((got - base_logits).abs().max()), "same_tokens": same_tokens}
    ratio, iqr = res.median_ratio["candidate"], res.iqr_ratio["candidate"]
    cal = {"median_ratio": res.median_ratio["identity"], "iqr": res.iqr_ratio["identity"],
           "holds": calibration_holds(res.median_ratio["identity"], res.iqr_ratio["identity"])}
    correct = corr["candidate"]["argmax_agrees"] and corr["candidate"]["kl_last_step"] < 1e-3
    rec = ResultRecord(
        kind="ab", outcome=outcome(ratio, iqr, correct=correct) if cal["holds"] else "error",
        config_name=args.name,
        workload={"prompt_len": args.prompt_len, "fill": args.fill, "tokens_per_call": args.tokens, "seed": args.seed,
                  "baseline": args.baseline, "candidate": args.candidate, "bytes_per_token": per_token},
        bench=res.to_dict(), correctness=corr, calibration=cal)
    if args.record:
        rec.append_to(args.record)
    med = res.median_ms
    log(f"baseline {med['baseline'] / args.tokens * 1e3:.1f} us/token, candidate "
        f"{med['candidate'] / args.tokens * 1e3:.1f} us/token: ratio {ratio:.4f} (IQR {iqr:.4f}), "
        f"identity {cal['median_ratio']:.4f}, outcome {rec.outcome}; candidate KL {corr['candidate']['kl_last_step']:.2e}")
    print(json.dumps(rec.to_dict(), sort_keys=True))
    return 0


if __name__ == "__main__":
    sys.exit(main())
