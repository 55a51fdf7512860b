"""Config 5 benchmark: bs=1 greedy decode of the int4 Qwen3.5-4B-shaped hybrid on one MI355X.

    python bench.py [--steps 256] [--warmup 8] [--prompt-len 4096] [--no-cpu-baseline]
                    [--engine persistent|graph]

A step is one greedy decode token. By default (``--engine persistent``) all ``steps`` tokens
run inside one launch of the persistent kernel ``df::pd::decode_kernel`` (every layer of every
token in one cooperative launch); ``--engine graph`` replays the per-op kernels as one captured
HIP graph per token instead. The prompt (4096 random ids, seed 1) is prefilled untimed by the
parallel prefill, the caches are snapshotted, ``warmup`` tokens run and the snapshot is
restored, then exactly ``steps`` tokens are timed with HIP events on the stream the decode runs
on, between device synchronisations. Weights are random-init in the model's real shapes
(synthetic data: there is no checkpoint here). One JSON line is printed.

``roofline`` is for the dominant kernel. With the persistent engine that is the decode launch
itself: achieved = the reference bytes model's weight + state + KV bytes per token
(``harness/bytes_model.py``) x tokens per launch / launch time; traffic = the HBM bytes per
launch from calibrated ``rocprofv3 --pmc FETCH_SIZE`` / ``WRITE_SIZE`` passes
(``PERSISTENT_TRAFFIC_BYTES_PER_TOKEN``). With the graph engine it is the fused RMSNorm +
gate/up int4 GEMV + SwiGLU, timed around a captured graph of the 32 layers' launches;
``--roofline-only`` runs just that graph plus a plain 256 MiB device copy for its PMC passes.
``cpu_baseline`` times the CPU oracle (``oracle/``, plain PyTorch, fp32 dequant as the
reference does) on decode steps of the same model at the same context on the host cores: the
median of ``--cpu-steps`` steps, with the thread count and the CPU model.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "decode tok/s bs=1 ctx4k on 1 MI355X; achieved HBM GB/s as % of 8 TB/s"


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt-len", type=int, default=4096)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-steps", type=int, default=3, help="CPU oracle decode steps timed (median reported)")
    ap.add_argument("--roofline-reps", type=int, default=10)
    ap.add_argument("--roofline-only", action="store_true")
    ap.add_argument("--calibration-copy", action="store_true",
                    help="after the timed decode, run three plain 256 MiB device copies (for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
    ap.add_argument("--prefill", choices=("parallel", "steps"), default="parallel",
                    help="parallel: the prompt through each layer at once (deltaforge_amd.prefill, persistent "
                         "engine only); steps: teacher-forced decode steps")
    ap.add_argument("--engine", choices=("persistent", "graph"), default="persistent",
                    help="persistent: one cooperative launch per decode run (df_decode_persistent); "
                         "graph: the per-op kernels replayed as one HIP graph per step")
    return ap.parse_args()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


GATE_UP_KERNEL = "w4_gemv_kernel<RMSNORM, SWIGLU> (post-attention norm + gate/up 2560 x 18432 + SwiGLU)"
# HBM bytes one gate/up launch actually moves: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes
# over ``--roofline-only`` (12049 KiB fetched, 18 KiB written per launch), each scaled by what
# the counter reads for a plain 256 MiB device copy (x 2.000 for FETCH_SIZE, x 1.000 for
# WRITE_SIZE). Re-measure when the kernel changes.
GATE_UP_TRAFFIC_BYTES = 12049 * 1024 * 2 + 18 * 1024
# HBM bytes per decode token of the persistent kernel from the calibrated PMC passes over the
# timed 256-token launch (334,344,530.5 KiB fetched x 1.99982, 17,625,739.0 KiB written, / 256),
# recorded with their commands in PERSISTENT_TRAFFIC_SOURCE. Re-measure when the kernel changes.
PERSISTENT_TRAFFIC_BYTES_PER_TOKEN = 2739225546
PERSISTENT_TRAFFIC_SOURCE = ("profiles/decode_persistent_config5.md: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                             "over bench.py --steps 256, scaled by a 256 MiB copy in the same process")


def gate_up_bytes(cfg) -> int:
    """Algorithmic HBM bytes of one gate/up launch: int4 weights, bf16 scales, the bf16 h row
    and norm weight read, the bf16 activation row written."""
    from deltaforge_amd.harness.bytes_model import int4_bytes

    k, n = cfg.hidden_size, 2 * cfg.intermediate_size
    return int4_bytes(k, n) + 2 * k * 2 + cfg.intermediate_size * 2


def time_gate_up(engine, reps: int) -> float:
    """Average duration (s) of one gate/up launch: a graph of every layer's launch (weights
    stream from HBM as in decode), replayed ``reps`` times between HIP events."""
    from deltaforge_amd import _native as N

    def enqueue():
        for layer in engine.layers:
            engine._gemv(layer.gate_up, engine.h, prologue=N.PRO_RMSNORM, norm_w=layer.post_norm,
                         epilogue=N.EPI_SWIGLU, out=engine.act)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        enqueue()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        enqueue()
    graph.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        graph.replay()
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / 1e3 / (reps * len(engine.layers))


def copy_calibration(mib: int = 256) -> None:
    """A plain device copy of ``mib`` MiB (reads and writes exactly that much) for scaling the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters."""
    a = torch.empty(mib * 1024 * 1024 // 2, dtype=torch.bfloat16, device="cuda").fill_(1.0)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    log(f"calibration copy: {mib} MiB read + {mib} MiB written per launch (3 launches)")


def cpu_model_name() -> str:
    """The host CPU's model name as ``lscpu`` prints it (``/proc/cpuinfo`` if lscpu is absent)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        name = next((ln.split(":", 1)[1].strip() for ln in out.splitlines() if ln.startswith("Model name")), None)
        if name:
            return name
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        with open("/proc/cpuinfo") as f:
            return next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")), "unknown CPU")
    except OSError:
        return "unknown CPU"


def cpu_baseline(model, position: int, steps: int = 3) -> dict:
    """``steps`` decode steps of the CPU oracle at ``position`` (a bounded sample of the same
    workload), median reported. Threads are torch's default for this process (the box sets
    ``OMP_NUM_THREADS``); the count reported is ``torch.get_num_threads()``."""
    import statistics

    from oracle.int4 import dequantise_int4_k_major
    from oracle.model import OracleModel

    params = dict(model.params)
    head = model.linears["lm_head"]
    params["embed_tokens.weight"] = dequantise_int4_k_major(head.packed, head.scale, 128).to(torch.bfloat16).t().contiguous()
    oracle = OracleModel(model.config, params, {n: (w.packed, w.scale, 128) for n, w in model.linears.items()})
    cache = oracle.new_cache(1, position + 2)
    gen = torch.Generator().manual_seed(3)
    for layer in cache.layers:  # a filled cache: values do not change the cost
        for t in layer.values():
            t.copy_(torch.randn(t.shape, generator=gen).to(t.dtype) * 0.1)
    cache.seq_len = position
    token = torch.tensor([[17]])
    times = []
    with torch.no_grad():
        for _ in range(max(steps, 3)):
            t0 = time.perf_counter()
            oracle.forward(token, cache, num_logits_to_keep=1)
            times.append(time.perf_counter() - t0)
            cache.seq_len = position
    med = statistics.median(times)
    threads = torch.get_num_threads()
    cpu = cpu_model_name()
    return {"value": 1.0 / med, "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"median of {len(times)} decode steps (each {', '.join(f'{t:.2f}' for t in times)} s) of the "
                      f"same 32-layer int4 model at context {position}, CPU oracle (plain PyTorch, fp32 dequant per "
                      f"linear); torch.get_num_threads() = {threads} (os.cpu_count() = {os.cpu_count()}); "
                      f"lscpu model name: {cpu}",
            "threads": threads, "cpu_model": cpu, "seconds_per_token": med}


def run_prefill(engine, model, args, persistent: bool) -> dict:
    """Fill the engine's caches with the benchmark prompt; time it with HIP events.

    Parallel mode runs ``Prefiller.fill`` twice: the first call loads the kernels, the second is
    timed. Steps mode times the engine's own teacher-forced decode steps. The decode timing
    below does not include this."""
    prompt = synth_prompt(engine.config, args.prompt_len).cuda()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    if args.prefill == "parallel" and persistent:
        from deltaforge_amd.prefill import Prefiller

        pre = Prefiller(model)
        pre.fill(engine, prompt)
        torch.cuda.synchronize()
        start.record(stream)
        pre.fill(engine, prompt)
        end.record(stream)
        mode = "parallel (deltaforge_amd.prefill: int4 GEMM, chunked delta rule, causal attention)"
        del pre
    else:
        start.record(stream)
        engine.prefill(prompt)
        end.record(stream)
        mode = "teacher-forced decode steps"
    torch.cuda.synchronize()
    if persistent:
        engine.check()
    ms = start.elapsed_time(end)
    log(f"prefill of {args.prompt_len} tokens ({mode}) in {ms:.1f} ms")
    return {"tokens": args.prompt_len, "ms": round(ms, 2), "tok_per_s": round(args.prompt_len / ms * 1e3, 1),
            "mode": mode}


def run_decode(engine, args, persistent: bool) -> tuple[float, list[int]]:
    """Warm up on a snapshot of the prefilled caches, restore, then time exactly ``args.steps``
    greedy tokens with HIP events on the stream the decode runs on. Returns (seconds, first tokens)."""
    snap = engine.snapshot()
    engine.decode(args.warmup)
    if persistent:
        engine.check()
    torch.cuda.synchronize()
    engine.restore(snap)
    torch.cuda.synchronize()

    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    engine.decode(args.steps)
    end.record(stream)
    torch.cuda.synchronize()
    if persistent:
        engine.check()
    return start.elapsed_time(end) / 1e3, engine.token_log[0, :8].tolist()


def synth_prompt(cfg, n: int) -> torch.Tensor:
    from deltaforge_amd import synth

    return synth.prompt_ids(cfg.vocab_size, n, seed=1)


PERSISTENT_KERNEL = "df::pd::decode_kernel (every layer of every decode step in one cooperative launch)"


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (this path has no "
              "multi-GPU mode; it would shard by value head, KV split and vocabulary rows).", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    from deltaforge_amd import synth
    from deltaforge_amd.config import qwen3_5_4b_config
    from deltaforge_amd.engine import DecodeEngine
    from deltaforge_amd.harness.bytes_model import HBM_PEAK_BYTES_PER_S, mean_decode_bytes
    from deltaforge_amd.persistent import PersistentDecoder

    cfg = qwen3_5_4b_config()
    t0 = time.perf_counter()
    model = synth.synth_model(cfg, seed=args.seed)
    log(f"synthetic model drawn in {time.perf_counter() - t0:.1f}s ({model.nbytes() / 1e9:.2f} GB)")
    persistent = args.engine == "persistent" and not args.roofline_only
    max_len = args.prompt_len + args.steps + args.warmup + 64
    if persistent:
        engine = PersistentDecoder(model, max_seq_len=max_len, max_new_tokens=args.steps + args.warmup)
    else:
        engine = DecodeEngine(model, max_seq_len=max_len, max_new_tokens=args.steps + args.warmup)
    torch.cuda.synchronize()
    log(f"{args.engine} engine ready: {engine.weight_bytes() / 1e9:.3f} GB of int4 weights in HBM")
    if args.roofline_only:
        gu_s = time_gate_up(engine, args.roofline_reps)
        log(f"gate/up GEMV: {gu_s * 1e6:.2f} us/launch, {gate_up_bytes(cfg) / gu_s / 1e9:.1f} GB/s")
        copy_calibration()
        return 0

    prefill = run_prefill(engine, model, args, persistent)
    seconds, tokens = run_decode(engine, args, persistent)
    if args.calibration_copy:
        copy_calibration()
    tok_s = args.steps / seconds
    bytes_per_token = mean_decode_bytes(cfg, args.prompt_len, args.steps)
    achieved = bytes_per_token * tok_s
    log(f"decode: {args.steps} tokens in {seconds * 1e3:.1f} ms -> {tok_s:.1f} tok/s, "
        f"{achieved / 1e9:.1f} GB/s ({100 * achieved / HBM_PEAK_BYTES_PER_S:.1f}% of 8 TB/s)")

    if persistent:
        # the dominant (only) kernel is the persistent decode launch; one launch = `steps` tokens
        launch_bytes = int(bytes_per_token * args.steps)
        roofline = {
            "kernel": PERSISTENT_KERNEL,
            "bound": "hbm",
            "achieved": round(launch_bytes / seconds / 1e9, 1),
            "peak": 8000.0,
            "unit": "GB/s",
            "frac": round(launch_bytes / seconds / 8e12, 4),
            "traffic": PERSISTENT_TRAFFIC_BYTES_PER_TOKEN * args.steps if PERSISTENT_TRAFFIC_BYTES_PER_TOKEN else None,
            "traffic_source": PERSISTENT_TRAFFIC_SOURCE,
            "us_per_launch": round(seconds * 1e6, 1),
            "bytes_per_launch": launch_bytes,
            "tokens_per_launch": args.steps,
        }
    else:
        gu_s = time_gate_up(engine, args.roofline_reps)
        gu_gbps = gate_up_bytes(cfg) / gu_s / 1e9
        log(f"gate/up GEMV: {gu_s * 1e6:.2f} us/launch, {gu_gbps:.1f} GB/s")
        roofline = {
            "kernel": GATE_UP_KERNEL,
            "bound": "hbm",
            "achieved": round(gu_gbps, 1),
            "peak": 8000.0,
            "unit": "GB/s",
            "frac": round(gu_gbps / 8000.0, 4),
            "traffic": GATE_UP_TRAFFIC_BYTES,
            "us_per_launch": round(gu_s * 1e6, 3),
            "bytes_per_launch": gate_up_bytes(cfg),
        }

    baseline = None
    if not args.no_cpu_baseline:
        t0 = time.perf_counter()
        baseline = cpu_baseline(model, args.prompt_len, args.cpu_steps)
        log(f"cpu baseline: {baseline['seconds_per_token']:.2f} s/token on {baseline['cores']} threads "
            f"(sample took {time.perf_counter() - t0:.1f}s)")
        baseline.pop("seconds_per_token")

    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(seconds * 1e3 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "config 5: bs=1 greedy decode of a random-init 32-layer Qwen3.5-4B-shaped hybrid "
                        "(24 Gated DeltaNet + 8 gated GQA layers), int4 group-128 weights, tied int4 head, "
                        f"prompt {args.prompt_len} ids (seed 1), {args.steps} timed greedy steps",
            "engine": args.engine,
            "batch": 1,
            "context": args.prompt_len,
            "weights": "int4 g128 nibbles + bf16 scales; bf16 activations; fp32 accumulation and state",
            "bytes_per_token": int(bytes_per_token),
            "achieved_GBps": round(achieved / 1e9, 1),
            "hbm_fraction": round(achieved / HBM_PEAK_BYTES_PER_S, 4),
            "first_tokens": tokens,
        },
        "roofline": roofline,
        "cpu_baseline": baseline,
        "prefill": prefill,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
