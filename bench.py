"""Benchmark: bf16 batch-1 greedy decode of a random-init Llama-3.2-1B on one MI355X.

Prints ONE JSON line.  The workloads (ms/token of batch-1 bf16 decode):

* ctx 1 (the headline ``value``): 1-token prompt, 256 new tokens, 64 per persistent launch;
* ctx 4096 and ctx 32768: a seeded prompt of that length prefilled, then 64 new tokens in one
  launch (reported under ``ctx4096`` / ``ctx32768``).

Each runs on a package of the same weights planned for its context: 321 positions with the
planner's default attention chunking (one fused chunk) for ctx 1, 4160 positions in 130-step
chunks for ctx 4096, 32832 positions in 1026-step chunks for ctx 32768.

A step is one ctx-1 generation of 256 tokens (``--steps`` / ``--warmup`` count them);
``value`` is ms/token of the generate launches, timed with HIP events on the context stream
(prefill, setup and readback excluded, as the reference's ``tile_runtime bench``), and
``ms_per_step`` the same per 256-token step.  The roofline block prices the decoder_worker
launches against HBM: algorithmic bytes = every weight byte plus 32 KiB of K/V per visible
position per token; ``traffic`` comes from rocprofv3 counter passes on the same worker sources
(tiles_amd/counters.py), null when none match.  ``cpu_baseline`` times the PyTorch-eager CPU
oracle (oracle/decoder.py) on the same weights, on a bounded sample (bf16 and fp32, ctx 1 and
4096).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

S_BOS = 128000                        # the prompt token of every configuration (Llama-3 BOS)
WEIGHT_BYTES = 2_471_628_800          # bf16 weights streamed per token: 1,235,814,400 parameters x 2 bytes
KV_BYTES_PER_POSITION = 32_768        # 16 layers x (K + V) x 8 heads x 64 x 2 bytes
LM_HEAD_STEP_BYTES = 525_344_768      # 128256 x 2048 bf16 LM-head rows + the hidden vector and final-norm weight
PEAK_HBM_GBPS = 8000.0                # MI355X published HBM3E bandwidth
# HBM bytes per generate launch from rocprofv3 FETCH_SIZE / WRITE_SIZE passes (tiles_amd/counters.py),
# used only while they were measured on the current worker sources.
TRAFFIC_SUMMARY = ROOT / "profiles" / "decoder_worker_hbm_traffic.json"


def log(*args) -> None:
    print(*args, file=sys.stderr, flush=True)


def bytes_per_token(position: int) -> int:
    """Algorithmic bytes to decode the token at `position` (visible prefix position + 1)."""
    return WEIGHT_BYTES + (position + 1) * KV_BYTES_PER_POSITION


def cpu_threads() -> int:
    """The host cores this process may run on: its CPU affinity set, capped by OMP_NUM_THREADS
    when that is set.  A GPU box gives one GPU's job a share of the host (16 threads), whatever
    os.cpu_count() reports for the whole machine."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(weights: dict, tokens: int) -> dict:
    """The oracle's eager decode on the host cores: median ms per decoded
    token of `tokens` greedy steps, in bf16 and fp32, at ctx 1 (after a 1-token prompt) and ctx
    4096 (after a deterministic synthetic K/V prefix of 4096 positions, uniform in [-1, 1), as the
    reference's diagnostic context fills for timing, diagnostic_context.cu:89-118)."""
    import torch

    from oracle import decoder as ref

    threads = cpu_threads()
    torch.set_num_threads(threads)
    results = {}
    for label, dtype in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        w = weights if dtype is torch.bfloat16 else {k: v.float() for k, v in weights.items()}
        for ctx in (1, 4096):
            spec = ref.Spec(hidden_size=2048, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
                            head_dim=64, max_context=ctx + tokens + 1, layers=16, vocab_size=128256)
            cache = ref.StackCache.empty(spec, dtype)
            samples = []
            with torch.inference_mode():
                if ctx == 1:
                    out = ref.decode_token(S_BOS, w, spec, cache)
                else:
                    generator = torch.Generator().manual_seed(ctx)
                    for layer in cache.layers:
                        for table in (layer.k, layer.v):
                            table[:ctx] = (torch.rand(table[:ctx].shape, generator=generator) * 2 - 1).to(dtype)
                        layer.position = ctx
                    out = ref.decode_token(S_BOS, w, spec, cache)
                for _ in range(tokens):
                    token = ref.greedy(out["logits"])
                    start = time.perf_counter()
                    out = ref.decode_token(token, w, spec, cache)
                    samples.append((time.perf_counter() - start) * 1e3)
            results[f"{label}_ctx{ctx}"] = statistics.median(samples)
            log(f"cpu baseline {label} ctx {ctx}: {results[f'{label}_ctx{ctx}']:.1f} ms/token")
        del w
        gc.collect()
    return {"value": results["bf16_ctx1"], "unit": "ms/token", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "by_config": results,
            "sample": f"{tokens} greedy decode steps per configuration (bf16 and fp32; ctx 1 after a 1-token "
                      f"prompt, ctx 4096 after a synthetic 4096-position K/V prefix) of the same random-init "
                      f"Llama-3.2-1B, PyTorch eager CPU oracle (oracle/decoder.py), median step time; value is "
                      f"bf16 at ctx 1"}


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=4,
                        help="timed steps; a step is one ctx-1 generation of 256 tokens (4 persistent launches)")
    parser.add_argument("--warmup", type=int, default=1, help="untimed steps before them")
    parser.add_argument("--no-ctx4096", action="store_true")
    parser.add_argument("--cpu-tokens", type=int, default=24, help="decode steps per CPU-baseline configuration")
    # Each configuration runs on a package planned for its context.  ctx 1 (positions 1-256): a
    # 321-position package with the planner's default chunking, one fused chunk (the planner fuses
    # contexts up to 384 positions).  ctx 4096: 130-step chunks split the 4160-position context
    # into 32 chunks per K/V head, 256 attention tasks for 256 workers (128 would give 33 chunks and
    # two tasks to 8 workers).
    parser.add_argument("--chunk-steps", type=int, default=130, help="attention chunk steps of the ctx-4096 package")
    parser.add_argument("--no-ctx32768", action="store_true",
                        help="skip the 64 tokens at context 32768 (BASELINE config 5: a package with max_context 32832 "
                             "and 1026-step attention chunks: 32 per K/V head, one attention task per worker)")
    parser.add_argument("--write-package", type=Path, default=None,
                        help="only write the ctx-1 package to this directory and its prompt to DIR.ctx1.json "
                             "(for `tiles_amd/tile_runtime bench` under a profiler), then exit")
    parser.add_argument("--write-package-ctx4096", type=Path, default=None,
                        help="only write the ctx-4096 package (max_context 4160, --chunk-steps) to this directory and "
                             "its 4096-token prompt to DIR.ctx4096.json, then exit")
    parser.add_argument("--lm-head-only", action="store_true",
                        help="only the isolated LM-head step (BASELINE config 2) on the ctx-1 package: print its JSON "
                             "object and exit (for a kernel trace of that launch alone)")
    parser.add_argument("--lm-head-rounds", type=int, default=20, help="rounds of the isolated LM-head step")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the decode worker is single-GPU); --gpus {args.gpus} is not supported",
              file=sys.stderr)
        return 2
    steps = max(1, args.steps)

    from tiles_amd import runtime as R
    from tiles_amd import synthetic as S
    from tiles_amd.tileplan import probe

    target = probe.probe_library()
    new_tokens = 256
    prompt = [S.BOS]
    ctx1_context = len(prompt) + new_tokens + 64
    if args.write_package is not None:
        S.llama_package(args.write_package, ctx1_context, "bfloat16", seed=0, target=target)
        Path(f"{args.write_package}.ctx1.json").write_text(json.dumps({"tokens": [S.BOS]}) + "\n")
        log(f"wrote {args.write_package} and {args.write_package}.ctx1.json")
        return 0
    if args.write_package_ctx4096 is not None:
        out = args.write_package_ctx4096
        S.llama_package(out, 4096 + 64, "bfloat16", seed=0, chunk_steps=args.chunk_steps, target=target)
        Path(f"{out}.ctx4096.json").write_text(json.dumps({"tokens": S.prompt(4096, seed=4096)}) + "\n")
        log(f"wrote {out} and {out}.ctx4096.json")
        return 0
    stream_gbps = R.measure_stream_read(2 << 30, 3)
    log(f"measured stream read {stream_gbps:.1f} GB/s")
    work = S.scratch_dir()
    start = time.time()
    spec, weights = S.llama_package(work / "llama", ctx1_context, "bfloat16", seed=0, target=target)
    log(f"ctx-1 package built in {time.time() - start:.1f}s")
    plan = R.load_plan(work / "llama", verify_weights=False)
    model = R.DecoderModel(plan)

    # The LM-head step alone: h ~ N(0, 1) bf16 [2048] through the final
    # RMSNorm (weight 1.0), the tied 128256 x 2048 bf16 embedding ~ N(0, 0.02) of the ctx-1 model
    # and greedy argmax, as launches of the worker's logits tasks of their own
    # (ti_context_lm_head_step): the median round's worker launch (HIP events around it), against
    # its 525,344,768 bytes.  A seed kernel before it publishes h, a selection kernel after it
    # reduces the tasks' candidates; both are outside the timed launch.
    import torch

    hidden = torch.randn(2048, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    head_ctx = model.create_context()
    bits = hidden.view(torch.int16).numpy().view("uint16")
    head = head_ctx.wait(head_ctx.enqueue_lm_head_step(bits, rounds=args.lm_head_rounds))
    del head_ctx
    head_us = head.compute_us
    lm_head_step = {"us": head_us, "bytes": LM_HEAD_STEP_BYTES, "GBps": LM_HEAD_STEP_BYTES / (head_us * 1e-6) / 1e9,
                    "fraction_of_stream_read": LM_HEAD_STEP_BYTES / (head_us * 1e-6) / 1e9 / stream_gbps,
                    "token": head.generated[0], "rounds": args.lm_head_rounds,
                    "measured": "isolated LM-head step (ti_context_lm_head_step): median over the rounds of the "
                                "worker launch running the logits tasks alone (HIP events around it)"}
    log(f"LM-head step: {head_us:.1f} us, {lm_head_step['GBps']:.0f} GB/s, token {head.generated[0]}")
    if args.lm_head_only:
        print(json.dumps({"lm_head_step": lm_head_step, "hbm_stream_read_GBps": stream_gbps}), flush=True)
        return 0
    ctx = model.create_context()

    # ctx 1: 1-token prompt, 256 new tokens (4 launches of 64)
    times, generated = [], None
    for round_ in range(args.warmup + steps):
        ctx.wait(ctx.enqueue_reset())
        ctx.wait(ctx.enqueue_prefill(prompt))
        result = ctx.wait(ctx.enqueue_generate(new_tokens))
        if generated is None:
            generated = result.generated
        elif generated != result.generated:
            raise RuntimeError("benchmark generated different tokens across rounds")
        if round_ >= args.warmup:
            times.append(result.compute_us)
    mean_us = statistics.mean(times)
    ms_per_token = mean_us / new_tokens / 1e3
    positions = range(len(prompt), len(prompt) + new_tokens)
    total_bytes = sum(bytes_per_token(p) for p in positions)
    launches = (new_tokens + 63) // 64
    achieved = total_bytes / (mean_us * 1e-6) / 1e9
    floor_ms = total_bytes / new_tokens / (stream_gbps * 1e9) * 1e3
    log(f"ctx1: {ms_per_token * 1e3:.1f} us/token, floor {floor_ms * 1e3:.1f} us")

    del ctx, model, plan
    gc.collect()
    ctx4096 = None
    if not args.no_ctx4096:
        start = time.time()
        S.llama_package(work / "llama4k", 4096 + 64, "bfloat16", seed=0, chunk_steps=args.chunk_steps, target=target,
                        weights=weights)
        log(f"ctx-4096 package built in {time.time() - start:.1f}s")
        model = R.DecoderModel(R.load_plan(work / "llama4k", verify_weights=False))
        ctx = model.create_context()
        long_prompt = S.prompt(4096, seed=4096)
        start = time.time()
        ctx.wait(ctx.enqueue_prefill(long_prompt))
        prefill_s = time.time() - start
        result = ctx.wait(ctx.enqueue_generate(64))
        long_bytes = sum(bytes_per_token(p) for p in range(4096, 4096 + 64))
        long_ms = result.compute_us / 64 / 1e3
        long_floor = long_bytes / 64 / (stream_gbps * 1e9) * 1e3
        ctx4096 = {"ms_per_token": long_ms, "tokens_per_second": 1e3 / long_ms,
                   "floor_ms_per_token": long_floor, "fraction_of_floor": long_floor / long_ms,
                   "achieved_GBps": long_bytes / (result.compute_us * 1e-6) / 1e9,
                   "prefill_tokens": 4096, "prefill_s": prefill_s, "new_tokens": 64}
        log(f"ctx4096: {long_ms * 1e3:.1f} us/token, floor {long_floor * 1e3:.1f} us")
        # Release device objects while the HIP runtime is alive (profilers finalize at exit).
        del ctx, model
        gc.collect()
    ctx32768 = None
    if not args.no_ctx32768:
        long_context = 32768 + 64
        start = time.time()
        S.llama_package(work / "llama32k", long_context, "bfloat16", seed=0, chunk_steps=1026, target=target,
                        weights=weights)
        log(f"ctx32768 package built in {time.time() - start:.1f}s")
        model = R.DecoderModel(R.load_plan(work / "llama32k", verify_weights=False))
        ctx = model.create_context()
        start = time.time()
        ctx.wait(ctx.enqueue_prefill(S.prompt(32768, seed=32768)))
        prefill_s = time.time() - start
        result = ctx.wait(ctx.enqueue_generate(64))
        long_bytes = sum(bytes_per_token(p) for p in range(32768, 32768 + 64))
        long_ms = result.compute_us / 64 / 1e3
        long_floor = long_bytes / 64 / (stream_gbps * 1e9) * 1e3
        ctx32768 = {"ms_per_token": long_ms, "tokens_per_second": 1e3 / long_ms, "floor_ms_per_token": long_floor,
                    "fraction_of_floor": long_floor / long_ms,
                    "achieved_GBps": long_bytes / (result.compute_us * 1e-6) / 1e9, "prefill_tokens": 32768,
                    "prefill_s": prefill_s, "new_tokens": 64, "attention_chunk_steps": 1026}
        log(f"ctx32768: {long_ms * 1e3:.1f} us/token, floor {long_floor * 1e3:.1f} us")
        del ctx, model
        gc.collect()
    baseline = None
    if args.cpu_tokens > 0:
        baseline = cpu_baseline(weights, args.cpu_tokens)
    from tiles_amd import counters
    traffic = counters.load(TRAFFIC_SUMMARY, "ctx1")
    line = {
        "metric": "ms/token bf16 batch-1 decode at ctx 1 & 4096; % of HBM byte floor",
        "value": ms_per_token,
        "unit": "ms/token",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_token * new_tokens,
        "tokens_per_step": new_tokens,
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init N(0,0.02) weights, norm weights 1.0, seed 0)",
        "config": {"workload": "Llama-3.2-1B bf16 batch-1 greedy decode, ctx 1: 1-token prompt, 256 new tokens, "
                               "64 per persistent launch (one step = one such generation); ctx 4096 and ctx 32768 "
                               "(prompt of that length, 64 new tokens) under ctx4096 / ctx32768",
                   "global_batch": 1, "seq_len": len(prompt) + new_tokens, "parallelism": "none",
                   "packages": {"ctx1": f"max_context {ctx1_context}, planner default attention chunking "
                                        "(one fused chunk)",
                                "ctx4096": f"max_context 4160, attention chunk steps {args.chunk_steps}"},
                   "workers": target["launch"]["worker_count"]},
        "tokens_per_second": 1e3 / ms_per_token,
        "hbm_stream_read_GBps": stream_gbps,
        "floor_ms_per_token": floor_ms,
        "fraction_of_floor": floor_ms / ms_per_token,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBPS,
                     "traffic": traffic["traffic_bytes_per_launch"] if traffic else None,
                     "kernel": "decoder_worker", "launches": launches * steps,
                     "bytes_per_launch": total_bytes / launches, "avg_launch_us": mean_us / launches},
        "ctx4096": ctx4096,
        "ctx32768": ctx32768,
        "lm_head_step": lm_head_step,
        "cpu_baseline": baseline,
        "generated_head": generated[:8],
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
