"""Runs one decode workload through the C-ABI library named by TILES_AMD_LIBRARY and saves what it
produced — TEST INFRASTRUCTURE ONLY (tests/test_gpu_delay_injection.py runs it once with the product
library and once with the delay-injection stress build, and compares the files bit for bit).

usage: python tests/delay_runner.py CASE PACKAGE OUT.npz
  m4      the decoder_m4 fixture tokens one decode each (logits per step), then 5 greedy tokens
  split   a 199-token prefill and 60 greedy tokens over 16-step attention chunks (up to 15 per head)
  config3 BASELINE config 3: a 1-token prompt, then 256 greedy tokens in one request (4 launches)
"""

import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parent.parent))

from tiles_amd import runtime as R  # noqa: E402
from tiles_amd import synthetic as S  # noqa: E402

M4_TOKENS = [0, 7, 15, 3, 47]


def main(case: str, package: str, out: str) -> None:
    ctx = R.DecoderModel(R.load_plan(package, verify_weights=False)).create_context()
    saved = {}
    if case == "m4":
        saved["logits"] = np.stack([ctx.collect(ctx.enqueue_decode(t, logits=True))["logits"] for t in M4_TOKENS])
        ctx.wait(ctx.enqueue_reset())
        ctx.wait(ctx.enqueue_prefill([7]))
        ticket = ctx.enqueue_generate(5, kv=True)
    elif case == "split":
        ctx.set_matrix_prefill(False)  # every position through the worker's split attention
        ctx.wait(ctx.enqueue_prefill(S.prompt(199, seed=11, vocab=512)))
        ticket = ctx.enqueue_generate(60, logits=True, kv=True)
    elif case == "config3":
        ctx.wait(ctx.enqueue_prefill([S.BOS]))
        ticket = ctx.enqueue_generate(256, logits=True, kv=True)
    else:
        raise SystemExit(f"unknown case {case}")
    result = ctx.wait(ticket)
    snap = ctx.collect(ticket)
    saved["tokens"] = np.array(result.generated, dtype=np.int64)
    saved["kv"] = snap["kv"]
    if case != "m4":
        saved["last_logits"] = snap["logits"]
    np.savez(out, **saved)
    print(f"{case} via {R.library_path().name}: {len(result.generated)} tokens", flush=True)


if __name__ == "__main__":
    main(*sys.argv[1:4])
