"""The streaming worker (bf16, hidden size 2048) against the exchange worker on the same packages.

Both workers are built from one kernel source and perform every rounding and every summation
in the same order: the streaming worker only changes where weight rows come from (an LDS ring
filled by streamer waves instead of each task's own loads) and how the compute waves meet.
Their logits, K/V caches and greedy tokens must therefore be bit-identical.  The exchange
worker itself is pinned against the oracle by test_gpu_parity.py.  TILES_AMD_WORKER selects
the worker per launch ("stream" or "exchange").

Cases: fused single-chunk attention, split-context chunks with the merge, generation across
launches (the ring's slot sequence repeats per step), an EOS stop in the middle of a launch
(the streamer waves must leave when the compute waves do), and head_dim 64 and 128.
"""

import os

import numpy as np
import pytest
import torch

from tiles_amd import runtime as R
from tiles_amd import synthetic as S
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def target():
    return probe.probe_library()


@pytest.fixture(scope="module")
def tmp(tmp_path_factory):
    return tmp_path_factory.mktemp("stream")


def stack(head_dim: int, layers: int = 3, vocab: int = 3000, max_context: int = 400) -> P.StackSpec:
    # 4352 = 17 FFN rows per worker: two rows per wave in the gate/up phase with a partial second
    # pair, and a partial batch of down rows.
    heads = 2048 // head_dim
    block = P.BlockSpec(hidden_size=2048, intermediate_size=4352, num_attention_heads=heads,
                        num_key_value_heads=heads // 4, head_dim=head_dim, max_context=max_context)
    return P.StackSpec(block, layers, vocab, True)


def run(path, worker: str, prompt: list[int], new_tokens: int, eos: int | None = None):
    """Decode `prompt` (logits and K/V of the last prompt token), then generate."""
    previous = os.environ.get("TILES_AMD_WORKER")
    os.environ["TILES_AMD_WORKER"] = worker
    try:
        model = R.DecoderModel(R.load_plan(path))
        ctx = model.create_context()
        ctx.wait(ctx.enqueue_prefill(prompt[:-1]))
        snapshot = ctx.collect(ctx.enqueue_decode(prompt[-1], logits=True, kv=True))
        result = ctx.wait(ctx.enqueue_generate(new_tokens, eos_id=eos))
        last = ctx.collect(ctx.enqueue_decode(result.generated[-1] if result.generated else prompt[-1], logits=True))
        return snapshot, result, last
    finally:
        if previous is None:
            os.environ.pop("TILES_AMD_WORKER", None)
        else:
            os.environ["TILES_AMD_WORKER"] = previous


@pytest.mark.parametrize("head_dim,chunk_steps,prompt_length", [
    (64, 128, 60),    # one fused chunk
    (64, 128, 300),   # three split chunks merged by the last one
    (128, 128, 200),  # 128-dim heads, two chunks
])
def test_stream_worker_bit_identical_to_exchange_worker(target, tmp, head_dim, chunk_steps, prompt_length):
    spec = stack(head_dim)
    weights = K.random_weights(spec, seed=head_dim + prompt_length, std=0.05, dtype=torch.float32)
    path = tmp / f"ring_{head_dim}_{prompt_length}"
    K.build_stack_package(spec, weights, target, path, "bfloat16", chunk_steps=chunk_steps, fused_steps=chunk_steps)
    prompt = S.prompt(prompt_length, seed=prompt_length, vocab=spec.vocab_size)
    # 70 new tokens: two launches (64 + 6 steps)
    want_snapshot, want, want_last = run(path, "exchange", prompt, 70)
    got_snapshot, got, got_last = run(path, "stream", prompt, 70)
    np.testing.assert_array_equal(got_snapshot["logits"], want_snapshot["logits"])
    np.testing.assert_array_equal(got_snapshot["kv"], want_snapshot["kv"])
    assert got.generated == want.generated
    assert got.position == want.position and got.stop_reason == want.stop_reason
    np.testing.assert_array_equal(got_last["logits"], want_last["logits"])


def test_stream_worker_eos_stop_mid_launch(target, tmp):
    spec = stack(64, layers=2)
    weights = K.random_weights(spec, seed=3, std=0.05, dtype=torch.float32)
    path = tmp / "ring_eos"
    K.build_stack_package(spec, weights, target, path, "bfloat16", chunk_steps=128, fused_steps=128)
    prompt = S.prompt(20, seed=4, vocab=spec.vocab_size)
    _, free, _ = run(path, "stream", prompt, 12)
    eos = free.generated[5]
    first = free.generated.index(eos)
    _, got, got_last = run(path, "stream", prompt, 12, eos=eos)
    _, want, want_last = run(path, "exchange", prompt, 12, eos=eos)
    assert got.generated == want.generated == free.generated[:first + 1]
    assert got.stop_reason == "eos" and got.position == want.position
    # the context keeps working after the early stop
    np.testing.assert_array_equal(got_last["logits"], want_last["logits"])
