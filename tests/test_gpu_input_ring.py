"""The context's pinned input ring (runtime.cpp, stage_input): host token ids are staged in a ring
of max_context + 64 pinned slots and copied to the device on the context's stream, so that a
request can be enqueued while earlier ones still run.  When a request's tokens do not fit after
the cursor, the ring waits for the stream and starts again from slot 0.  The reference's ring
test (sequence_ring_smoke.cu:76-140) enqueues past the ring's end with requests in flight and
checks that every request still decodes its own tokens; so does this one.
"""

import numpy as np
import pytest
import torch

from tiles_amd import runtime as R
from tiles_amd import synthetic as S
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu


def test_input_ring_wraps_with_requests_in_flight(tmp_path):
    spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                                   head_dim=64, max_context=160), 2, 512, True)
    weights = K.random_weights(spec, seed=41, std=0.08, dtype=torch.float32)
    K.build_stack_package(spec, weights, probe.probe_library(), tmp_path / "pkg", "bfloat16", chunk_steps=16)
    model = R.DecoderModel(R.load_plan(tmp_path / "pkg"))
    # Ring capacity 160 + 64 = 224 token slots: 100 + 90 fit, the third prompt's 120 wrap to slot 0
    # while the first two requests may still be in flight, and the fourth's 50 follow it.
    prompts = [S.prompt(n, seed=seed, vocab=512) for n, seed in ((100, 1), (90, 2), (120, 3), (50, 4))]
    assert sum(len(p) for p in prompts[:3]) > 160 + 64

    want = []
    for prompt in prompts:
        fresh = model.create_context()
        ticket = fresh.enqueue_prefill(prompt, logits=True)
        want.append(fresh.collect(ticket)["logits"])
        fresh.wait(ticket)
        del fresh

    ctx = model.create_context()
    tickets = []
    for prompt in prompts:
        tickets.append(ctx.enqueue_reset())
        tickets.append(ctx.enqueue_prefill(prompt, logits=True))
    got = [ctx.collect(t)["logits"] for t in tickets[1::2]]
    for t in tickets:
        ctx.wait(t)
    for index, (g, w) in enumerate(zip(got, want)):
        np.testing.assert_array_equal(g, w, err_msg=f"prompt {index}")
    # The context continues from the last prompt after the wrap.
    follow = ctx.wait(ctx.enqueue_generate(8)).generated
    fresh = model.create_context()
    fresh.wait(fresh.enqueue_prefill(prompts[-1]))
    assert follow == fresh.wait(fresh.enqueue_generate(8)).generated
