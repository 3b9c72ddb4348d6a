"""The traced timeline of a real launch and its loss budget (the reference's
kernel_regression.py:35-76 check_timeline): every task of the plan recorded once with ordered
stamps, the budget's columns summing to the traced step, and the traced step agreeing with the
launch's own per-token time."""

import json

import pytest

from tiles_amd import runtime as R
from tiles_amd import timeline as T
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("prompt_length", [1, 100])
def test_timeline_budget_sums_to_the_traced_step(tmp_path, prompt_length):
    # Llama-1B widths, 4 layers and a small vocabulary; chunks of 80 positions, so that the
    # traced step of the short prompt runs one fused chunk and the longer one splits over 3.
    block = P.BlockSpec(hidden_size=2048, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
                        head_dim=64, max_context=192)
    spec = P.StackSpec(block, 4, 8192, True)
    K.build_stack_package(spec, K.random_weights(spec, seed=3), probe.probe_library(), tmp_path / "p", "bfloat16",
                          chunk_steps=80, fused_steps=80)
    plan = json.loads((tmp_path / "p" / "plan.json").read_text())
    ctx = R.DecoderModel(R.load_plan(tmp_path / "p")).create_context()
    prompt = list(range(1, prompt_length + 1))
    ctx.set_timeline(True)
    ctx.wait(ctx.enqueue_prefill(prompt))
    done = ctx.wait(ctx.enqueue_generate(64))
    stamps = ctx.timeline().reshape(-1, 4)
    imap = T.instruction_map(plan)
    assert len(stamps) == len(imap)
    tasks = [i for i, (_, _, t) in enumerate(imap) if t >= 0]
    assert sorted(imap[i][2] for i in tasks) == list(range(len(plan["tasks"])))
    assert all(stamps[i, 0] != 0 for i in tasks), "every task of the traced step records its start"
    for i in tasks:
        start, read, ready, end = (int(v) for v in stamps[i])
        assert start <= end
        if ready:
            assert start <= ready <= end and (not read or read <= ready)

    position = prompt_length + 63
    report = T.budget(plan, stamps, position, 5000.0)
    parts = report["ideal_stream_us"] + sum(report["components_us"].values())
    assert abs(parts - report["traced_kernel_us"]) < 1e-6
    assert set(report["phases"]) == set(T.PHASES)
    assert sum(p["waves"] for p in report["phases"].values()) == len(plan["waves"])
    per_token = done.compute_us / 64
    print(f"prompt {prompt_length}: traced {report['traced_kernel_us']:.1f} us, launch {per_token:.1f} us/token, "
          f"components {({k: round(v, 1) for k, v in report['components_us'].items()})}", flush=True)
    # The last step alone against the launch's average step (which also carries the launch and
    # the first step's instruction-stream copy): within 25%.
    assert 0.75 * per_token < report["traced_kernel_us"] < 1.25 * per_token
    assert T.active_chunks(plan["model"], position) == {1: 1, 100: 3}[prompt_length]
