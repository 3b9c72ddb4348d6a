"""The loss budget on a synthetic, known trace (the reference's tileplan/tests/test_timeline.py
checks its budget the same way): a tiny stack plan, every task's four device-clock stamps set
by a schedule whose exchange latency, task times and byte count are known, and the budget's
columns checked against them."""

from xml.etree import ElementTree

import numpy as np
import pytest

from tiles_amd import timeline as T
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

LATENCY = 30      # ticks from the last producer's end to the consumers' inputs ready
EARLY = 5         # ticks a task starts (and issues its loads) before the previous wave ends
WORK = 200        # ticks of a task after its inputs are ready, plus its worker index
BASE = 10_000


def tiny_plan(tmp_path, max_context=32, chunk_steps=None, fused_steps=None):
    block = P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                        head_dim=64, max_context=max_context)
    spec = P.StackSpec(block, 2, 512, True)
    kwargs = {"chunk_steps": chunk_steps, "fused_steps": fused_steps}
    K.build_stack_package(spec, K.random_weights(spec, seed=1), probe.mi355x_target(8), tmp_path / "p", "bfloat16",
                          **kwargs)
    return spec, K.read_plan(tmp_path / "p")


def synthetic_stamps(plan):
    """Wave 0 (the embedding) starts at BASE and waits for nothing.  Every later task starts
    EARLY ticks before the previous wave's last end E, reads at E + 1, is ready at E + LATENCY
    and ends WORK + worker ticks after that."""
    imap = T.instruction_map(plan)
    stamps = np.zeros((len(imap), 4), dtype=np.uint64)
    previous_end = None
    for wave in range(len(plan["waves"])):
        last = 0
        for index, (worker, w, task) in enumerate(imap):
            if w != wave or task < 0:
                continue
            if previous_end is None:
                start, read, ready = BASE, 0, 0
                end = BASE + WORK + worker
            else:
                start, read, ready = previous_end - EARLY, previous_end + 1, previous_end + LATENCY
                end = ready + WORK + worker
            stamps[index] = (start, read, ready, end)
            last = max(last, end)
        previous_end = last
    return stamps, (previous_end - BASE) * T.TICK_NS / 1e3


def algorithmic_bytes(spec, position):
    """Every weight once (tied LM head read as the embedding, plus one embedding row) and the
    K and V rows of positions 0..position, from the model's shape alone."""
    b = spec.block
    d, f, kvw = b.hidden_size, b.intermediate_size, b.num_key_value_heads * b.head_dim
    per_layer = d * (d + 2 * kvw) + d * d + 3 * d * f
    return 2 * (spec.layers * per_layer + d + spec.vocab_size * d + spec.layers * 2 * (position + 1) * kvw)


@pytest.mark.parametrize("position", [0, 9, 31])
def test_budget_recovers_the_synthetic_schedule(tmp_path, position):
    # Chunks of 8 positions, prefixes of up to 4 fused: 1, 2 and 4 active chunks.
    spec, plan = tiny_plan(tmp_path, chunk_steps=8, fused_steps=4)
    assert T.active_chunks(plan["model"], position) == {0: 1, 9: 2, 31: 4}[position]
    stamps, traced = synthetic_stamps(plan)
    report = T.budget(plan, stamps, position, 200.0)
    assert report["traced_kernel_us"] == pytest.approx(traced, abs=1e-9)
    parts = report["ideal_stream_us"] + sum(report["components_us"].values())
    assert parts == pytest.approx(report["traced_kernel_us"], abs=1e-9)
    waves = len(plan["waves"])
    # Exchange latency: LATENCY ticks before every wave except the first.
    assert report["components_us"]["barrier_sync"] == pytest.approx((waves - 1) * LATENCY * T.TICK_NS / 1e3)
    # Ideal streaming: the closed-form bytes at 200 GB/s.
    assert report["ideal_stream_us"] == pytest.approx(algorithmic_bytes(spec, position) / 200.0 / 1e3)
    assert sum(p["waves"] for p in report["phases"].values()) == waves
    assert sum(p["duration_us"] for p in report["phases"].values()) == pytest.approx(traced)
    for w in report["waves"]:
        assert w["duration_ns"] == pytest.approx(w["sync_ns"] + w["ideal_ns"] + w["work_ns"] + w["tail_ns"])
        # the slowest busy worker sets the wave's end: its worker index is the largest
        assert w["tail_ns"] >= 0
    # A task waits from its start to ready: EARLY + LATENCY ticks, for every task after wave 0.
    waited = sum(len(lane) for wave in plan["waves"][1:] for lane in wave["workers"])
    assert report["mean_barrier_wait_us"] == pytest.approx(
        waited * (EARLY + LATENCY) * T.TICK_NS / plan["target"]["worker_count"] / 1e3)
    svg = T.render_timeline_svg(plan, T.events(plan, stamps), title="synthetic",
                                window=T.layer_window(plan, T.events(plan, stamps), 1))
    assert ElementTree.fromstring(svg).tag == "{http://www.w3.org/2000/svg}svg"


def test_budget_rejects_a_timeline_of_another_plan(tmp_path):
    _, plan = tiny_plan(tmp_path)
    stamps, _ = synthetic_stamps(plan)
    with pytest.raises(ValueError, match="instruction count"):
        T.budget(plan, stamps[:-1], 0, 200.0)
    stamps[np.nonzero(stamps[:, 0])[0][3], 3] = 1  # an end before its start
    with pytest.raises(ValueError, match="ends before it starts"):
        T.budget(plan, stamps, 0, 200.0)
