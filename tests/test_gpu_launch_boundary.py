"""The launch boundary driven by a host of its own, and one model shared by two contexts.

* ``ti_enqueue_worker`` with caller-owned buffers (tests/launch_boundary.py): the model's program
  view, PyTorch device tensors for every worker buffer, the exchange area zeroed once and the
  epoch advanced by exactly ``ti_epochs_per_launch`` per launch, as INTEGRATION.md prescribes.
  Its prefill and multi-launch greedy generation must give the runtime's own tokens and K/V
  cache bit for bit (the reference's launcher contract, detail/launch.cuh:87-88).
* two sequence contexts of one uploaded model, interleaved, each bit-identical to a context
  that ran alone (tileinfer/tests/sequence_context_smoke.cpp:60-166).
"""

import numpy as np
import pytest
import torch

from tests.launch_boundary import LaunchHost
from tiles_amd import runtime as R
from tiles_amd import synthetic as S
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def package(tmp_path_factory):
    """Two layers, 16-step attention chunks (the split path from 17 positions on), bf16."""
    spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                                   head_dim=64, max_context=240), 2, 512, True)
    weights = K.random_weights(spec, seed=21, std=0.08, dtype=torch.float32)
    path = tmp_path_factory.mktemp("boundary") / "pkg"
    K.build_stack_package(spec, weights, probe.probe_library(), path, "bfloat16", chunk_steps=16)
    return path


def test_enqueue_worker_with_caller_owned_buffers(package):
    plan = K.read_plan(package)
    model = R.DecoderModel(R.load_plan(package))
    prompt = S.prompt(70, seed=3, vocab=512)
    ctx = model.create_context()
    # The host feeds the prompt through the worker, 64 positions per launch; the context's bf16
    # matrix prefill sums its dot products in another order, so the context is kept on the worker.
    ctx.set_matrix_prefill(False)
    ctx.wait(ctx.enqueue_prefill(prompt))
    ticket = ctx.enqueue_generate(150, kv=True)
    want = ctx.wait(ticket).generated
    kv_want = ctx.collect(ticket)["kv"]

    host = LaunchHost(model, plan)
    host.feed(prompt)
    got = host.generate(150)
    assert got == want and len(got) == 150
    np.testing.assert_array_equal(host.kv_values(), kv_want)
    launches = 2 + 3  # 70 prompt steps, then 150 generated
    assert host.epoch == 1 + launches * R.library().ti_epochs_per_launch(2)
    # a stop mid-launch: the epoch goes back to follow the launch that ran
    eos = got[5]
    host2 = LaunchHost(model, plan)
    host2.feed(prompt)
    stopped = host2.generate(150, eos=eos)
    assert stopped == got[: got.index(eos) + 1]
    assert host2.epoch == 1 + 3 * R.library().ti_epochs_per_launch(2)
    more = host2.generate(3)  # continues from the stop as the runtime does
    ctx.wait(ctx.enqueue_reset())
    ctx.wait(ctx.enqueue_prefill(prompt))
    ctx.wait(ctx.enqueue_generate(150, eos_id=eos))
    assert more == ctx.wait(ctx.enqueue_generate(3)).generated


def test_two_contexts_share_one_model(package):
    model = R.DecoderModel(R.load_plan(package))
    a_prompt, b_prompt = S.prompt(40, seed=5, vocab=512), S.prompt(90, seed=6, vocab=512)

    def alone(prompt, count):
        ctx = model.create_context()
        ctx.wait(ctx.enqueue_prefill(prompt))
        t = ctx.enqueue_generate(count, kv=True)
        return ctx.wait(t).generated, ctx.collect(t)["kv"]

    want_a, want_b = alone(a_prompt, 70), alone(b_prompt, 100)
    a, b = model.create_context(), model.create_context()
    a.enqueue_prefill(a_prompt)
    b.enqueue_prefill(b_prompt)
    ta = a.enqueue_generate(70, kv=True)
    tb = b.enqueue_generate(100, kv=True)
    assert b.wait(tb).generated == want_b[0]
    assert a.wait(ta).generated == want_a[0]
    np.testing.assert_array_equal(a.collect(ta)["kv"], want_a[1])
    np.testing.assert_array_equal(b.collect(tb)["kv"], want_b[1])


@pytest.mark.parametrize("fields", [0, R.TIMELINE_REFERENCE_FIELDS, R.TIMELINE_FIELDS])
def test_timeline_records_stay_inside_a_buffer_of_their_size(package, fields):
    """A host that allocates the reference's kTimelineFields (3) words per instruction
    (diagnostic_context.cu:264) and leaves timeline_fields zero, or asks for 3 or for this build's
    4, gets every task's record inside that buffer: guard words past its end are intact, barrier
    records untouched, and each task record ordered in time (reference record: end cycle after
    the start cycle, a start time in ns; this build's: start <= inputs complete <= end)."""
    plan = K.read_plan(package)
    info = R.load_plan(package).inspect()
    count, tasks = info["instruction_count"], info["task_count"]
    width = fields or R.TIMELINE_REFERENCE_FIELDS
    guard_words, guard = 256, 0x5A5A5A5A5A5A5A5A
    host = LaunchHost(R.DecoderModel(R.load_plan(package)), plan)
    host.timeline = torch.full((width * count + guard_words,), guard, dtype=torch.int64, device="cuda")
    host.timeline_fields = fields
    host.feed(S.prompt(40, seed=9, vocab=512))
    torch.cuda.synchronize()
    words = host.timeline.cpu().numpy().view(np.uint64)
    assert (words[width * count:] == guard).all()
    records = words[: width * count].reshape(count, width)
    written = ~(records == guard).all(axis=1)
    assert int(written.sum()) == tasks
    r = records[written].astype(np.int64)
    if width == R.TIMELINE_REFERENCE_FIELDS:
        assert (r[:, 1] > r[:, 0]).all() and (r[:, 2] > 0).all()
        # all workers share the ns clock: the step's records span well under a second
        assert r[:, 2].max() - r[:, 2].min() < 1_000_000_000
    else:
        ready = r[:, 2] > 0
        assert (r[:, 3] >= r[:, 0]).all() and (r[ready, 2] >= r[ready, 0]).all() and (r[ready, 3] >= r[ready, 2]).all()


def test_stuck_waits_end_the_launch_and_reset_recovers(package):
    """The timeout path that replaces the reference's grid barrier (worker_kernel.cu:107,192, which
    has none): with the spin limit at 0 (ti_set_worker_spin_limit), the first wait of a launch
    that has to poll again declares the exchange stuck, every wait of every worker then gives up
    and every block returns (the call ends), a generating launch stores TI_DEVICE_SYNC_TIMEOUT in
    its status, and the runtime fails the request with "worker synchronization timed out", then
    requires a reset; after the reset the context decodes exactly as a fresh one."""
    plan = K.read_plan(package)
    model = R.DecoderModel(R.load_plan(package))
    lib = R.library()
    prompt = S.prompt(30, seed=12, vocab=512)
    fresh = model.create_context()
    fresh.wait(fresh.enqueue_prefill(prompt))
    want = fresh.wait(fresh.enqueue_generate(70)).generated

    host = LaunchHost(model, plan)
    host.feed(prompt)
    ctx = model.create_context()
    ctx.wait(ctx.enqueue_prefill(prompt))
    lib.ti_set_worker_spin_limit(0)
    try:
        host.generate(70)
        assert int(host.status[2].item()) == 3  # TI_DEVICE_SYNC_TIMEOUT
        assert int(host.exchange[0].item()) != 0  # the control word a stuck wait sets
        with pytest.raises(RuntimeError, match="worker synchronization timed out"):
            ctx.wait(ctx.enqueue_generate(70))
    finally:
        lib.ti_set_worker_spin_limit(R.DEFAULT_SPIN_LIMIT)
    with pytest.raises(RuntimeError, match="reset required"):
        ctx.wait(ctx.enqueue_decode(5))
    ctx.wait(ctx.enqueue_reset())
    ctx.wait(ctx.enqueue_prefill(prompt))
    assert ctx.wait(ctx.enqueue_generate(70)).generated == want
