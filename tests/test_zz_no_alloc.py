"""The entry point that allocates nothing (ti_enqueue_worker_static) against ti_enqueue_worker.

Both run the same model with the same caller-owned buffers except the exchange area, which the
static variant takes from the library's device array.  Two calls in a row, the second with a
smaller input (50 prompt tokens, then 10), then a generation that continues from them: logits,
K/V cache and tokens must be bit-identical, and no wait may time out.
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


def test_static_exchange_matches_caller_exchange(tmp_path):
    spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                                   head_dim=64, max_context=160), 2, 512, True)
    weights = K.random_weights(spec, seed=31, std=0.08, dtype=torch.float32)
    K.build_stack_package(spec, weights, probe.probe_library(), tmp_path / "pkg", "bfloat16", chunk_steps=16)
    plan = K.read_plan(tmp_path / "pkg")
    model = R.DecoderModel(R.load_plan(tmp_path / "pkg"))
    assert R.library().ti_static_exchange_words() == 1 << 21
    caller, static = LaunchHost(model, plan), LaunchHost(model, plan, static=True)
    for length, seed in ((50, 1), (10, 2)):
        tokens = S.prompt(length, seed=seed, vocab=512)
        caller.feed(tokens)
        static.feed(tokens)
        np.testing.assert_array_equal(static.logits_values(), caller.logits_values())
        np.testing.assert_array_equal(static.kv_values(), caller.kv_values())
        assert int(static.timeout.item()) == 0
    assert static.generate(30) == caller.generate(30)
    np.testing.assert_array_equal(static.kv_values(), caller.kv_values())
    assert int(static.timeout.item()) == 0


def test_static_exchange_under_graph_capture(tmp_path):
    """ti_enqueue_worker_static captured in a HIP graph: after one eager call (which finds the
    device array's address), a 40-token feed and a 25-token generation are captured on torch's
    capture stream and the graph is replayed three times, with eager work and synchronizations
    between the replays.  Each replay runs the same positions over the same buffers, so each must
    leave logits, K/V cache, tokens and the timeout flag bit-identical to the same calls made
    eagerly (the clear and control-read kernels are captured with the worker; nothing allocates)."""
    spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                                   head_dim=64, max_context=160), 2, 512, True)
    weights = K.random_weights(spec, seed=33, std=0.08, dtype=torch.float32)
    K.build_stack_package(spec, weights, probe.probe_library(), tmp_path / "pkg", "bfloat16", chunk_steps=16)
    plan = K.read_plan(tmp_path / "pkg")
    model = R.DecoderModel(R.load_plan(tmp_path / "pkg"))
    prompt = S.prompt(40, seed=4, vocab=512)
    LaunchHost(model, plan, static=True).feed([3])  # the array's address is found outside the capture

    eager = LaunchHost(model, plan, static=True)
    eager.feed(prompt)
    want_tokens = eager.generate(25)
    want_kv, want_logits = eager.kv_values(), eager.logits_values()
    assert int(eager.timeout.item()) == 0

    host = LaunchHost(model, plan, static=True)
    host.tokens[: len(prompt)] = torch.tensor(prompt, dtype=torch.int32)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        host.stream = torch.cuda.current_stream().cuda_stream
        host._launch(len(prompt), R.TokenInput(-1, host.tokens.data_ptr(), len(prompt)), R.Selection())
        host.status.zero_()
        host.generated.fill_(-1)
        host._launch(25, R.TokenInput(-1, None, 25),
                     R.Selection(host.generated.data_ptr(), host.status.data_ptr(), 0, -1))
    for replay in range(3):
        host.kv.zero_()
        host.logits.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        n = int(host.status[0].item())
        assert host.generated[:n].tolist() == want_tokens, replay
        np.testing.assert_array_equal(host.kv_values(), want_kv, err_msg=f"replay {replay}")
        np.testing.assert_array_equal(host.logits_values(), want_logits, err_msg=f"replay {replay}")
        assert int(host.timeout.item()) == 0
