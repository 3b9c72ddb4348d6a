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
