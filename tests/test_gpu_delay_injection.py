"""The exchange protocol under injected delays (the reference runs its cases under
racecheck/synccheck and requires bit-identical logits with random delays before tasks,
tileinfer/tests/sanitizers.py:170, counter_probe.cu:14-15).

tiles_amd/libtileinfer_amd_delay.so is the library with the worker compiled with
TILES_DELAY_INJECTION: at every task's start and before every exchange publish, K/V cache-row
store and poll, each wave sleeps a pseudo-random 0 to about 2.5 us.  The workloads of the bf16
decoder_m4 bit-exact test, the split-merge test and BASELINE config 3 (tests/delay_runner.py) run
once through each library, each in its own process; tokens, logits and the whole K/V cache must
be bit-identical."""

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from tiles_amd import runtime as R
from tiles_amd import synthetic as S
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu
RUNNER = Path(__file__).with_name("delay_runner.py")
GOLDEN = Path(__file__).parent / "golden"


def package(case: str, root: Path) -> Path:
    target = probe.probe_library()
    path = root / case
    if case == "m4":
        import json
        model = json.loads((GOLDEN / "decoder_m4" / "model.json").read_text())
        block = P.BlockSpec(**{k: model[k] for k in P.BlockSpec.__dataclass_fields__ if k in model})
        spec = P.StackSpec(block, model["layers"], model["vocab_size"], model["tie_word_embeddings"])
        with np.load(GOLDEN / "decoder_m4" / "weights.npz", allow_pickle=False) as data:
            weights = {k: torch.from_numpy(data[k].copy()) for k in data.files}
        K.build_stack_package(spec, weights, target, path, "bfloat16")
    elif case == "split":
        spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4,
                                       num_key_value_heads=1, head_dim=64, max_context=264), 2, 512, True)
        weights = K.random_weights(spec, seed=5, std=0.08, dtype=torch.float32)
        K.build_stack_package(spec, weights, target, path, "bfloat16", chunk_steps=16)
    else:
        S.llama_package(path, 256 + 8, "bfloat16", seed=0, target=target)
    return path


def run(case: str, path: Path, out: Path, library: str) -> dict:
    env = dict(os.environ, TILES_AMD_LIBRARY=library)
    subprocess.run([sys.executable, str(RUNNER), case, str(path), str(out)], env=env, check=True, timeout=600)
    with np.load(out, allow_pickle=False) as data:
        return {k: data[k].copy() for k in data.files}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("case", ["m4", "split", "config3"])
def test_delayed_worker_is_bit_identical(tmp_path, case):
    assert (R.LIBRARY.parent / "libtileinfer_amd_delay.so").exists(), "build the library first (tiles_amd.build)"
    path = package(case, tmp_path)
    plain = run(case, path, tmp_path / "plain.npz", "libtileinfer_amd.so")
    delayed = run(case, path, tmp_path / "delayed.npz", "libtileinfer_amd_delay.so")
    assert plain.keys() == delayed.keys()
    for key in plain:
        np.testing.assert_array_equal(delayed[key].view(np.uint8), plain[key].view(np.uint8), err_msg=key)
